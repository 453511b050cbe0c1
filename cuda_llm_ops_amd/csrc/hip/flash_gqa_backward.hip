// GQA prefill backward (dQ, dK, dV) for gfx950.
//
// Stands in for the reference's Triton-only flash_gqa_backward_bf16_kernel
// (src/python/Triton/flash_gqa_backward_kernel.py:159-310, launcher :312-478).
// Same maths, per query row i of head h and key j of its KV head:
//   delta_i = sum_x O_i[x] dO_i[x]                            (:16-50)
//   P_ij    = exp(q_i.k_j * scale - lse_i); 0 where j > i (causal, top-left)
//             or j >= Skv                                       (:253-262)
//   dV_j   += bf16(P_ij) dO_i                                   (:263, :271-272)
//   dP_ij   = dO_i . v_j                                        (:274-275)
//   dS_ij   = bf16(P_ij (dP_ij - delta_i) scale)                (:283-285)
//   dK_j   += dS_ij q_i          dQ_i += dS_ij k_j               (:287-293)
// fp32 accumulation, bf16 results (:470-472).
//
// Three launches on the caller's stream:
//   bwd_prep_kernel     per query row: -lse*log2(e) and -delta*scale into the
//                       workspace; zeroes the row's fp32 dQ accumulator (and,
//                       when heads are split over workgroups, the fp32 dK/dV
//                       accumulators).
//   bwd_kv_kernel       one workgroup = one 128-key block of one KV head and a
//                       subset of its query heads.  Wave w owns keys 32w..32w+31
//                       of the block: their K and V rows stay in registers as
//                       MFMA operands and their dK, dV (fp32, 32 x 128 each) are
//                       accumulated in registers over the whole loop over
//                       (head, 32-row query block).  Per query block:
//                         S  = Q K^T,  dP = dO V^T     (C[q][key], Q/dO rows from LDS)
//                         P, dS on the VALU            (P -> bf16 in place as the
//                                                       A operand of the next two)
//                         dV += P^T dO, dK += dS^T Q   (dO/Q read transposed, ds_read_b64_tr_b16)
//                         dS^T -> LDS
//                       and one step later, once every wave's dS^T is in LDS,
//                         dQ = dS K over the 128 keys (each wave 32 of the 128
//                         columns of D), added to the fp32 dQ accumulator with
//                         global float atomics.
//                       Q, dO, -lse*log2e and -delta*scale of the next block
//                       stream into LDS (buffer_load ... lds) during the current one.
//   bwd_convert_kernel  fp32 accumulators -> bf16 outputs (any strides).
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

#include "fgqa_device.h"
#include "fgqa_internal.h"

namespace fgqa {

struct BwdParams {
    const __bf16* q;
    const __bf16* k;
    const __bf16* v;
    const __bf16* o;
    const __bf16* dout;
    const float* lse;
    __bf16* dq;
    __bf16* dk;
    __bf16* dv;
    int64_t q_sb, q_ss, q_sh;
    int64_t k_sb, k_ss, k_sh;
    int64_t v_sb, v_ss, v_sh;
    int64_t o_sb, o_ss, o_sh;
    int64_t do_sb, do_ss, do_sh;
    int64_t dq_sb, dq_ss, dq_sh;
    int64_t dk_sb, dk_ss, dk_sh;
    int64_t dv_sb, dv_ss, dv_sh;
    // workspace
    float* rowstat;   // [2][B*Hq*Sq]: -lse*log2(e), then -delta*scale
    float* dq_acc;    // [B, Hq, Sq, D] fp32
    float* dk_acc;    // [B, Hkv, Skv, D] fp32 (heads split), else null
    float* dv_acc;
    int batch, sq, skv, hq, hkv, group, causal;
    int hs;           // query heads per workgroup
    int n_hsplit;     // group / hs
    int n_kvblocks;   // ceil(skv / 128)
    int n_streams;    // n_hsplit * hkv * batch
    int n_qblocks;    // ceil(sq / 32)
    float scale;
    float scale_log2;   // scale * log2(e)
};

constexpr int kBwWaves = 4;
constexpr int kBwThreads = kBwWaves * kWave;
constexpr int kBwKeys = 128;                          // keys per workgroup
constexpr int kBwRows = 32;                           // query rows per step
constexpr int kBwRowBytes = kHeadDim * 2;             // one Q / dO / K row
constexpr int kBwTileBytes = kBwRows * kBwRowBytes;   // 8 KB: Q or dO of one step
constexpr int kBwDsRowBytes = kBwRows * 2;            // one dS^T row (a key, 32 query rows)
constexpr int kBwDsBytes = kBwKeys * kBwDsRowBytes;   // 8 KB
constexpr int kBwStatBytes = 2 * kBwRows * 4;         // -lse*log2e and -delta*scale of 32 rows
// LDS map (bytes): Q[2] | dO[2] | dS^T[2] | stats[2].  The prologue stages
// the workgroup's K block (128 rows, 32 KB) over Q[2] and dO[2].
constexpr int kBwQOff = 0;
constexpr int kBwDoOff = 2 * kBwTileBytes;
constexpr int kBwDsOff = 4 * kBwTileBytes;
constexpr int kBwStatOff = kBwDsOff + 2 * kBwDsBytes;
constexpr int kBwSmemBytes = kBwStatOff + 2 * kBwStatBytes;
static_assert(kBwKeys * kBwRowBytes <= kBwDsOff, "K staging must fit below the dS buffers");

// Q, dO and K rows (256 B) sit in LDS with their 16-byte chunks permuted:
// chunk c of row r goes to slot c ^ bw_swz(r).  bw_swz is a bijection on
// r % 16 (16 consecutive rows read at the same chunk hit 16 different slots:
// conflict-free b128 row reads) whose top two bits are r % 4 (4 consecutive
// rows read over 4 consecutive chunks hit 4 disjoint slot groups:
// conflict-free transposed reads).
__device__ __forceinline__ int bw_swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

// dS^T rows are 64 bytes (32 query rows); chunk c (16 B) of key row r goes to
// slot c ^ ((r >> 2) & 3) and its 8-byte halves are exchanged when r & 16,
// which keeps both the b64 writes and the transposed reads conflict-free.
__device__ __forceinline__ int bw_ds_addr(int r, int chunk, int half) {
    return r * kBwDsRowBytes + ((chunk ^ ((r >> 2) & 3)) << 4) + 8 * (half ^ ((r >> 4) & 1));
}

__device__ __forceinline__ void bw_dma16(uint32_t lds_addr, uint32_t voffset, __amdgpu_buffer_rsrc_t rsrc) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :: "s"(lds_addr), "v"(voffset), "s"(rsrc) : "memory");
}
__device__ __forceinline__ void bw_dma4(uint32_t lds_addr, uint32_t voffset, __amdgpu_buffer_rsrc_t rsrc) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds"
                 :: "s"(lds_addr), "v"(voffset), "s"(rsrc) : "memory");
}
__device__ __forceinline__ void bw_wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__device__ __forceinline__ void atomic_add_f32(float* p, float v) {
    __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------- prep
// 16 lanes per query row (8 elements each).  Rows are numbered (b, h, i) in
// the LSE layout [B, Hq, Sq].
__global__ __launch_bounds__(256) void bwd_prep_kernel(BwdParams p) {
    const int64_t rows_q = (int64_t)p.batch * p.hq * p.sq;
    const int64_t rows_kv = (int64_t)p.batch * p.hkv * p.skv;
    const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    const int part = threadIdx.x & 15;
    if (row < rows_q) {
        const int i = (int)(row % p.sq);
        const int64_t bh = row / p.sq;
        const int h = (int)(bh % p.hq);
        const int b = (int)(bh / p.hq);
        const u32x4_t ov = *reinterpret_cast<const u32x4_t*>(p.o + b * p.o_sb + i * p.o_ss + h * p.o_sh + part * 8);
        const u32x4_t dv = *reinterpret_cast<const u32x4_t*>(p.dout + b * p.do_sb + i * p.do_ss + h * p.do_sh + part * 8);
        const bf16x8_t o8 = as_bf16x8(ov), d8 = as_bf16x8(dv);
        float acc = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc += (float)o8[e] * (float)d8[e];
        acc = xor_sum(acc, 1);
        acc = xor_sum(acc, 2);
        acc = xor_sum(acc, 4);
        acc = xor_sum(acc, 8);
        if (part == 0) {
            p.rowstat[row] = -p.lse[row] * kLog2e;
            p.rowstat[rows_q + row] = -acc * p.scale;
        }
        f32x4_t* z = reinterpret_cast<f32x4_t*>(p.dq_acc + row * kHeadDim + part * 8);
        z[0] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        z[1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    if (p.dk_acc != nullptr && row < rows_kv) {
        f32x4_t* zk = reinterpret_cast<f32x4_t*>(p.dk_acc + row * kHeadDim + part * 8);
        f32x4_t* zv = reinterpret_cast<f32x4_t*>(p.dv_acc + row * kHeadDim + part * 8);
        zk[0] = zk[1] = zv[0] = zv[1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
}

// ---------------------------------------------------------------- convert
__device__ __forceinline__ void bw_store_row(__bf16* dst, const float* src) {
    const f32x4_t a = *reinterpret_cast<const f32x4_t*>(src);
    const f32x4_t c = *reinterpret_cast<const f32x4_t*>(src + 4);
    bf16x8_t w;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        w[e] = (__bf16)a[e];
        w[4 + e] = (__bf16)c[e];
    }
    *reinterpret_cast<bf16x8_t*>(dst) = w;
}

__global__ __launch_bounds__(256) void bwd_convert_kernel(BwdParams p) {
    const int64_t rows_q = (int64_t)p.batch * p.hq * p.sq;
    const int64_t rows_kv = (int64_t)p.batch * p.hkv * p.skv;
    const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    const int part = threadIdx.x & 15;
    if (row < rows_q) {
        const int i = (int)(row % p.sq);
        const int64_t bh = row / p.sq;
        const int h = (int)(bh % p.hq);
        const int b = (int)(bh / p.hq);
        bw_store_row(p.dq + b * p.dq_sb + i * p.dq_ss + h * p.dq_sh + part * 8, p.dq_acc + row * kHeadDim + part * 8);
    }
    if (p.dk_acc != nullptr && row < rows_kv) {
        const int j = (int)(row % p.skv);
        const int64_t bh = row / p.skv;
        const int kvh = (int)(bh % p.hkv);
        const int b = (int)(bh / p.hkv);
        bw_store_row(p.dk + b * p.dk_sb + j * p.dk_ss + kvh * p.dk_sh + part * 8, p.dk_acc + row * kHeadDim + part * 8);
        bw_store_row(p.dv + b * p.dv_sb + j * p.dv_ss + kvh * p.dv_sh + part * 8, p.dv_acc + row * kHeadDim + part * 8);
    }
}

// ---------------------------------------------------------------- main
__global__ __launch_bounds__(kBwThreads, 1) void bwd_kv_kernel(BwdParams p) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int l32 = lane & 31;
    const int l16 = lane & 15;
    const int g2 = lane >> 5;          // half of the wave
    const int gq = (lane >> 4) & 1;    // 16-lane group within the half
    const int s4 = l16 >> 2;           // source row (within 4) of a transposed read
    const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)smem;

    // Block -> (key block, head subset, kv head, batch).  Key blocks in
    // ascending order: under the causal mask block 0 sees every query block,
    // so the heaviest workgroups are dispatched first.
    const int stream = blockIdx.x % p.n_streams;
    const int kb = blockIdx.x / p.n_streams;
    const int hsp = stream % p.n_hsplit;
    const int kvh = (stream / p.n_hsplit) % p.hkv;
    const int b = stream / (p.n_hsplit * p.hkv);
    const int kv0 = kb * kBwKeys;
    const int h0 = kvh * p.group + hsp * p.hs;

    // ---- K, V rows of this wave's keys as B operands of S = Q K^T, dP = dO V^T:
    // lane (key l32, half g2), k-step ks holds elements 16ks + 8g2 .. +7.
    // Keys >= skv read as zero.
    const uint32_t kss = (uint32_t)(p.k_ss * 2);
    const uint32_t vss = (uint32_t)(p.v_ss * 2);
    const __amdgpu_buffer_rsrc_t krs =
        make_rsrc(p.k + b * p.k_sb + kvh * p.k_sh, (uint32_t)(p.skv - 1) * kss + kBwRowBytes);
    const __amdgpu_buffer_rsrc_t vrs =
        make_rsrc(p.v + b * p.v_sb + kvh * p.v_sh, (uint32_t)(p.skv - 1) * vss + kBwRowBytes);
    const int key_l = 32 * wave + l32;   // this lane's key within the block
    const int key = kv0 + key_l;
    bf16x8_t kop[8], vop[8];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
        kop[ks] = as_bf16x8(buf_load16(krs, (uint32_t)key * kss + (16 * ks + 8 * g2) * 2));
        vop[ks] = as_bf16x8(buf_load16(vrs, (uint32_t)key * vss + (16 * ks + 8 * g2) * 2));
    }

    // ---- K block staged in LDS (rows swizzled), then read transposed as the B
    // operand of dQ = dS K: lane (column 32*wave + l32 of D, half g2), k-step ks
    // holds keys 16ks + 4g2 + 0..3 and 16ks + 8 + 4g2 + 0..3 (the same key order
    // as the dS operand below).
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int r0 = 4 * (wave + 4 * i);
        const int r = r0 + (lane >> 4);
        bw_dma16(lds_base + r0 * kBwRowBytes, (uint32_t)(kv0 + r) * kss + ((l16 ^ bw_swz(r)) << 4), krs);
    }
    bw_wait_vmem();
    __syncthreads();
    // transposed-read offsets for 256-byte swizzled rows: source lane supplies
    // row 4g2 + s4 (+8), chunk 4*cb + 2gq + (l16>>1 & 1), half l16 & 1
    auto tr_off = [&](int cb, int h8) {
        const int r = 4 * g2 + s4 + 8 * h8;
        const int c = 4 * cb + 2 * gq + ((l16 >> 1) & 1);
        return r * kBwRowBytes + ((c ^ bw_swz(r)) << 4) + 8 * (l16 & 1);
    };
    bf16x8_t ktr[8];
    {
        const int o0 = tr_off(wave, 0), o1 = tr_off(wave, 1);
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            const unsigned char* base = smem + ks * 16 * kBwRowBytes;
            const bf16x4_t lo = lds_read_tr16(reinterpret_cast<const __bf16*>(base + o0));
            const bf16x4_t hi = lds_read_tr16(reinterpret_cast<const __bf16*>(base + o1));
            ktr[ks] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        }
    }
    __syncthreads();   // K staging area is reused for Q / dO below

    // ---- iteration space: head hh = h0 + t / per_head, query block qb0 + t % per_head
    const int qb0 = p.causal ? min(kv0 / kBwRows, p.n_qblocks) : 0;
    const int per_head = p.n_qblocks - qb0;
    const int n_iter = (p.skv > 0) ? p.hs * per_head : 0;

    const uint32_t qss = (uint32_t)(p.q_ss * 2);
    const uint32_t dss = (uint32_t)(p.do_ss * 2);
    const int64_t rows_q = (int64_t)p.batch * p.hq * p.sq;
    const __amdgpu_buffer_rsrc_t srs = make_rsrc(p.rowstat, (uint32_t)(2 * rows_q * 4));
    // Q, dO rows of step t (32 rows, wave w fetches rows 8w..8w+7 of each)
    // and their statistics (wave 0) into buffer bi.
    auto issue = [&](int t, int bi) {
        const int hh = h0 + t / per_head;
        const int q0 = (qb0 + t % per_head) * kBwRows;
        const __amdgpu_buffer_rsrc_t qrs =
            make_rsrc(p.q + b * p.q_sb + hh * p.q_sh, (uint32_t)(p.sq - 1) * qss + kBwRowBytes);
        const __amdgpu_buffer_rsrc_t drs =
            make_rsrc(p.dout + b * p.do_sb + hh * p.do_sh, (uint32_t)(p.sq - 1) * dss + kBwRowBytes);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int r0 = 8 * wave + 4 * j;
            const int r = r0 + (lane >> 4);
            const int slot = (l16 ^ bw_swz(r)) << 4;
            bw_dma16(lds_base + kBwQOff + bi * kBwTileBytes + r0 * kBwRowBytes, (uint32_t)(q0 + r) * qss + slot, qrs);
            bw_dma16(lds_base + kBwDoOff + bi * kBwTileBytes + r0 * kBwRowBytes, (uint32_t)(q0 + r) * dss + slot, drs);
        }
        if (wave == 0) {
            const int r = q0 + l32;
            const int64_t idx = ((int64_t)b * p.hq + hh) * p.sq + r + (g2 ? rows_q : 0);
            const uint32_t off = (r < p.sq) ? (uint32_t)(idx * 4) : 0xFFFFFFF0u;   // out of range -> 0
            bw_dma4(lds_base + kBwStatOff + bi * kBwStatBytes, off, srs);
        }
    };

    f32x16_t dk_acc[4], dv_acc[4];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) dk_acc[db][i] = dv_acc[db][i] = 0.f;

    // transposed-read offsets into the Q / dO tiles (same row pattern as ktr)
    int trq[4][2];
#pragma unroll
    for (int db = 0; db < 4; ++db) {
        trq[db][0] = tr_off(db, 0);
        trq[db][1] = tr_off(db, 1);
    }
    // dS^T transposed reads for dQ: rows 4g2 + s4 (+8) of each 16-key step,
    // query chunk 2gq + (l16>>1 & 1), half l16 & 1 (the half swap of bw_ds_addr
    // depends on bit 4 of the key, i.e. on the parity of the step)
    int trs[2][2];
#pragma unroll
    for (int par = 0; par < 2; ++par)
#pragma unroll
        for (int h8 = 0; h8 < 2; ++h8)
            trs[par][h8] = bw_ds_addr(16 * par + 4 * g2 + s4 + 8 * h8, 2 * gq + ((l16 >> 1) & 1), l16 & 1) -
                           16 * par * kBwDsRowBytes;
    const int fl = bw_swz(l32);

    // dQ of the step held in dS^T buffer bi, for rows q0.. of head hh: wave w
    // computes columns 32w..32w+31 of D over all 128 keys and adds them to the
    // fp32 accumulator.
    auto dq_step = [&](int bi, int hh, int q0) {
        const unsigned char* dsl = smem + kBwDsOff + bi * kBwDsBytes;
        f32x16_t acc;
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[i] = 0.f;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            const unsigned char* base = dsl + ks * 16 * kBwDsRowBytes;
            const bf16x4_t lo = lds_read_tr16(reinterpret_cast<const __bf16*>(base + trs[ks & 1][0]));
            const bf16x4_t hi = lds_read_tr16(reinterpret_cast<const __bf16*>(base + trs[ks & 1][1]));
            acc = mfma32(__builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7), ktr[ks], acc);
        }
        // C[q][d]: lane (d = 32w + l32, half g2), register 4i + r -> row 8i + 4g2 + r
        float* dst = p.dq_acc + (((int64_t)b * p.hq + hh) * p.sq + q0) * kHeadDim + 32 * wave + l32;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int q = 8 * i + 4 * g2 + r;
                if (q0 + q < p.sq) atomic_add_f32(dst + q * kHeadDim, acc[4 * i + r]);
            }
    };

    const float c2 = p.scale_log2;
    const float scale = p.scale;
    // this lane's key is seen by query rows [lo_row, sq)
    const int lo_row = (key >= p.skv) ? 0x7fffffff : (p.causal ? key : 0);

    if (n_iter > 0) issue(0, 0);
    bw_wait_vmem();
    __syncthreads();

    int prev_h = 0, prev_q0 = 0;
    for (int t = 0; t < n_iter; ++t) {
        const int bi = t & 1;
        const int hh = h0 + t / per_head;
        const int q0 = (qb0 + t % per_head) * kBwRows;
        if (t + 1 < n_iter) issue(t + 1, bi ^ 1);
        if (t > 0) dq_step(bi ^ 1, prev_h, prev_q0);

        // S = Q K^T and dP = dO V^T: C[q][key], lane (key l32, half g2),
        // register 4i + r <-> query row 8i + 4g2 + r
        const unsigned char* ql = smem + kBwQOff + bi * kBwTileBytes;
        const unsigned char* dl = smem + kBwDoOff + bi * kBwTileBytes;
        f32x16_t s, dp;
#pragma unroll
        for (int i = 0; i < 16; ++i) s[i] = dp[i] = 0.f;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            const int off = l32 * kBwRowBytes + (((2 * ks + g2) ^ fl) << 4);
            s = mfma32(*reinterpret_cast<const bf16x8_t*>(ql + off), kop[ks], s);
            dp = mfma32(*reinterpret_cast<const bf16x8_t*>(dl + off), vop[ks], dp);
        }

        // P = exp2(S*scale*log2e - lse*log2e) (0 where masked), dS = P (dP - delta) scale
        const float* st = reinterpret_cast<const float*>(smem + kBwStatOff + bi * kBwStatBytes);
        bf16x8_t pop[2], dsop[2];
        float dsv[16];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const f32x4_t nl = *reinterpret_cast<const f32x4_t*>(st + 8 * i + 4 * g2);
            const f32x4_t nd = *reinterpret_cast<const f32x4_t*>(st + kBwRows + 8 * i + 4 * g2);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int q = q0 + 8 * i + 4 * g2 + r;
                const bool valid = (q >= lo_row) && (q < p.sq);
                float pv = fast_exp2(__builtin_fmaf(s[4 * i + r], c2, nl[r]));
                pv = valid ? pv : 0.f;
                const float ds = pv * __builtin_fmaf(dp[4 * i + r], scale, nd[r]);
                pop[i >> 1][(i & 1) * 4 + r] = (__bf16)pv;
                dsop[i >> 1][(i & 1) * 4 + r] = (__bf16)ds;
                dsv[4 * i + r] = ds;
            }
        }

        // dV += P^T dO, dK += dS^T Q: C[key][d], 4 column tiles of D; the
        // k-step ks takes query rows 16ks + 4g2 + 0..3 and 16ks + 8 + 4g2 + 0..3
        // (registers 8ks .. 8ks+7 of S / dP), read transposed from the tiles.
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                const int rb = ks * 16 * kBwRowBytes;
                const bf16x4_t dlo = lds_read_tr16(reinterpret_cast<const __bf16*>(dl + rb + trq[db][0]));
                const bf16x4_t dhi = lds_read_tr16(reinterpret_cast<const __bf16*>(dl + rb + trq[db][1]));
                dv_acc[db] = mfma32(pop[ks], __builtin_shufflevector(dlo, dhi, 0, 1, 2, 3, 4, 5, 6, 7), dv_acc[db]);
                const bf16x4_t qlo = lds_read_tr16(reinterpret_cast<const __bf16*>(ql + rb + trq[db][0]));
                const bf16x4_t qhi = lds_read_tr16(reinterpret_cast<const __bf16*>(ql + rb + trq[db][1]));
                dk_acc[db] = mfma32(dsop[ks], __builtin_shufflevector(qlo, qhi, 0, 1, 2, 3, 4, 5, 6, 7), dk_acc[db]);
            }

        // dS^T rows of this wave's keys: query rows 8i + 4g2 .. +3 = chunk i, half g2
        unsigned char* dsl = smem + kBwDsOff + bi * kBwDsBytes;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            bf16x4_t w;
#pragma unroll
            for (int r = 0; r < 4; ++r) w[r] = (__bf16)dsv[4 * i + r];
            *reinterpret_cast<bf16x4_t*>(dsl + bw_ds_addr(key_l, i, g2)) = w;
        }

        prev_h = hh;
        prev_q0 = q0;
        bw_wait_vmem();
        __syncthreads();
    }
    if (n_iter > 0) dq_step((n_iter - 1) & 1, prev_h, prev_q0);

    // ---- dK, dV of this wave's keys: C[key][d], lane (d = 32db + l32, half g2),
    // register 4i + r <-> key 32w + 8i + 4g2 + r
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int j = kv0 + 32 * wave + 8 * i + 4 * g2 + r;
            if (j >= p.skv) continue;
            if (p.dk_acc != nullptr) {
                float* dkr = p.dk_acc + (((int64_t)b * p.hkv + kvh) * p.skv + j) * kHeadDim + l32;
                float* dvr = p.dv_acc + (((int64_t)b * p.hkv + kvh) * p.skv + j) * kHeadDim + l32;
#pragma unroll
                for (int db = 0; db < 4; ++db) {
                    atomic_add_f32(dkr + 32 * db, dk_acc[db][4 * i + r]);
                    atomic_add_f32(dvr + 32 * db, dv_acc[db][4 * i + r]);
                }
            } else {
                __bf16* dkr = p.dk + b * p.dk_sb + (int64_t)j * p.dk_ss + kvh * p.dk_sh + l32;
                __bf16* dvr = p.dv + b * p.dv_sb + (int64_t)j * p.dv_ss + kvh * p.dv_sh + l32;
#pragma unroll
                for (int db = 0; db < 4; ++db) {
                    dkr[32 * db] = (__bf16)dk_acc[db][4 * i + r];
                    dvr[32 * db] = (__bf16)dv_acc[db][4 * i + r];
                }
            }
        }
}

namespace {

struct BwdPlan {
    int n_hsplit;
    size_t stat_bytes, dq_bytes, dkv_bytes, ws_bytes;
};

size_t round256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

int validate_backward(const fgqa_prefill_backward_args* a) {
    if (a == nullptr) return FGQA_ERR_INVALID_ARGUMENT;
    if (a->batch < 0 || a->seqlen_q < 0 || a->seqlen_kv < 0 || a->num_q_heads <= 0 ||
        a->num_kv_heads <= 0 || a->head_dim <= 0)
        return FGQA_ERR_INVALID_ARGUMENT;
    if (a->num_q_heads % a->num_kv_heads != 0) return FGQA_ERR_INVALID_ARGUMENT;
    if (!isfinite(a->scale)) return FGQA_ERR_INVALID_ARGUMENT;
    const int64_t* strides[8] = {a->q_stride, a->k_stride, a->v_stride, a->o_stride,
                                 a->grad_o_stride, a->grad_q_stride, a->grad_k_stride, a->grad_v_stride};
    for (const int64_t* s : strides)
        for (int i = 0; i < 3; ++i)
            if (s[i] < 0) return FGQA_ERR_INVALID_ARGUMENT;
    if (a->head_dim != kHeadDim) return FGQA_ERR_UNSUPPORTED;
    const int64_t lim = (int64_t)1 << 31;
    if ((int64_t)(a->seqlen_q + 128) * a->q_stride[1] * 2 >= lim ||
        (int64_t)(a->seqlen_q + 128) * a->grad_o_stride[1] * 2 >= lim ||
        (int64_t)(a->seqlen_kv + 128) * a->k_stride[1] * 2 >= lim ||
        (int64_t)(a->seqlen_kv + 128) * a->v_stride[1] * 2 >= lim)
        return FGQA_ERR_UNSUPPORTED;
    // the row statistics are addressed through one buffer resource
    if ((int64_t)a->batch * a->num_q_heads * a->seqlen_q * 8 >= lim) return FGQA_ERR_UNSUPPORTED;
    return FGQA_OK;
}

int validate_backward_pointers(const fgqa_prefill_backward_args* a) {
    if (a->q == nullptr || a->k == nullptr || a->v == nullptr || a->o == nullptr || a->lse == nullptr ||
        a->grad_o == nullptr || a->grad_q == nullptr || a->grad_k == nullptr || a->grad_v == nullptr)
        return FGQA_ERR_INVALID_ARGUMENT;
    const void* ptrs[8] = {a->q, a->k, a->v, a->o, a->grad_o, a->grad_q, a->grad_k, a->grad_v};
    for (const void* ptr : ptrs)
        if (!aligned16(ptr)) return FGQA_ERR_UNSUPPORTED;
    const int64_t* strides[8] = {a->q_stride, a->k_stride, a->v_stride, a->o_stride,
                                 a->grad_o_stride, a->grad_q_stride, a->grad_k_stride, a->grad_v_stride};
    for (const int64_t* s : strides)
        for (int i = 0; i < 3; ++i)
            if (s[i] & 7) return FGQA_ERR_UNSUPPORTED;
    return FGQA_OK;
}

// Heads per workgroup: all G query heads of a KV head (dK/dV written once,
// straight from registers) unless that leaves fewer than 2 workgroups per CU,
// in which case the heads are split over workgroups and dK/dV go through fp32
// accumulators.  FGQA_BWD_HSPLIT=<n> forces n (a divisor of G) for tests.
BwdPlan plan_backward(const fgqa_prefill_backward_args* a, int cus) {
    BwdPlan pl;
    const int group = a->num_q_heads / a->num_kv_heads;
    const int64_t base = ceil_div(a->seqlen_kv, kBwKeys) * (int64_t)a->num_kv_heads * a->batch;
    pl.n_hsplit = group;
    for (int d = 1; d <= group; ++d)
        if (group % d == 0 && base * d >= 2 * (int64_t)cus) {
            pl.n_hsplit = d;
            break;
        }
    if (const char* e = getenv("FGQA_BWD_HSPLIT")) {
        const int d = atoi(e);
        if (d >= 1 && d <= group && group % d == 0) pl.n_hsplit = d;
    }
    const size_t rows_q = (size_t)a->batch * a->num_q_heads * a->seqlen_q;
    const size_t rows_kv = (size_t)a->batch * a->num_kv_heads * a->seqlen_kv;
    pl.stat_bytes = round256(2 * rows_q * sizeof(float));
    pl.dq_bytes = round256(rows_q * kHeadDim * sizeof(float));
    pl.dkv_bytes = pl.n_hsplit > 1 ? round256(rows_kv * kHeadDim * sizeof(float)) : 0;
    pl.ws_bytes = pl.stat_bytes + pl.dq_bytes + 2 * pl.dkv_bytes;
    return pl;
}

}  // namespace
}  // namespace fgqa

using namespace fgqa;

extern "C" int fgqa_prefill_backward_workspace_bytes(const fgqa_prefill_backward_args* a, size_t* bytes) {
    if (bytes == nullptr) return FGQA_ERR_INVALID_ARGUMENT;
    const int st = validate_backward(a);
    if (st != FGQA_OK) return st;
    const int cus = device_cu_count();
    if (cus <= 0) return FGQA_ERR_HIP;
    *bytes = plan_backward(a, cus).ws_bytes;
    return FGQA_OK;
}

extern "C" int fgqa_prefill_backward_bf16(const fgqa_prefill_backward_args* a, void* stream) {
    int st = validate_backward(a);
    if (st != FGQA_OK) return st;
    if (a->batch == 0 || (a->seqlen_q == 0 && a->seqlen_kv == 0)) return FGQA_OK;
    st = validate_backward_pointers(a);
    if (st != FGQA_OK) return st;
    const int cus = device_cu_count();
    if (cus <= 0) return FGQA_ERR_HIP;
    const BwdPlan pl = plan_backward(a, cus);

    unsigned char* ws = static_cast<unsigned char*>(a->workspace);
    if (ws == nullptr) {
        ws = static_cast<unsigned char*>(internal_workspace(pl.ws_bytes, &st));
        if (ws == nullptr) return st;
    } else if (a->workspace_bytes < pl.ws_bytes) {
        return FGQA_ERR_WORKSPACE;
    } else if ((reinterpret_cast<uintptr_t>(ws) & 255) != 0) {
        return FGQA_ERR_UNSUPPORTED;
    }

    BwdParams p;
    p.q = static_cast<const __bf16*>(a->q);
    p.k = static_cast<const __bf16*>(a->k);
    p.v = static_cast<const __bf16*>(a->v);
    p.o = static_cast<const __bf16*>(a->o);
    p.dout = static_cast<const __bf16*>(a->grad_o);
    p.lse = a->lse;
    p.dq = static_cast<__bf16*>(a->grad_q);
    p.dk = static_cast<__bf16*>(a->grad_k);
    p.dv = static_cast<__bf16*>(a->grad_v);
    p.q_sb = a->q_stride[0]; p.q_ss = a->q_stride[1]; p.q_sh = a->q_stride[2];
    p.k_sb = a->k_stride[0]; p.k_ss = a->k_stride[1]; p.k_sh = a->k_stride[2];
    p.v_sb = a->v_stride[0]; p.v_ss = a->v_stride[1]; p.v_sh = a->v_stride[2];
    p.o_sb = a->o_stride[0]; p.o_ss = a->o_stride[1]; p.o_sh = a->o_stride[2];
    p.do_sb = a->grad_o_stride[0]; p.do_ss = a->grad_o_stride[1]; p.do_sh = a->grad_o_stride[2];
    p.dq_sb = a->grad_q_stride[0]; p.dq_ss = a->grad_q_stride[1]; p.dq_sh = a->grad_q_stride[2];
    p.dk_sb = a->grad_k_stride[0]; p.dk_ss = a->grad_k_stride[1]; p.dk_sh = a->grad_k_stride[2];
    p.dv_sb = a->grad_v_stride[0]; p.dv_ss = a->grad_v_stride[1]; p.dv_sh = a->grad_v_stride[2];
    p.rowstat = reinterpret_cast<float*>(ws);
    p.dq_acc = reinterpret_cast<float*>(ws + pl.stat_bytes);
    p.dk_acc = pl.n_hsplit > 1 ? reinterpret_cast<float*>(ws + pl.stat_bytes + pl.dq_bytes) : nullptr;
    p.dv_acc = pl.n_hsplit > 1 ? reinterpret_cast<float*>(ws + pl.stat_bytes + pl.dq_bytes + pl.dkv_bytes) : nullptr;
    p.batch = a->batch;
    p.sq = a->seqlen_q;
    p.skv = a->seqlen_kv;
    p.hq = a->num_q_heads;
    p.hkv = a->num_kv_heads;
    p.group = a->num_q_heads / a->num_kv_heads;
    p.causal = a->causal ? 1 : 0;
    p.n_hsplit = pl.n_hsplit;
    p.hs = p.group / pl.n_hsplit;
    p.n_kvblocks = (int)ceil_div(p.skv, kBwKeys);
    p.n_streams = pl.n_hsplit * p.hkv * p.batch;
    p.n_qblocks = (int)ceil_div(p.sq, kBwRows);
    p.scale = a->scale;
    p.scale_log2 = a->scale * kLog2e;

    const hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t rows_q = (int64_t)p.batch * p.hq * p.sq;
    const int64_t rows_kv = (int64_t)p.batch * p.hkv * p.skv;
    const int64_t rows = (pl.n_hsplit > 1 && rows_kv > rows_q) ? rows_kv : rows_q;
    const int64_t units = (int64_t)p.n_kvblocks * p.n_streams;
    if (ceil_div(rows, 16) >= ((int64_t)1 << 31) || units >= ((int64_t)1 << 31)) return FGQA_ERR_UNSUPPORTED;

    if (rows > 0) hipLaunchKernelGGL(bwd_prep_kernel, dim3((unsigned)ceil_div(rows, 16)), dim3(256), 0, s, p);
    if (units > 0) {
        static bool smem_set = false;
        if (!smem_set) {
            if (hipFuncSetAttribute(reinterpret_cast<const void*>(bwd_kv_kernel),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, kBwSmemBytes) != hipSuccess)
                return FGQA_ERR_HIP;
            smem_set = true;
        }
        hipLaunchKernelGGL(bwd_kv_kernel, dim3((unsigned)units), dim3(kBwThreads), kBwSmemBytes, s, p);
    }
    if (rows > 0) hipLaunchKernelGGL(bwd_convert_kernel, dim3((unsigned)ceil_div(rows, 16)), dim3(256), 0, s, p);
    if (hipGetLastError() != hipSuccess) return FGQA_ERR_HIP;
    return FGQA_OK;
}
