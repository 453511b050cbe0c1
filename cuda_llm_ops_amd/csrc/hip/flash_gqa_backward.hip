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
// The reference adds dQ (and dK, dV) with fp32 atomics.  On MI355X a float
// atomic add sustains ~1.3 TB/s against ~10 TB/s for plain stores, and the
// dQ updates alone are ~0.55 GB at the 4096-token, 16-head shape, so here no
// gradient goes through an atomic: each is owned by exactly one workgroup and
// P, dP are recomputed where needed.  Results are deterministic.
//
// Launches on the caller's stream, in this order:
//   bwd_dq_kernel      query-major, the forward kernel's work unit (128 query
//                      rows: heads x positions of one KV group, one wave per
//                      32 rows): first each row's -lse*log2(e) and
//                      -delta*scale (stored for dK/dV), then per 64-key tile
//                      S^T = K Q^T, dP^T = V dO^T (Q^T, dO^T in registers,
//                      K/V tiles in LDS), dS^T on the VALU, dQ^T += K^T dS^T
//                      (K read transposed).  bwd_dq_split_kernel: the same
//                      unit with its key range split over two wave groups.
//   bwd_dkdv_kernel    key-major: a workgroup owns a 128-key block of one KV
//                      head (wave w: keys 32w..32w+31, K/V rows in registers)
//                      and loops over (query head of its subset, 32-row query
//                      block):  S = Q K^T, dP = dO V^T (Q/dO rows from LDS),
//                      P and dS on the VALU (in place as bf16 A operands),
//                      dV += P^T dO, dK += dS^T Q (dO/Q read transposed,
//                      ds_read_b64_tr_b16).  dK/dV stay in registers (fp32).
//   bwd_dkdv_reduce_kernel  only when a KV head's query heads are split over
//                      several workgroups: sums their fp32 partial dK/dV.
#include <math.h>
#include <stdint.h>

#include <type_traits>

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
    float* dk_part;   // [n_hsplit][B, Hkv, Skv, D] fp32 partial sums (heads split), else null
    float* dv_part;
    int batch, sq, skv, hq, hkv, group, causal;
    int window;       // > 0: sliding window (causal), row i uses keys (i - window, i]
    // key-major (dK/dV) grid
    int hs;           // query heads per workgroup
    int n_hsplit;     // group / hs
    int n_kvblocks;   // ceil(skv / 128)
    int kv_streams;   // n_hsplit * hkv * batch
    int n_qblocks32;  // ceil(sq / 32)
    // query-major (dQ) grid, as the forward's
    int hb;           // heads per 128-row unit
    int n_hgroups;    // group / hb
    int n_qunits;     // ceil(sq / (128 / hb))
    int q_streams;    // n_hgroups * hkv * batch
    float scale;
    float scale_log2;   // scale * log2(e)
};

constexpr int kBwWaves = 4;
constexpr int kBwThreads = kBwWaves * kWave;
constexpr int kBwRowBytes = kHeadDim * 2;             // one Q / dO / K / V row
constexpr int kBwHiRowBytes = 128;                    // dims 128..191 of a 192-wide Q / K row

// ---- key-major kernel
constexpr int kKvRing = 6;                            // operands read ahead in a step
constexpr int kKvKeys = 128;                          // keys per workgroup
constexpr int kKvRows = 32;                           // query rows per step
constexpr int kKvTileBytes = kKvRows * kBwRowBytes;   // 8 KB: Q or dO of one step
constexpr int kKvStatBytes = 2 * kKvRows * 4;         // -lse*log2e and -delta*scale of 32 rows
// LDS: Q[3] | dO[3] | stats[3]
constexpr int kKvQOff = 0;
constexpr int kKvDoOff = 3 * kKvTileBytes;
constexpr int kKvStatOff = 6 * kKvTileBytes;
constexpr int kKvSmemBytes = kKvStatOff + 3 * kKvStatBytes;
// MLA: the 128-byte parts of Q[3] follow
constexpr int kKvQHiTileBytes = kKvRows * kBwHiRowBytes;   // 4 KB
constexpr int kKvQHiOff = kKvSmemBytes;
template <int kDk>
constexpr int kv_smem_bytes() { return kDk > 128 ? kKvSmemBytes + 3 * kKvQHiTileBytes : kKvSmemBytes; }

// ---- query-major kernel
constexpr int kDqTile = 64;                           // keys per tile
constexpr int kDqTileBytes = kDqTile * kBwRowBytes;   // 16 KB
// LDS: K[2] | V[2]
constexpr int kDqSmemBytes = 4 * kDqTileBytes;
// MLA: the 128-byte parts of K[2] follow
constexpr int kDqKHiTileBytes = kDqTile * kBwHiRowBytes;   // 8 KB
constexpr int kDqKHiOff = kDqSmemBytes;
template <int kDk>
constexpr int dq_smem_bytes() { return kDk > 128 ? kDqSmemBytes + 2 * kDqKHiTileBytes : kDqSmemBytes; }

// Q, dO, K and V rows (256 B) sit in LDS with their 16-byte chunks permuted:
// chunk c of row r goes to slot c ^ bw_swz(r).  bw_swz is a bijection on
// r % 16 (16 consecutive rows read at the same chunk hit 16 different slots:
// conflict-free b128 row reads) whose top two bits are r % 4 (4 consecutive
// rows read over 4 consecutive chunks hit 4 disjoint slot groups:
// conflict-free transposed reads).
__device__ __forceinline__ int bw_swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

__device__ __forceinline__ void bw_dma16(uint32_t lds_addr, uint32_t voffset, __amdgpu_buffer_rsrc_t rsrc) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :: "s"(lds_addr), "v"(voffset), "s"(rsrc) : "memory");
}
__device__ __forceinline__ void bw_dma4(uint32_t lds_addr, uint32_t voffset, __amdgpu_buffer_rsrc_t rsrc) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds"
                 :: "s"(lds_addr), "v"(voffset), "s"(rsrc) : "memory");
}
__device__ __forceinline__ void bw_wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Byte offset, within a block of 16 swizzled 256-byte rows, that lane supplies
// to a transposed read (ds_read_b64_tr_b16) so that the wave receives the
// 32x32x16 MFMA operand  X[k = row][n = 32*cb + l32]  with the k order used
// throughout: slots 0..3 of lane (l32, half g2) = rows 4*g2 + 0..3 (h8 = 0),
// slots 4..7 = rows 8 + 4*g2 + 0..3 (h8 = 1).  Source lane (g2, gq, l16)
// points at row 4*g2 + l16/4 + 8*h8, columns 32*cb + 16*gq + 4*(l16%4) .. +3.
__device__ __forceinline__ int bw_tr_off(int lane, int cb, int h8) {
    const int l16 = lane & 15, gq = (lane >> 4) & 1, g2 = lane >> 5;
    const int r = 4 * g2 + (l16 >> 2) + 8 * h8;
    const int c = 4 * cb + 2 * gq + ((l16 >> 1) & 1);
    return r * kBwRowBytes + ((c ^ bw_swz(r)) << 4) + 8 * (l16 & 1);
}

// MLA (Q/K head dim 192, V/O 128): a 192-wide Q or K row is kept as a
// 256-byte part (dims 0..127, laid out as above) and a 128-byte part (dims
// 128..191) in a separate tile, whose chunk c of row r sits in slot
// c ^ bw_swz_hi(r).  bw_swz_hi is a bijection on (r / 2) % 8: 16 consecutive
// rows read at one chunk fall in 16 different 16-byte bank groups (rows of
// either parity share none, 128-byte rows alternate halves of a 256-byte
// bank line).  Its top bit is (r / 2) % 2: rows r and r + 2 read over 4
// consecutive chunks land in different 4-chunk halves, so the transposed
// reads are conflict-free too.
__device__ __forceinline__ int bw_swz_hi(int r) { return (((r >> 1) & 1) << 2) | ((r >> 2) & 3); }
// bw_tr_off for the 128-byte part (column block cb = 0, 1: dims 128 + 32cb ..)
__device__ __forceinline__ int bw_tr_off_hi(int lane, int cb, int h8) {
    const int l16 = lane & 15, gq = (lane >> 4) & 1, g2 = lane >> 5;
    const int r = 4 * g2 + (l16 >> 2) + 8 * h8;
    const int c = 4 * cb + 2 * gq + ((l16 >> 1) & 1);
    return r * kBwHiRowBytes + ((c ^ bw_swz_hi(r)) << 4) + 8 * (l16 & 1);
}
template <int kDk>
struct BwDims {
    static_assert(kDk == 128 || kDk == 192, "Q/K head dim");
    static constexpr bool kHi = kDk > 128;        // a 128-byte part per row
    static constexpr int kRowBytes = kDk * 2;     // one Q / K row in HBM
    static constexpr int kSteps = kDk / 16;       // MFMA k-steps of S over the Q/K dim
    static constexpr int kDb = kDk / 32;          // 32-column blocks of dQ / dK
};

__device__ __forceinline__ bf16x8_t tr_pair(const unsigned char* base, int off0, int off1) {
    const bf16x4_t lo = lds_read_tr16(reinterpret_cast<const __bf16*>(base + off0));
    const bf16x4_t hi = lds_read_tr16(reinterpret_cast<const __bf16*>(base + off1));
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

template <int N, int I = 0, typename F>
__device__ __forceinline__ void bw_static_for(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        bw_static_for<N, I + 1>(f);
    }
}

// ---------------------------------------------------------------- row statistics
// -lse*log2(e) and -delta*scale of one query row, delta = sum_d O[d] dO[d],
// computed by the dQ kernels (which hold the row's dO) and stored for the
// dK/dV kernel that runs after them.  A lane holds elements 16kk + 8g2 .. +7
// of the row (kk = 0..7): part 2kk + g2 of 16 eight-element parts.  delta is
// the parts' sums added as a balanced tree over the part index (partner
// p ^ 1, then p ^ 2, p ^ 4, p ^ 8), so it does not depend on how the row is
// spread over lanes.
__device__ __forceinline__ float row_delta(const bf16x8_t (&oop)[8], const bf16x8_t (&doop)[8]) {
    float pair[8];   // parts 2kk and 2kk + 1 (the other half-wave holds the second)
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
        float acc = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc += (float)oop[kk][e] * (float)doop[kk][e];
        pair[kk] = xor_sum(acc, 32);
    }
    return ((pair[0] + pair[1]) + (pair[2] + pair[3])) + ((pair[4] + pair[5]) + (pair[6] + pair[7]));
}

// ---------------------------------------------------------------- dK / dV
// Software pipelined one step ahead: step t runs
//   phase A: S(t+1), dP(t+1) on the MFMA pipe  ||  P(t), dS(t) on the VALU
//   phase B: dV += P(t)^T dO(t), dK += dS(t)^T Q(t) on the MFMA pipe
// with Q/dO(t+2) streaming into the third LDS buffer meanwhile.
// kSwa: sliding window (a separate instantiation, so the causal kernels carry
// none of its work).  kAddMask: the mask enters as an additive -inf on S (any
// nonzero scale); without it (scale 0, where -inf * 0 is not -inf) as a select
// on P.
template <bool kSwa, int kDk, bool kAddMask>
__global__ __launch_bounds__(kBwThreads, 1) void bwd_dkdv_kernel(BwdParams p) {
    using D = BwDims<kDk>;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int l32 = lane & 31;
    const int l16 = lane & 15;
    const int g2 = lane >> 5;
    const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)smem;

    // Block -> (key block, head subset, kv head, batch).  Key blocks in
    // ascending order: under the causal mask block 0 sees every query block,
    // so the heaviest workgroups are dispatched first.
    const int stream = blockIdx.x % p.kv_streams;
    const int kb = blockIdx.x / p.kv_streams;
    const int hsp = stream % p.n_hsplit;
    const int kvh = (stream / p.n_hsplit) % p.hkv;
    const int b = stream / (p.n_hsplit * p.hkv);
    const int kv0 = kb * kKvKeys;
    const int h0 = kvh * p.group + hsp * p.hs;

    // K, V rows of this wave's keys as B operands of S = Q K^T, dP = dO V^T:
    // lane (key l32, half g2), k-step ks holds elements 16ks + 8g2 .. +7.
    // Keys >= skv read as zero.
    const uint32_t kss = (uint32_t)(p.k_ss * 2);
    const uint32_t vss = (uint32_t)(p.v_ss * 2);
    const __amdgpu_buffer_rsrc_t krs =
        make_rsrc(p.k + b * p.k_sb + kvh * p.k_sh, (uint32_t)(p.skv - 1) * kss + D::kRowBytes);
    const __amdgpu_buffer_rsrc_t vrs =
        make_rsrc(p.v + b * p.v_sb + kvh * p.v_sh, (uint32_t)(p.skv - 1) * vss + kBwRowBytes);
    const int key = kv0 + 32 * wave + l32;   // this lane's key (column of S)
    bf16x8_t kop[D::kSteps], vop[8];
#pragma unroll
    for (int ks = 0; ks < D::kSteps; ++ks)
        kop[ks] = as_bf16x8(buf_load16(krs, (uint32_t)key * kss + (16 * ks + 8 * g2) * 2));
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
        vop[ks] = as_bf16x8(buf_load16(vrs, (uint32_t)key * vss + (16 * ks + 8 * g2) * 2));

    // step t: head h0 + t / per_head, query block qb0 + t % per_head
    const int qb0 = p.causal ? min(kv0 / kKvRows, p.n_qblocks32) : 0;
    // a window ends the key block's rows at its last key + window - 1
    const int qb_end = kSwa ? min(p.n_qblocks32, (kv0 + kKvKeys + p.window - 2) / kKvRows + 1) : p.n_qblocks32;
    const int per_head = max(0, qb_end - qb0);
    const int n_iter = p.hs * per_head;

    const uint32_t qss = (uint32_t)(p.q_ss * 2);
    const uint32_t dss = (uint32_t)(p.do_ss * 2);
    const int64_t rows_q = (int64_t)p.batch * p.hq * p.sq;
    const __amdgpu_buffer_rsrc_t srs = make_rsrc(p.rowstat, (uint32_t)(2 * rows_q * 4));
    // Q, dO rows of step t (wave w fetches rows 8w..8w+7 of each) and their
    // statistics (wave 0) into buffer bi.  Rows >= sq read as zero.
    // Steps are loaded in order, so the (head, query block) of the next load
    // advances by one per call (no division per step).
    int ld_h = h0, ld_qb = qb0;
    int cur_qb = qb0;   // query block of the step being computed
    auto issue = [&](int bi) {
        const int hh = ld_h;
        const int q0 = ld_qb * kKvRows;
        if (++ld_qb == qb_end) {
            ld_qb = qb0;
            ++ld_h;
        }
        const __amdgpu_buffer_rsrc_t qrs =
            make_rsrc(p.q + b * p.q_sb + hh * p.q_sh, (uint32_t)(p.sq - 1) * qss + D::kRowBytes);
        const __amdgpu_buffer_rsrc_t drs =
            make_rsrc(p.dout + b * p.do_sb + hh * p.do_sh, (uint32_t)(p.sq - 1) * dss + kBwRowBytes);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int r0 = 8 * wave + 4 * j;
            const int r = r0 + (lane >> 4);
            const int slot = (l16 ^ bw_swz(r)) << 4;
            bw_dma16(lds_base + kKvQOff + bi * kKvTileBytes + r0 * kBwRowBytes, (uint32_t)(q0 + r) * qss + slot, qrs);
            bw_dma16(lds_base + kKvDoOff + bi * kKvTileBytes + r0 * kBwRowBytes, (uint32_t)(q0 + r) * dss + slot, drs);
        }
        if constexpr (D::kHi) {
            // dims 128..191 of rows 8w..8w+7: lane l fills slot l % 8 of row 8w + l / 8
            const int r = 8 * wave + (lane >> 3);
            const int c = (lane & 7) ^ bw_swz_hi(r);
            bw_dma16(lds_base + kKvQHiOff + bi * kKvQHiTileBytes + 8 * wave * kBwHiRowBytes,
                     (uint32_t)(q0 + r) * qss + kBwRowBytes + 16 * c, qrs);
        }
        if (wave == 0) {
            const int r = q0 + l32;
            const int64_t idx = ((int64_t)b * p.hq + hh) * p.sq + r + (g2 ? rows_q : 0);
            const uint32_t off = (r < p.sq) ? (uint32_t)(idx * 4) : 0xFFFFFFF0u;   // out of range -> 0
            bw_dma4(lds_base + kKvStatOff + bi * kKvStatBytes, off, srs);
        }
    };

    f32x16_t dk_acc[D::kDb], dv_acc[4];
#pragma unroll
    for (int db = 0; db < D::kDb; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) dk_acc[db][i] = 0.f;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) dv_acc[db][i] = 0.f;

    // transposed-read offsets into the Q / dO tiles
    int trq[4][2], trq_hi[2][2];
#pragma unroll
    for (int db = 0; db < 4; ++db) {
        trq[db][0] = bw_tr_off(lane, db, 0);
        trq[db][1] = bw_tr_off(lane, db, 1);
    }
    if constexpr (D::kHi) {
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            trq_hi[cb][0] = bw_tr_off_hi(lane, cb, 0);
            trq_hi[cb][1] = bw_tr_off_hi(lane, cb, 1);
        }
    }
    // b128 row-read offsets of the A operands of S and dP (row l32, chunk 2ks + g2)
    int roff[8], roff_hi[4];
    const int fl = bw_swz(l32);
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) roff[ks] = l32 * kBwRowBytes + (((2 * ks + g2) ^ fl) << 4);
    if constexpr (D::kHi) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
            roff_hi[ks] = l32 * kBwHiRowBytes + (((2 * ks + g2) ^ bw_swz_hi(l32)) << 4);
    }
    const float c2 = p.scale_log2;
    const float scale = p.scale;
    // S = Q K^T and dP = dO V^T of the step in buffer bi: C[q][key], lane
    // (key l32, half g2), register 4i + r <-> query row 8i + 4g2 + r
    // Element (i, r) of a step's S block is query row q0 + 8i + 4g2 + r; it is
    // masked (P = 0) when 8i + r < m, with m = key - q0 - 4g2 under the causal
    // mask, and (window) when 8i + r > mx, mx = key + window - 1 - q0 - 4g2;
    // steps past n_iter are fully masked.  Rows >= sq need no mask: their dO
    // rows and -delta*scale read as zero, so P.dO and dS vanish; keys >= skv
    // only reach their own dK/dV rows, which are never stored.
    //
    // kAddMask: the accumulator of a step's S starts at 0 or, on a step whose
    // block the mask cuts (wave-uniform: the diagonal, the window's edge,
    // padding), at ninf for each masked element, ninf = -inf times the sign of
    // scale, so that S * scale * log2(e) is -inf and P = exp2(-inf) = +0 and
    // dS = 0 * x, the values the select gives (for finite Q and K).  Only the
    // first MFMA of S's chain differs between the two (its C operand: the
    // literal 0, or the start values), and the softmax carries no
    // per-element select: two VALU ops per element fewer.
    const int wk0 = kv0 + 32 * wave;   // the wave's first key
    const float ninf = c2 > 0.f ? -INFINITY : INFINITY;
    auto is_cut = [&](int ts, int q0s) {
        bool cut = ts >= n_iter || (p.causal && q0s < wk0 + 31);
        if constexpr (kSwa) cut = cut || q0s + 31 > wk0 + p.window - 1;
        return cut;
    };
    // the start values of a cut step's S block
    auto bias = [&](int ts, int q0s) {
        const int m = (ts < n_iter) ? (p.causal ? key - q0s - 4 * g2 : -64) : 64;
        const int mx = key + p.window - 1 - q0s - 4 * g2;
        f32x16_t b;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const bool vis = kSwa ? (8 * i + r >= m && 8 * i + r <= mx) : (8 * i + r >= m);
                b[4 * i + r] = vis ? 0.f : ninf;
            }
        return b;
    };
    // S's first MFMA (k-step 0), with the mask's start values on cut steps
    auto s_first = [&](const bf16x8_t& a, int ts, int q0s) -> f32x16_t {
        f32x16_t z;
#pragma unroll
        for (int i = 0; i < 16; ++i) z[i] = 0.f;
        if (kAddMask && is_cut(ts, q0s)) return mfma32(a, kop[0], bias(ts, q0s));
        return mfma32(a, kop[0], z);
    };
    auto sdp = [&](f32x16_t& s, f32x16_t& dp, auto bi_c) {
        constexpr int bi = decltype(bi_c)::value;
        const unsigned char* ql = smem + kKvQOff + bi * kKvTileBytes;
        const unsigned char* dl = smem + kKvDoOff + bi * kKvTileBytes;
#pragma unroll
        for (int i = 0; i < 16; ++i) dp[i] = 0.f;
        s = s_first(*reinterpret_cast<const bf16x8_t*>(ql + roff[0]), 0, qb0 * kKvRows);
        dp = mfma32(*reinterpret_cast<const bf16x8_t*>(dl + roff[0]), vop[0], dp);
#pragma unroll
        for (int ks = 1; ks < 8; ++ks) {
            s = mfma32(*reinterpret_cast<const bf16x8_t*>(ql + roff[ks]), kop[ks], s);
            dp = mfma32(*reinterpret_cast<const bf16x8_t*>(dl + roff[ks]), vop[ks], dp);
        }
        if constexpr (D::kHi) {
            const unsigned char* qh = smem + kKvQHiOff + bi * kKvQHiTileBytes;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
                s = mfma32(*reinterpret_cast<const bf16x8_t*>(qh + roff_hi[ks]), kop[8 + ks], s);
        }
    };
    // P = exp2(S*scale*log2e - lse*log2e), dS = P (dP - delta) scale, both as
    // bf16 A operands (k-step ks = registers 8ks .. 8ks+7); without kAddMask
    // the mask above is a select here.
    bf16x8_t pop[2], dsop[2];
    auto softmax = [&](const f32x16_t& s, const f32x16_t& dp, auto bi_c, int m, int mx) {
        constexpr int bi = decltype(bi_c)::value;
        const float* st = reinterpret_cast<const float*>(smem + kKvStatOff + bi * kKvStatBytes);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const f32x4_t nl = *reinterpret_cast<const f32x4_t*>(st + 8 * i + 4 * g2);
            const f32x4_t nd = *reinterpret_cast<const f32x4_t*>(st + kKvRows + 8 * i + 4 * g2);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float pv = fast_exp2(__builtin_fmaf(s[4 * i + r], c2, nl[r]));
                if constexpr (!kAddMask && kSwa)
                    pv = (8 * i + r >= m && 8 * i + r <= mx) ? pv : 0.f;
                else if constexpr (!kAddMask)
                    pv = (8 * i + r >= m) ? pv : 0.f;
                const float ds = pv * __builtin_fmaf(dp[4 * i + r], scale, nd[r]);
                pop[i >> 1][(i & 1) * 4 + r] = (__bf16)pv;
                dsop[i >> 1][(i & 1) * 4 + r] = (__bf16)ds;
            }
        }
    };

    // Triple-buffered Q/dO: step t reads buffers t%3 (dV/dK) and (t+1)%3
    // (S/dP of the next step) while step t+2 lands in (t+2)%3, which step t-1
    // finished with before the barrier that ended it.  The loop runs a
    // multiple of 3 steps so that every buffer offset is a constant; steps
    // past n_iter are fully masked (m = 64) and read buffers that hold zeros
    // or an earlier step's rows, so they add exact zeros.  No branch touches
    // the accumulators.
    {
        // zero the buffers first: a padded step may read one never loaded
        const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
        for (int off = tid * 16; off < kv_smem_bytes<kDk>(); off += kBwThreads * 16)
            *reinterpret_cast<f32x4_t*>(smem + off) = z;
    }
    __syncthreads();
    if (n_iter > 0) issue(0);
    if (n_iter > 1) issue(1);
    bw_wait_vmem();
    __syncthreads();

    using C0 = std::integral_constant<int, 0>;
    using C1 = std::integral_constant<int, 1>;
    using C2 = std::integral_constant<int, 2>;
    // step t: sc/dpc hold S/dP(t), sn/dpn receive S/dP(t+1); buffers BC = t%3,
    // BN = (t+1)%3, BF = (t+2)%3
    auto step = [&](f32x16_t& sc, f32x16_t& dpc, f32x16_t& sn, f32x16_t& dpn, int t, auto bc, auto bn, auto bf) {
        if (t + 2 < n_iter) issue(decltype(bf)::value);
        // query block of step t (advanced once per step, as the loads are)
        const int q0 = cur_qb * kKvRows;
        if (++cur_qb == qb_end) cur_qb = qb0;
        [[maybe_unused]] const int m = (t < n_iter) ? (p.causal ? key - q0 - 4 * g2 : -64) : 64;
        [[maybe_unused]] const int mx = key + p.window - 1 - q0 - 4 * g2;

        // S/dP(t+1), then dV += P^T dO and dK += dS^T Q of step t (C[key][d],
        // 4 column tiles of D; k-step ks takes query rows 16ks + 4g2 + 0..3
        // and 16ks + 8 + 4g2 + 0..3, read transposed from the tiles), as one
        // stream of operands read kKvRing MFMAs ahead into a ring of
        // registers (6 ahead: 0.4 % faster than 4 at the 4096-token, 16-head
        // shape, 1.5 % with the MLA head dims); P/dS(t) on the VALU between
        // (the scheduler moves them up under the S/dP MFMAs).  Pinning the
        // order with sched_group_barrier
        // (reads kKvRing ahead, with or without the VALU spread over the S/dP
        // MFMAs) was 5-17 % slower.
        constexpr int BC = decltype(bc)::value, BN = decltype(bn)::value;
        constexpr int kS = D::kHi ? 20 : 16;
        constexpr int kOps = kS + (D::kHi ? 20 : 16);
        constexpr int kR = kKvRing;
        const unsigned char* qln = smem + kKvQOff + BN * kKvTileBytes;
        const unsigned char* dln = smem + kKvDoOff + BN * kKvTileBytes;
        const unsigned char* qlc = smem + kKvQOff + BC * kKvTileBytes;
        const unsigned char* dlc = smem + kKvDoOff + BC * kKvTileBytes;
        auto fetch = [&](auto ic) -> bf16x8_t {
            constexpr int i = decltype(ic)::value;
            if constexpr (i < 16) {
                // S (i even) / dP (i odd) A operand, k-step i / 2
                return *reinterpret_cast<const bf16x8_t*>((i % 2 == 0 ? qln : dln) + roff[i / 2]);
            } else if constexpr (i < kS) {
                const unsigned char* qh = smem + kKvQHiOff + BN * kKvQHiTileBytes;
                return *reinterpret_cast<const bf16x8_t*>(qh + roff_hi[(i - 16) % 4]);
            } else if constexpr (i < kS + 16) {
                // dV (r even) / dK (r odd) B operand: k-step r / 8, column block (r / 2) % 4
                constexpr int r = i - kS, ks = r / 8, db = (r / 2) % 4;
                return tr_pair((r % 2 == 0 ? dlc : qlc) + ks * 16 * kBwRowBytes, trq[db % 4][0], trq[db % 4][1]);
            } else {
                constexpr int r = i - kS - 16, ks = r / 2, cb = r % 2;
                const unsigned char* qh = smem + kKvQHiOff + BC * kKvQHiTileBytes + ks * 16 * kBwHiRowBytes;
                return tr_pair(qh, trq_hi[cb % 2][0], trq_hi[cb % 2][1]);
            }
        };
        bf16x8_t ring[kR];
        bw_static_for<kR>([&](auto ic) { ring[decltype(ic)::value] = fetch(ic); });
#pragma unroll
        for (int i = 0; i < 16; ++i) dpn[i] = 0.f;
        // S(t+1)'s first MFMA ahead of the scheduled stream (cur_qb is now
        // step t+1's block); its operand slot is refilled as op 0 would
        sn = s_first(ring[0], t + 1, cur_qb * kKvRows);
        ring[0] = fetch(std::integral_constant<int, kR>{});
        auto op = [&](auto ic) {
            constexpr int i = decltype(ic)::value;
            const bf16x8_t a = ring[i % kR];
            if constexpr (i == 0) {
                (void)a;   // issued above
            } else if constexpr (i < 16) {
                if constexpr (i % 2 == 0) sn = mfma32(a, kop[i / 2], sn);
                else dpn = mfma32(a, vop[i / 2], dpn);
            } else if constexpr (i < kS) {
                sn = mfma32(a, kop[8 + (i - 16) % 4], sn);
            } else if constexpr (i < kS + 16) {
                constexpr int r = i - kS, ks = r / 8, db = (r / 2) % 4;
                if constexpr (r % 2 == 0) dv_acc[db] = mfma32(pop[ks], a, dv_acc[db]);
                else dk_acc[db] = mfma32(dsop[ks], a, dk_acc[db]);
            } else {
                constexpr int r = i - kS - 16, ks = r / 2, cb = r % 2;
                dk_acc[4 + cb % 2] = mfma32(dsop[ks], a, dk_acc[4 + cb % 2]);
            }
            if constexpr (i > 0 && i + kR < kOps) ring[i % kR] = fetch(std::integral_constant<int, i + kR>{});
        };
        // The scheduler's small-GEMM interleave (LLVM's IGLP strategy 0)
        // issues the operand reads progressively further ahead of their
        // MFMAs (up to 14 in flight) instead of just before each; without
        // it most MFMAs waited on an LDS read (lgkmcnt 0 or 1).  Strategies
        // 1-3 were slower.
        __builtin_amdgcn_iglp_opt(0);
        bw_static_for<kS>(op);
        softmax(sc, dpc, bc, m, mx);
        bw_static_for<kOps - kS>([&](auto ic) { op(std::integral_constant<int, kS + decltype(ic)::value>{}); });
        bw_wait_vmem();
        __syncthreads();
    };
    f32x16_t sa, dpa, sb, dpb, sx, dpx;
    sdp(sa, dpa, C0{});
    for (int t = 0; t < n_iter; t += 3) {
        step(sa, dpa, sb, dpb, t, C0{}, C1{}, C2{});
        step(sb, dpb, sx, dpx, t + 1, C1{}, C2{}, C0{});
        step(sx, dpx, sa, dpa, t + 2, C2{}, C0{}, C1{});
    }

    // dK, dV of this wave's keys: C[key][d], lane (d = 32db + l32, half g2),
    // register 4i + r <-> key 32w + 8i + 4g2 + r.  One workgroup per (key
    // block, head subset): bf16 straight out, or an fp32 partial per subset.
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int j = kv0 + 32 * wave + 8 * i + 4 * g2 + r;
            if (j >= p.skv) continue;
            if (p.dk_part != nullptr) {
                const int64_t row = (((int64_t)hsp * p.batch + b) * p.hkv + kvh) * p.skv + j;
                float* dkr = p.dk_part + row * kDk + l32;
                float* dvr = p.dv_part + row * kHeadDim + l32;
#pragma unroll
                for (int db = 0; db < D::kDb; ++db) dkr[32 * db] = dk_acc[db][4 * i + r];
#pragma unroll
                for (int db = 0; db < 4; ++db) dvr[32 * db] = dv_acc[db][4 * i + r];
            } else {
                __bf16* dkr = p.dk + b * p.dk_sb + (int64_t)j * p.dk_ss + kvh * p.dk_sh + l32;
                __bf16* dvr = p.dv + b * p.dv_sb + (int64_t)j * p.dv_ss + kvh * p.dv_sh + l32;
#pragma unroll
                for (int db = 0; db < D::kDb; ++db) dkr[32 * db] = (__bf16)dk_acc[db][4 * i + r];
#pragma unroll
                for (int db = 0; db < 4; ++db) dvr[32 * db] = (__bf16)dv_acc[db][4 * i + r];
            }
        }
}

// Sum of the n_hsplit fp32 partials -> bf16 dK, dV.  16 lanes per key row:
// lane `part` sums dK elements kDk/16 * part .. (8 or 12) and dV elements
// 8 * part .. +7.
template <int kDk>
__global__ __launch_bounds__(256) void bwd_dkdv_reduce_kernel(BwdParams p) {
    constexpr int kKq = kDk / 64;   // f32x4 of dK per lane (2 or 3)
    const int64_t rows_kv = (int64_t)p.batch * p.hkv * p.skv;
    const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    const int part = threadIdx.x & 15;
    if (row >= rows_kv) return;
    f32x4_t kq[kKq], v0 = {0.f, 0.f, 0.f, 0.f}, v1 = v0;
#pragma unroll
    for (int e = 0; e < kKq; ++e) kq[e] = v0;
    for (int s = 0; s < p.n_hsplit; ++s) {
        const f32x4_t* pk = reinterpret_cast<const f32x4_t*>(p.dk_part + (s * rows_kv + row) * kDk + part * 4 * kKq);
        const f32x4_t* pv = reinterpret_cast<const f32x4_t*>(p.dv_part + (s * rows_kv + row) * kHeadDim + part * 8);
#pragma unroll
        for (int e = 0; e < kKq; ++e) kq[e] += pk[e];
        v0 += pv[0];
        v1 += pv[1];
    }
    const int j = (int)(row % p.skv);
    const int64_t bh = row / p.skv;
    const int kvh = (int)(bh % p.hkv);
    const int b = (int)(bh / p.hkv);
    __bf16* dkr = p.dk + b * p.dk_sb + j * p.dk_ss + kvh * p.dk_sh + part * 4 * kKq;
#pragma unroll
    for (int e = 0; e < kKq; ++e) {
        bf16x4_t w;
#pragma unroll
        for (int x = 0; x < 4; ++x) w[x] = (__bf16)kq[e][x];
        *reinterpret_cast<bf16x4_t*>(dkr + 4 * e) = w;
    }
    bf16x8_t wv;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        wv[e] = (__bf16)v0[e];
        wv[4 + e] = (__bf16)v1[e];
    }
    *reinterpret_cast<bf16x8_t*>(p.dv + b * p.dv_sb + j * p.dv_ss + kvh * p.dv_sh + part * 8) = wv;
}

// ---------------------------------------------------------------- dQ
// Unit = 128 query rows: hb heads of one KV group x (128 / hb) positions,
// wave w -> head (w % hb), positions 32 * (w / hb) .. +31 of the unit, as the
// forward kernel; the whole key range of the unit (the split form,
// dq_unit_pp below, gives each half of it to a group of its own).
template <bool kSwa, int kDk, bool kAddMask>
__device__ __forceinline__ void dq_unit(const BwdParams& p, unsigned char* smem, int qb, int hg, int kvh, int b) {
    using D = BwDims<kDk>;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int l32 = lane & 31;
    const int l16 = lane & 15;
    const int g2 = lane >> 5;
    const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)smem;

    const int qrows = 128 / p.hb;
    const int q_wg0 = qb * qrows;
    const int h = kvh * p.group + hg * p.hb + (wave % p.hb);
    const int q0w = q_wg0 + (wave / p.hb) * 32;
    const int qrow = q0w + l32;

    // Q^T and dO^T as B operands: lane holds row qrow, elements 16kk + 8g2 .. +7;
    // rows >= sq read as zero.
    const uint32_t qss = (uint32_t)(p.q_ss * 2);
    const uint32_t dss = (uint32_t)(p.do_ss * 2);
    const __amdgpu_buffer_rsrc_t qrs =
        make_rsrc(p.q + b * p.q_sb + h * p.q_sh, (uint32_t)(p.sq - 1) * qss + D::kRowBytes);
    const __amdgpu_buffer_rsrc_t drs =
        make_rsrc(p.dout + b * p.do_sb + h * p.do_sh, (uint32_t)(p.sq - 1) * dss + kBwRowBytes);
    const uint32_t oss = (uint32_t)(p.o_ss * 2);
    const __amdgpu_buffer_rsrc_t ors =
        make_rsrc(p.o + b * p.o_sb + h * p.o_sh, (uint32_t)(p.sq - 1) * oss + kBwRowBytes);
    bf16x8_t qop[D::kSteps], doop[8], oop[8];
#pragma unroll
    for (int kk = 0; kk < D::kSteps; ++kk)
        qop[kk] = as_bf16x8(buf_load16(qrs, (uint32_t)qrow * qss + (16 * kk + 8 * g2) * 2));
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
        doop[kk] = as_bf16x8(buf_load16(drs, (uint32_t)qrow * dss + (16 * kk + 8 * g2) * 2));
        oop[kk] = as_bf16x8(buf_load16(ors, (uint32_t)qrow * oss + (16 * kk + 8 * g2) * 2));
    }
    const int64_t rows_q = (int64_t)p.batch * p.hq * p.sq;
    const int64_t ridx = ((int64_t)b * p.hq + h) * p.sq + qrow;
    const float nl = (qrow < p.sq) ? -p.lse[ridx] * kLog2e : 0.f;
    float nd = 0.f;   // set once O has arrived (after the first tile's loads are issued)

    int kv_end = p.skv;
    if (p.causal) kv_end = min(kv_end, min(q_wg0 + qrows, p.sq));
    // a window starts the unit at the tile holding its first row's first key
    const int t_lo = kSwa ? max(0, q_wg0 - p.window + 1) / kDqTile : 0;
    const int unit_tiles = max(0, (kv_end + kDqTile - 1) / kDqTile - t_lo);
    const int n_tiles = unit_tiles;
    const int t_first = t_lo;
    // keys this lane's row may use: below kv_hi (end of the unit's range) and,
    // under the causal mask, at most qrow
    const int kv_hi = min(kv_end, (t_first + n_tiles) * kDqTile);
    const int row_lim = (qrow >= p.sq) ? 0 : min(kv_hi, p.causal ? qrow + 1 : p.skv);

    const uint32_t kss = (uint32_t)(p.k_ss * 2);
    const uint32_t vss = (uint32_t)(p.v_ss * 2);
    const __amdgpu_buffer_rsrc_t krs =
        make_rsrc(p.k + b * p.k_sb + kvh * p.k_sh, (uint32_t)(p.skv - 1) * kss + D::kRowBytes);
    const __amdgpu_buffer_rsrc_t vrs =
        make_rsrc(p.v + b * p.v_sb + kvh * p.v_sh, (uint32_t)(p.skv - 1) * vss + kBwRowBytes);
    // K, V tile j (of the group) into buffer bi: rows r = 4*(wave + 4i) + lane/16;
    // keys >= skv read as zero
    auto issue = [&](int j, int bi) {
        const int t0 = (t_first + j) * kDqTile;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r0 = 4 * (wave + 4 * i);
            const int r = r0 + (lane >> 4);
            const int slot = (l16 ^ bw_swz(r)) << 4;
            bw_dma16(lds_base + bi * kDqTileBytes + r0 * kBwRowBytes, (uint32_t)(t0 + r) * kss + slot, krs);
            bw_dma16(lds_base + (2 + bi) * kDqTileBytes + r0 * kBwRowBytes, (uint32_t)(t0 + r) * vss + slot, vrs);
        }
        if constexpr (D::kHi) {
            // dims 128..191: instruction i fills rows 8(wave + 4i) .. +7, lane l
            // slot l % 8 of row 8(wave + 4i) + l / 8
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int r0 = 8 * (wave + 4 * i);
                const int r = r0 + (lane >> 3);
                const int c = (lane & 7) ^ bw_swz_hi(r);
                bw_dma16(lds_base + kDqKHiOff + bi * kDqKHiTileBytes + r0 * kBwHiRowBytes,
                         (uint32_t)(t0 + r) * kss + kBwRowBytes + 16 * c, krs);
            }
        }
    };

    f32x16_t dq_acc[D::kDb];
#pragma unroll
    for (int db = 0; db < D::kDb; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) dq_acc[db][i] = 0.f;
    int trk[4][2], trk_hi[2][2];
#pragma unroll
    for (int db = 0; db < 4; ++db) {
        trk[db][0] = bw_tr_off(lane, db, 0);
        trk[db][1] = bw_tr_off(lane, db, 1);
    }
    if constexpr (D::kHi) {
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            trk_hi[cb][0] = bw_tr_off_hi(lane, cb, 0);
            trk_hi[cb][1] = bw_tr_off_hi(lane, cb, 1);
        }
    }
    int roff[8], roff_hi[4];
    const int fl = bw_swz(l32);
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) roff[kk] = l32 * kBwRowBytes + (((2 * kk + g2) ^ fl) << 4);
    if constexpr (D::kHi) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
            roff_hi[kk] = l32 * kBwHiRowBytes + (((2 * kk + g2) ^ bw_swz_hi(l32)) << 4);
    }
    const float c2 = p.scale_log2;
    const float scale = p.scale;

    // One tile from buffer BI.  Element (tb, i) of S^T/dP^T is key
    // 32tb + 8(i/4) + 4g2 + i%4 of the tile; it is used when 32tb + 8(i/4) + i%4 < m,
    // m = row_lim - (tile start) - 4g2 (m <= 0 masks the whole tile), and
    // (window) when it is >= lo, lo = qrow - window + 1 - (tile start) - 4g2.
    // kAddMask: as in the dK/dV kernel, S^T's accumulators start at 0, or on
    // a tile the mask cuts for this wave's rows (`cut`, wave-uniform) at
    // ninf for each unused element, and dS^T carries no select.
    const float ninf = c2 > 0.f ? -INFINITY : INFINITY;
    auto tile = [&](auto bi_c, int m, int lo, bool cut) {
        constexpr int bi = decltype(bi_c)::value;
        const unsigned char* kl = smem + bi * kDqTileBytes;
        const unsigned char* vl = smem + (2 + bi) * kDqTileBytes;
        [[maybe_unused]] const unsigned char* khl = smem + kDqKHiOff + bi * kDqKHiTileBytes;
        // S^T = K Q^T, dP^T = V dO^T (C[key][q], lane (q = l32, half g2)), then
        // dQ^T += K^T dS^T, as one stream of operands read kR MFMAs ahead into
        // a ring of registers, with dS^T on the VALU between the two parts
        // (6 ahead at head dim 192; 3 at 128, where a deeper ring spills).
        // Operand i < 32: k-step i / 4, 32-key block (i / 2) % 2, K (i even) or
        // V; then (192-wide) the K rows' 128-byte parts; then per 16-key block
        // kb the transposed K operands of dQ^T's column blocks.
        constexpr int kSd = 32 + (D::kHi ? 8 : 0);
        constexpr int kPer = D::kHi ? 6 : 4;
        constexpr int kOps = kSd + 4 * kPer;
        constexpr int kR = D::kHi ? 6 : 3;
        auto fetch = [&](auto ic) -> bf16x8_t {
            constexpr int i = decltype(ic)::value;
            if constexpr (i < 32) {
                constexpr int kk = i / 4, tb = (i / 2) % 2;
                return *reinterpret_cast<const bf16x8_t*>((i % 2 == 0 ? kl : vl) + tb * 32 * kBwRowBytes + roff[kk]);
            } else if constexpr (i < kSd) {
                constexpr int r = i - 32, kk = r / 2, tb = r % 2;
                return *reinterpret_cast<const bf16x8_t*>(khl + tb * 32 * kBwHiRowBytes + roff_hi[kk % 4]);
            } else {
                constexpr int r = i - kSd, kb = r / kPer, c = r % kPer;
                if constexpr (c < 4) return tr_pair(kl + 16 * kb * kBwRowBytes, trk[c][0], trk[c][1]);
                else return tr_pair(khl + 16 * kb * kBwHiRowBytes, trk_hi[(c - 4) % 2][0], trk_hi[(c - 4) % 2][1]);
            }
        };
        f32x16_t s[2], dp[2];
        bf16x8_t dsop[4];
        bf16x8_t ring[kR];
        bw_static_for<kR>([&](auto ic) { ring[decltype(ic)::value] = fetch(ic); });
#pragma unroll
        for (int tb = 0; tb < 2; ++tb)
#pragma unroll
            for (int i = 0; i < 16; ++i) dp[tb][i] = 0.f;
        if constexpr (kAddMask) {
            // the two S^T chains' first MFMAs (operands 0 and 2) ahead of the
            // scheduled stream, with the mask's start values on a cut tile;
            // their operand slots are refilled as ops 0 and 2 would
            f32x16_t z;
#pragma unroll
            for (int i = 0; i < 16; ++i) z[i] = 0.f;
            if (cut) {
                f32x16_t bias[2];
#pragma unroll
                for (int tb = 0; tb < 2; ++tb)
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int idx = 32 * tb + 8 * (i >> 2) + (i & 3);
                        const bool vis = kSwa ? (idx < m && idx >= lo) : (idx < m);
                        bias[tb][i] = vis ? 0.f : ninf;
                    }
                s[0] = mfma32(ring[0], qop[0], bias[0]);
                s[1] = mfma32(ring[2], qop[0], bias[1]);
            } else {
                s[0] = mfma32(ring[0], qop[0], z);
                s[1] = mfma32(ring[2], qop[0], z);
            }
            ring[0] = fetch(std::integral_constant<int, kR>{});
            ring[2 % kR] = fetch(std::integral_constant<int, 2 + kR>{});
        } else {
#pragma unroll
            for (int tb = 0; tb < 2; ++tb)
#pragma unroll
                for (int i = 0; i < 16; ++i) s[tb][i] = 0.f;
        }
        // ops 0 and 2 with kAddMask: issued above
        auto issued = [](int i) { return kAddMask && (i == 0 || i == 2); };
        auto op = [&](auto ic) {
            constexpr int i = decltype(ic)::value;
            const bf16x8_t a = ring[i % kR];
            if constexpr (issued(i)) {
                (void)a;
            } else if constexpr (i < 32) {
                constexpr int kk = i / 4, tb = (i / 2) % 2;
                if constexpr (i % 2 == 0) s[tb] = mfma32(a, qop[kk], s[tb]);
                else dp[tb] = mfma32(a, doop[kk], dp[tb]);
            } else if constexpr (i < kSd) {
                constexpr int r = i - 32, kk = r / 2, tb = r % 2;
                s[tb] = mfma32(a, qop[8 + kk % 4], s[tb]);
            } else {
                constexpr int r = i - kSd, kb = r / kPer, c = r % kPer;
                if constexpr (c < 4) dq_acc[c] = mfma32(a, dsop[kb], dq_acc[c]);
                else dq_acc[4 + (c - 4) % 2] = mfma32(a, dsop[kb], dq_acc[4 + (c - 4) % 2]);
            }
            if constexpr (!issued(i) && i + kR < kOps) ring[i % kR] = fetch(std::integral_constant<int, i + kR>{});
        };
        __builtin_amdgcn_iglp_opt(0);   // operand reads run ahead, as in the dK/dV step
        bw_static_for<kSd>(op);
        // dS^T = P^T (dP^T - delta) scale as the B operand of dQ^T += K^T dS^T:
        // block kb = 2tb + kh holds registers 8kh .. 8kh+7 of S^T block tb,
        // i.e. keys 16kb + 4g2 + 0..3 and 16kb + 8 + 4g2 + 0..3.
#pragma unroll
        for (int tb = 0; tb < 2; ++tb)
#pragma unroll
            for (int kh = 0; kh < 2; ++kh)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int i = kh * 8 + e;
                    float pv = fast_exp2(__builtin_fmaf(s[tb][i], c2, nl));
                    const int idx = 32 * tb + 8 * (i >> 2) + (i & 3);
                    if constexpr (!kAddMask && kSwa)
                        pv = (idx < m && idx >= lo) ? pv : 0.f;
                    else if constexpr (!kAddMask)
                        pv = (idx < m) ? pv : 0.f;
                    dsop[tb * 2 + kh][e] = (__bf16)(pv * __builtin_fmaf(dp[tb][i], scale, nd));
                }
        bw_static_for<kOps - kSd>([&](auto ic) { op(std::integral_constant<int, kSd + decltype(ic)::value>{}); });
    };

    // Double-buffered K/V, two tiles per trip so that buffer offsets are
    // constants; a trip's second tile past n_tiles is fully masked (m <= 0)
    // and reads a buffer that holds zeros or the previous tile.
    {
        const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
        for (int off = tid * 16; off < dq_smem_bytes<kDk>(); off += kBwThreads * 16)
            *reinterpret_cast<f32x4_t*>(smem + off) = z;
    }
    __syncthreads();
    if (n_tiles > 0) issue(0, 0);
    bw_wait_vmem();
    // the row's statistics, for this kernel's tiles and stored for dK/dV
    nd = (qrow < p.sq) ? -row_delta(oop, doop) * p.scale : 0.f;
    if (qrow < p.sq && g2 == 0) {
        p.rowstat[ridx] = nl;
        p.rowstat[rows_q + ridx] = nd;
    }
    __syncthreads();
    using C0 = std::integral_constant<int, 0>;
    using C1 = std::integral_constant<int, 1>;
    // Does the mask cut an element of tile jj for this wave's rows q0w ..
    // q0w+31 (wave-uniform)?  A tile past n_tiles, keys at or past kv_hi,
    // rows past sq, a key after the first row (causal), or a key before the
    // last row's window.  Every other tile is wholly visible.
    auto tile_cut = [&](int jj) {
        const int t0 = (t_first + jj) * kDqTile;
        bool cut = jj >= n_tiles || t0 + kDqTile > kv_hi || q0w + 31 >= p.sq || (p.causal && t0 + kDqTile - 1 > q0w);
        if constexpr (kSwa) cut = cut || t0 < q0w + 31 - p.window + 1;
        return cut;
    };
    for (int j = 0; j < n_tiles; j += 2) {
        if (j + 1 < n_tiles) issue(j + 1, 1);
        tile(C0{}, row_lim - (t_first + j) * kDqTile - 4 * g2, qrow - p.window + 1 - (t_first + j) * kDqTile - 4 * g2,
             tile_cut(j));
        bw_wait_vmem();
        __syncthreads();
        if (j + 2 < n_tiles) issue(j + 2, 0);
        tile(C1{}, (j + 1 < n_tiles) ? row_lim - (t_first + j + 1) * kDqTile - 4 * g2 : 0,
             qrow - p.window + 1 - (t_first + j + 1) * kDqTile - 4 * g2, tile_cut(j + 1));
        bw_wait_vmem();
        __syncthreads();
    }

    // dQ^T: lane (q = l32, half g2), block db register i <-> d = 32db + 8(i/4) + 4g2 + i%4
    if (qrow < p.sq) {
        __bf16* dst = p.dq + b * p.dq_sb + (int64_t)qrow * p.dq_ss + h * p.dq_sh;
#pragma unroll
        for (int db = 0; db < D::kDb; ++db)
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                bf16x4_t w;
#pragma unroll
                for (int e = 0; e < 4; ++e) w[e] = (__bf16)dq_acc[db][i4 * 4 + e];
                *reinterpret_cast<bf16x4_t*>(dst + db * 32 + i4 * 8 + g2 * 4) = w;
            }
    }
}

// Split dQ unit, ping-pong (head dim 128): dq_unit's unit, with the two halves
// of its key range on two groups of 4 waves that add their dQ through LDS at
// the end (dQ is a plain sum over keys: P comes from the final LSE).  The two waves of a SIMD (one per group)
// alternate an MFMA phase (dQ^T += K(j)^T dS^T(j), then S^T(j+1) = K(j+1) Q^T
// and dP^T(j+1) = V(j+1) dO^T: 48 MFMAs with their LDS reads) and a VALU phase
// (dS^T(j+1) from S^T, dP^T; then the tile loads for the MFMA phase after
// next), group 1 one phase behind group 0, with a workgroup barrier between
// phases.  Each group has its own tiles: K(j) in buffer j % 3 (an MFMA phase
// reads K(j) and K(j+1)), V(j) in buffer j % 2.
constexpr int kDqPpGroupBytes = 5 * kDqTileBytes;       // K[3] | V[2]: 80 KB
constexpr int kDqPpSmemBytes = 2 * kDqPpGroupBytes;     // 160 KB
constexpr int kRing = 3;                                 // operands read ahead (4: no faster)

template <bool kSwa>
__device__ __forceinline__ void dq_unit_pp(const BwdParams& p, unsigned char* smem_all, int qb, int hg, int kvh,
                                           int b) {
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave_wg = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int grp = wave_wg / kBwWaves;
    const int wave = wave_wg % kBwWaves;
    unsigned char* smem = smem_all + grp * kDqPpGroupBytes;
    const int l32 = lane & 31;
    const int l16 = lane & 15;
    const int g2 = lane >> 5;
    const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)smem;

    const int qrows = 128 / p.hb;
    const int q_wg0 = qb * qrows;
    const int h = kvh * p.group + hg * p.hb + (wave % p.hb);
    const int q0w = q_wg0 + (wave / p.hb) * 32;
    const int qrow = q0w + l32;

    const uint32_t qss = (uint32_t)(p.q_ss * 2);
    const uint32_t dss = (uint32_t)(p.do_ss * 2);
    const __amdgpu_buffer_rsrc_t qrs = make_rsrc(p.q + b * p.q_sb + h * p.q_sh, (uint32_t)(p.sq - 1) * qss + kBwRowBytes);
    const __amdgpu_buffer_rsrc_t drs =
        make_rsrc(p.dout + b * p.do_sb + h * p.do_sh, (uint32_t)(p.sq - 1) * dss + kBwRowBytes);
    const uint32_t oss = (uint32_t)(p.o_ss * 2);
    const __amdgpu_buffer_rsrc_t ors = make_rsrc(p.o + b * p.o_sb + h * p.o_sh, (uint32_t)(p.sq - 1) * oss + kBwRowBytes);
    bf16x8_t qop[8], doop[8], oop[8];
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
        qop[kk] = as_bf16x8(buf_load16(qrs, (uint32_t)qrow * qss + (16 * kk + 8 * g2) * 2));
        doop[kk] = as_bf16x8(buf_load16(drs, (uint32_t)qrow * dss + (16 * kk + 8 * g2) * 2));
    }
    if (grp == 0) {
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) oop[kk] = as_bf16x8(buf_load16(ors, (uint32_t)qrow * oss + (16 * kk + 8 * g2) * 2));
    }
    const int64_t rows_q = (int64_t)p.batch * p.hq * p.sq;
    const int64_t ridx = ((int64_t)b * p.hq + h) * p.sq + qrow;
    const float nl = (qrow < p.sq) ? -p.lse[ridx] * kLog2e : 0.f;
    float nd = 0.f;   // set once O has arrived (after the first tiles' loads are issued)
    // The rows' statistics, for this unit's tiles and stored for dK/dV.  Both
    // groups hold the same rows (wave w of each, lane for lane), so group 0
    // alone loads O and computes them, and hands -delta*scale to group 1
    // through group 1's third K buffer, which group 1 first fills in its first
    // VALU phase.
    float* const nd_x = reinterpret_cast<float*>(smem_all + kDqPpGroupBytes + 2 * kDqTileBytes) + wave * kWave + lane;
    auto stats = [&]() {
        if (grp != 0) return;
        nd = (qrow < p.sq) ? -row_delta(oop, doop) * p.scale : 0.f;
        *nd_x = nd;
        if (qrow < p.sq && g2 == 0) {
            p.rowstat[ridx] = nl;
            p.rowstat[rows_q + ridx] = nd;
        }
    };
    // group 1, after the barrier that follows stats(): the value is read and
    // awaited before the buffer's first tile load is issued
    auto stats_in = [&]() {
        if (grp != 1) return;
        nd = *nd_x;
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    };

    int kv_end = p.skv;
    if (p.causal) kv_end = min(kv_end, min(q_wg0 + qrows, p.sq));
    const int t_lo = kSwa ? max(0, q_wg0 - p.window + 1) / kDqTile : 0;
    const int unit_tiles = max(0, (kv_end + kDqTile - 1) / kDqTile - t_lo);
    const int n_tiles = (unit_tiles + 1) / 2;   // the same for both groups
    const int t_first = t_lo + grp * n_tiles;
    const int kv_hi = min(kv_end, (t_first + n_tiles) * kDqTile);
    const int row_lim = (qrow >= p.sq) ? 0 : min(kv_hi, p.causal ? qrow + 1 : p.skv);

    const uint32_t kss = (uint32_t)(p.k_ss * 2);
    const uint32_t vss = (uint32_t)(p.v_ss * 2);
    const __amdgpu_buffer_rsrc_t krs = make_rsrc(p.k + b * p.k_sb + kvh * p.k_sh, (uint32_t)(p.skv - 1) * kss + kBwRowBytes);
    const __amdgpu_buffer_rsrc_t vrs = make_rsrc(p.v + b * p.v_sb + kvh * p.v_sh, (uint32_t)(p.skv - 1) * vss + kBwRowBytes);
    // K(j) -> buffer j % 3, V(j) -> buffer 3 + j % 2; rows r = 4*(wave + 4i) + lane/16
    // (8 load instructions per wave); keys >= skv read as zero
    auto issue = [&](int j) {
        const int t0 = (t_first + j) * kDqTile;
        const uint32_t kb = lds_base + (uint32_t)(j % 3) * kDqTileBytes;
        const uint32_t vb = lds_base + (uint32_t)(3 + (j & 1)) * kDqTileBytes;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r0 = 4 * (wave + 4 * i);
            const int r = r0 + (lane >> 4);
            const int slot = (l16 ^ bw_swz(r)) << 4;
            bw_dma16(kb + r0 * kBwRowBytes, (uint32_t)(t0 + r) * kss + slot, krs);
            bw_dma16(vb + r0 * kBwRowBytes, (uint32_t)(t0 + r) * vss + slot, vrs);
        }
    };

    f32x16_t dq_acc[4];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) dq_acc[db][i] = 0.f;
    int trk[4][2];
#pragma unroll
    for (int db = 0; db < 4; ++db) {
        trk[db][0] = bw_tr_off(lane, db, 0);
        trk[db][1] = bw_tr_off(lane, db, 1);
    }
    int roff[8];
    const int fl = bw_swz(l32);
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) roff[kk] = l32 * kBwRowBytes + (((2 * kk + g2) ^ fl) << 4);
    const float c2 = p.scale_log2;
    const float scale = p.scale;

    if (n_tiles > 0) {
        f32x16_t s[2], dp[2];
        bf16x8_t dsop[4];
        // MFMA phase j: dQ(j) (when kDq) and S^T/dP^T(j+1) (when kSdp; j = -1
        // computes tile 0's).  Operand i of the phase's stream: dQ operand
        // (kb, db) = (i / 4, i % 4) for i < kQ, else S/dP operand r = i - kQ:
        // k-step r / 4, 32-key block (r / 2) % 2, K (r even) or V.  Each is
        // read kRing MFMAs ahead into a ring of kRing registers.
        auto mphase = [&](auto with_dq, auto with_sdp, int j) {
            constexpr bool kDq = decltype(with_dq)::value;
            constexpr bool kSdp = decltype(with_sdp)::value;
            constexpr int kQ = kDq ? 16 : 0;
            constexpr int kOps = kQ + (kSdp ? 32 : 0);
            // buffer offsets as opaque scalars: each per-lane offset then takes
            // one add per phase, the rest are instruction immediates
            uint32_t kco = (uint32_t)(kDq ? j % 3 : 0) * kDqTileBytes;
            uint32_t kno = (uint32_t)(kSdp ? (j + 1) % 3 : 0) * kDqTileBytes;
            uint32_t vno = (uint32_t)(3 + (kSdp ? (j + 1) & 1 : 0)) * kDqTileBytes;
            asm volatile("" : "+s"(kco), "+s"(kno), "+s"(vno));
            const unsigned char* kc = smem + kco;
            const unsigned char* kn = smem + kno;
            const unsigned char* vn = smem + vno;
            auto fetch = [&](auto ic) -> bf16x8_t {
                constexpr int i = decltype(ic)::value;
                if constexpr (i < kQ) {
                    constexpr int kb = i / 4, db = i % 4;
                    return tr_pair(kc + 16 * kb * kBwRowBytes, trk[db][0], trk[db][1]);
                } else {
                    constexpr int r = i - kQ, kk = r / 4, tb = (r / 2) % 2;
                    const unsigned char* base = (r % 2 == 0) ? kn : vn;
                    return *reinterpret_cast<const bf16x8_t*>(base + tb * 32 * kBwRowBytes + roff[kk]);
                }
            };
            bf16x8_t ring[kRing];
            bw_static_for<kRing>([&](auto ic) {
                if constexpr (decltype(ic)::value < kOps) ring[decltype(ic)::value] = fetch(ic);
            });
            if constexpr (kSdp) {
#pragma unroll
                for (int tb = 0; tb < 2; ++tb)
#pragma unroll
                    for (int i = 0; i < 16; ++i) s[tb][i] = dp[tb][i] = 0.f;
            }
            bw_static_for<kOps>([&](auto ic) {
                constexpr int i = decltype(ic)::value;
                const bf16x8_t a = ring[i % kRing];
                if constexpr (i < kQ) {
                    dq_acc[i % 4] = mfma32(a, dsop[i / 4], dq_acc[i % 4]);
                } else {
                    constexpr int r = i - kQ, kk = r / 4, tb = (r / 2) % 2;
                    if constexpr (r % 2 == 0) s[tb] = mfma32(a, qop[kk], s[tb]);
                    else dp[tb] = mfma32(a, doop[kk], dp[tb]);
                }
                if constexpr (i + kRing < kOps) ring[i % kRing] = fetch(std::integral_constant<int, i + kRing>{});
            });
            // DS reads: 2 per dQ operand, 1 per S/dP operand, kRing operands ahead
            if constexpr (kQ > 0) __builtin_amdgcn_sched_group_barrier(0x100, 2 * kRing, 0);
            else __builtin_amdgcn_sched_group_barrier(0x100, kRing, 0);
#pragma unroll
            for (int i = 0; i < kOps; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                if (i + kRing < kQ) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
                else if (i + kRing < kOps) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            __syncthreads();
        };
        // VALU phase after MFMA phase j: dS^T(j+1) as the B operand of
        // dQ^T += K^T dS^T (block kb = 2tb + kh holds registers 8kh .. 8kh+7
        // of S^T block tb); K(j+3), V(j+3) go into the buffers MFMA phase j
        // has finished with, and the loads of the previous VALU phase are
        // awaited at the end.
        auto vphase = [&](int j) {
            __builtin_amdgcn_s_setprio(1);
            const bool more = j + 3 < n_tiles;
            if (more) issue(j + 3);
            const int t0 = (t_first + j + 1) * kDqTile;
            const int m = row_lim - t0 - 4 * g2;
            [[maybe_unused]] const int lo = qrow - p.window + 1 - t0 - 4 * g2;
#pragma unroll
            for (int tb = 0; tb < 2; ++tb)
#pragma unroll
                for (int kh = 0; kh < 2; ++kh)
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const int i = kh * 8 + e;
                        float pv = fast_exp2(__builtin_fmaf(s[tb][i], c2, nl));
                        const int idx = 32 * tb + 8 * (i >> 2) + (i & 3);
                        if constexpr (kSwa)
                            pv = (idx < m && idx >= lo) ? pv : 0.f;
                        else
                            pv = (idx < m) ? pv : 0.f;
                        dsop[tb * 2 + kh][e] = (__bf16)(pv * __builtin_fmaf(dp[tb][i], scale, nd));
                    }
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) asm volatile("" : "+v"(dsop[kb]));
            if (more) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
            else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __builtin_amdgcn_s_setprio(0);
            __syncthreads();
        };

        // tiles 0 and 1 first; tile 0 is awaited now, tile 1 by the end of
        // the first VALU phase (vphase(-1) issues tile 2)
        issue(0);
        if (n_tiles > 1) {
            issue(1);
            asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
        } else {
            bw_wait_vmem();
        }
        stats();
        __syncthreads();
        stats_in();
        // Both groups pass the same number of barriers: group 1 computes
        // S/dP(0) in an extra leading phase, group 0 ends with an empty one.
        if (grp == 0) mphase(std::false_type{}, std::true_type{}, -1);
        else __syncthreads();
        if (grp == 1) mphase(std::false_type{}, std::true_type{}, -1);
        vphase(-1);
        for (int j = 0; j + 1 < n_tiles; ++j) {
            mphase(std::true_type{}, std::true_type{}, j);
            vphase(j);
        }
        mphase(std::true_type{}, std::false_type{}, n_tiles - 1);
        if (grp == 0) __syncthreads();
    } else {
        bw_wait_vmem();
        stats();
    }

    // group 1 hands its dQ^T to group 0 through group 0's (idle) tile
    // buffers: [wave][value][lane] floats
    float* mg = reinterpret_cast<float*>(smem_all) + wave * 64 * kWave + lane;
    if (grp == 1) {
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) mg[(db * 16 + i) * kWave] = dq_acc[db][i];
    }
    __syncthreads();
    if (grp == 1) return;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) dq_acc[db][i] += mg[(db * 16 + i) * kWave];

    // dQ^T: lane (q = l32, half g2), block db register i <-> d = 32db + 8(i/4) + 4g2 + i%4
    if (qrow < p.sq) {
        __bf16* dst = p.dq + b * p.dq_sb + (int64_t)qrow * p.dq_ss + h * p.dq_sh;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                bf16x4_t w;
#pragma unroll
                for (int e = 0; e < 4; ++e) w[e] = (__bf16)dq_acc[db][i4 * 4 + e];
                *reinterpret_cast<bf16x4_t*>(dst + db * 32 + i4 * 8 + g2 * 4) = w;
            }
    }
}

// Block -> unit, ranked heaviest first under the causal mask (the key range
// grows with the query block); the stream (head group, kv head, batch) is the
// fastest index.
__device__ __forceinline__ void dq_block_unit(const BwdParams& p, int* qb, int* hg, int* kvh, int* b) {
    const int stream = blockIdx.x % p.q_streams;
    const int rank = blockIdx.x / p.q_streams;
    *qb = p.causal ? p.n_qunits - 1 - rank : rank;
    *hg = stream % p.n_hgroups;
    *kvh = (stream / p.n_hgroups) % p.hkv;
    *b = stream / (p.n_hgroups * p.hkv);
}

// 128-wide: two workgroups per CU; 192-wide (MLA): one, with the whole
// register file (Q^T of 12 k-steps, dQ^T of 6 column blocks).
template <bool kSwa, int kDk, bool kAddMask>
__global__ __launch_bounds__(kBwThreads, kDk == 128 ? 2 : 1) void bwd_dq_kernel(BwdParams p) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    int qb, hg, kvh, b;
    dq_block_unit(p, &qb, &hg, &kvh, &b);
    dq_unit<kSwa, kDk, kAddMask>(p, smem, qb, hg, kvh, b);
}

template <bool kSwa>
__global__ __launch_bounds__(2 * kBwThreads, 1) void bwd_dq_split_kernel(BwdParams p) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    int qb, hg, kvh, b;
    dq_block_unit(p, &qb, &hg, &kvh, &b);
    dq_unit_pp<kSwa>(p, smem, qb, hg, kvh, b);
}

static_assert(kKvKeys == plan::kBackwardKvKeys, "keys per dK/dV workgroup");

}  // namespace fgqa

using namespace fgqa;

extern "C" int fgqa_prefill_backward_workspace_bytes(const fgqa_prefill_backward_args* a, size_t* bytes) {
    if (bytes == nullptr) return FGQA_ERR_INVALID_ARGUMENT;
    const int st = plan::validate_backward(a);
    if (st != FGQA_OK) return st;
    const int cus = device_cu_count();
    if (cus <= 0) return FGQA_ERR_HIP;
    *bytes = plan::backward_workspace_bytes(a, cus);
    return FGQA_OK;
}

namespace fgqa {
namespace {
int backward_launch(const fgqa_prefill_backward_args* a, hipStream_t s);
int backward_padded_launch(const fgqa_prefill_backward_args* a, hipStream_t s);
}  // namespace
}  // namespace fgqa

extern "C" int fgqa_prefill_backward_bf16(const fgqa_prefill_backward_args* a, void* stream) {
    int st = plan::validate_backward(a);
    if (st != FGQA_OK) return st;
    if (a->batch == 0 || (a->seqlen_q == 0 && a->seqlen_kv == 0)) return FGQA_OK;
    st = plan::validate_backward_pointers(a);
    if (st != FGQA_OK) return st;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    return plan::backward_padded(a) ? backward_padded_launch(a, s) : backward_launch(a, s);
}

namespace fgqa {
namespace {

// Head dims the kernels are not built for (plan::backward_padded): pad Q, K,
// V, O and dO, run the built kernels on the copies, unpad dQ, dK and dV.
// The copies live after the built call's own workspace, in the caller's
// workspace or with none in the library's cached buffer.
int backward_padded_launch(const fgqa_prefill_backward_args* a, hipStream_t s) {
    const int cus = device_cu_count();
    if (cus <= 0) return FGQA_ERR_HIP;
    fgqa_prefill_backward_args pa = plan::backward_padded_args(a);
    const size_t inner = plan::plan_backward(&pa, cus).ws_bytes;
    const plan::BwdPadLayout L = plan::backward_pad_layout(a, inner);
    std::unique_lock<std::mutex> lock;   // held through the launches when the library's buffer is used
    unsigned char* ws = static_cast<unsigned char*>(a->workspace);
    if (ws == nullptr && a->workspace_bytes == 0) {
        lock = workspace_lock();
        int st = FGQA_OK;
        ws = static_cast<unsigned char*>(internal_workspace(L.total, &st));
        if (st != FGQA_OK) return st;
    } else if (ws == nullptr || a->workspace_bytes < L.total) {
        return FGQA_ERR_WORKSPACE;
    } else if ((reinterpret_cast<uintptr_t>(ws) & 255) != 0) {
        return FGQA_ERR_UNSUPPORTED;
    }
    if (inner > 0) {
        pa.workspace = ws;   // the built call's workspace: the first `inner` bytes
        pa.workspace_bytes = inner;
    }
    const int B = a->batch, sq = a->seqlen_q, skv = a->seqlen_kv, hq = a->num_q_heads, hkv = a->num_kv_heads;
    const int dqk = a->head_dim, dv = a->head_dim_v == 0 ? a->head_dim : a->head_dim_v, dk = pa.head_dim;
    pa.q = ws + L.q;
    pa.k = ws + L.k;
    pa.v = ws + L.v;
    pa.o = ws + L.o;
    pa.grad_o = ws + L.dout;
    pa.grad_q = ws + L.dq;
    pa.grad_k = ws + L.dk;
    pa.grad_v = ws + L.dv;
    launch_pad_rows(a->q, a->q_stride, B, sq, hq, dqk, dk, ws + L.q, s);
    launch_pad_rows(a->k, a->k_stride, B, skv, hkv, dqk, dk, ws + L.k, s);
    launch_pad_rows(a->v, a->v_stride, B, skv, hkv, dv, kHeadDim, ws + L.v, s);
    launch_pad_rows(a->o, a->o_stride, B, sq, hq, dv, kHeadDim, ws + L.o, s);
    launch_pad_rows(a->grad_o, a->grad_o_stride, B, sq, hq, dv, kHeadDim, ws + L.dout, s);
    if (hipGetLastError() != hipSuccess) return FGQA_ERR_HIP;
    if (const int st = backward_launch(&pa, s); st != FGQA_OK) return st;
    launch_unpad_rows(ws + L.dq, dk, a->grad_q, a->grad_q_stride, B, sq, hq, dqk, s);
    launch_unpad_rows(ws + L.dk, dk, a->grad_k, a->grad_k_stride, B, skv, hkv, dqk, s);
    launch_unpad_rows(ws + L.dv, kHeadDim, a->grad_v, a->grad_v_stride, B, skv, hkv, dv, s);
    if (hipGetLastError() != hipSuccess) return FGQA_ERR_HIP;
    return FGQA_OK;
}

// The launches of a validated call with built head dims.
int backward_launch(const fgqa_prefill_backward_args* a, hipStream_t s) {
    int st = FGQA_OK;
    const int cus = device_cu_count();
    if (cus <= 0) return FGQA_ERR_HIP;
    const plan::BwdPlan pl = plan::plan_backward(a, cus);
    // (every count below fits the 32-bit fields of BwdParams)
    st = plan::check_backward_grid(a, pl);
    if (st != FGQA_OK) return st;

    // NULL with 0 bytes: the library's buffer; a call that needs no
    // workspace (no query rows and no head split) takes none.
    unsigned char* ws = nullptr;
    std::unique_lock<std::mutex> ws_lock;   // held through the launches when the library's buffer is used
    if (pl.ws_bytes > 0) {
        ws = static_cast<unsigned char*>(a->workspace);
        if (ws == nullptr && a->workspace_bytes == 0) {
            ws_lock = workspace_lock();
            ws = static_cast<unsigned char*>(internal_workspace(pl.ws_bytes, &st));
            if (st != FGQA_OK) return st;
        } else if (ws == nullptr || a->workspace_bytes < pl.ws_bytes) {
            return FGQA_ERR_WORKSPACE;
        } else if ((reinterpret_cast<uintptr_t>(ws) & 255) != 0) {
            return FGQA_ERR_UNSUPPORTED;
        }
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
    p.rowstat = reinterpret_cast<float*>(ws);   // NULL only without query rows: never read then
    p.dk_part = pl.n_hsplit > 1 && ws != nullptr ? reinterpret_cast<float*>(ws + pl.stat_bytes) : nullptr;
    p.dv_part = pl.n_hsplit > 1 && ws != nullptr ? reinterpret_cast<float*>(ws + pl.stat_bytes + pl.part_k_bytes)
                                                  : nullptr;
    p.batch = a->batch;
    p.sq = a->seqlen_q;
    p.skv = a->seqlen_kv;
    p.hq = a->num_q_heads;
    p.hkv = a->num_kv_heads;
    p.group = a->num_q_heads / a->num_kv_heads;
    p.causal = a->causal ? 1 : 0;
    p.window = a->window_size;
    p.n_hsplit = pl.n_hsplit;
    p.hs = p.group / pl.n_hsplit;
    p.n_kvblocks = (int)ceil_div(p.skv, kKvKeys);
    p.kv_streams = pl.n_hsplit * p.hkv * p.batch;
    p.n_qblocks32 = (int)ceil_div(p.sq, kKvRows);
    p.hb = (p.group % 4 == 0) ? 4 : (p.group % 2 == 0) ? 2 : 1;
    p.n_hgroups = p.group / p.hb;
    p.n_qunits = (int)ceil_div(p.sq, 128 / p.hb);
    p.q_streams = p.n_hgroups * p.hkv * p.batch;
    p.scale = a->scale;
    p.scale_log2 = a->scale * kLog2e;

    const int64_t rows_kv = (int64_t)p.batch * p.hkv * p.skv;
    const int64_t kv_units = (int64_t)p.n_kvblocks * p.kv_streams;
    const int64_t q_units = (int64_t)p.n_qunits * p.q_streams;

    // Few dQ units (fewer than 4 per CU): split each unit's key range over two
    // wave groups, as the forward does.  Under a sliding window the units
    // carry about the same number of tiles, so there is nothing to balance and
    // the whole-range kernel is faster.  The caller's dq_kernel field can
    // force either (the 192-wide dQ kernel has no split form: validated).
    const bool swa = p.window > 0;
    const bool mla = a->head_dim == 192;
    const bool dq_split = a->dq_kernel == FGQA_KERNEL_AUTO ? (q_units < 4 * (int64_t)cus && !swa && !mla)
                                                           : a->dq_kernel == FGQA_KERNEL_SPLIT;
    // the dK/dV kernel's mask: additive (-inf on S) unless the scale is 0
    const int am = p.scale_log2 != 0.f ? 1 : 0;
    // kernel table: [swa] of dK/dV ([additive mask] too), dQ, split dQ
    const void* kv_fn[2][2] = {{reinterpret_cast<const void*>(bwd_dkdv_kernel<false, 128, false>),
                                reinterpret_cast<const void*>(bwd_dkdv_kernel<false, 128, true>)},
                               {reinterpret_cast<const void*>(bwd_dkdv_kernel<true, 128, false>),
                                reinterpret_cast<const void*>(bwd_dkdv_kernel<true, 128, true>)}};
    const void* kv192_fn[2] = {reinterpret_cast<const void*>(bwd_dkdv_kernel<false, 192, false>),
                               reinterpret_cast<const void*>(bwd_dkdv_kernel<false, 192, true>)};
    const void* q_fn[2][2] = {{reinterpret_cast<const void*>(bwd_dq_kernel<false, 128, false>),
                               reinterpret_cast<const void*>(bwd_dq_kernel<false, 128, true>)},
                              {reinterpret_cast<const void*>(bwd_dq_kernel<true, 128, false>),
                               reinterpret_cast<const void*>(bwd_dq_kernel<true, 128, true>)}};
    const void* q192_fn[2] = {reinterpret_cast<const void*>(bwd_dq_kernel<false, 192, false>),
                              reinterpret_cast<const void*>(bwd_dq_kernel<false, 192, true>)};
    const void* q2_fn[2] = {reinterpret_cast<const void*>(bwd_dq_split_kernel<false>),
                            reinterpret_cast<const void*>(bwd_dq_split_kernel<true>)};
    // attribute slots 10..17 and 24..29: the backward kernels
    if (mla) {
        if ((st = set_kernel_smem_once(am ? 16 : 26, kv192_fn[am], kv_smem_bytes<192>())) != FGQA_OK) return st;
        if ((st = set_kernel_smem_once(am ? 17 : 29, q192_fn[am], dq_smem_bytes<192>())) != FGQA_OK) return st;
    } else {
        if ((st = set_kernel_smem_once((am ? 10 : 24) + swa, kv_fn[swa][am], kKvSmemBytes)) != FGQA_OK) return st;
        if ((st = set_kernel_smem_once((am ? 12 : 27) + swa, q_fn[swa][am], kDqSmemBytes)) != FGQA_OK) return st;
        if ((st = set_kernel_smem_once(14 + swa, q2_fn[swa], kDqPpSmemBytes)) != FGQA_OK) return st;
    }

    // dQ first: its kernels store each row's statistics, which dK/dV reads.
    // (Without query rows there are no dQ units, and dK/dV reads no row.)
    if (mla) {
        if (q_units > 0 && am)
            hipLaunchKernelGGL((bwd_dq_kernel<false, 192, true>), dim3((unsigned)q_units), dim3(kBwThreads),
                               dq_smem_bytes<192>(), s, p);
        else if (q_units > 0)
            hipLaunchKernelGGL((bwd_dq_kernel<false, 192, false>), dim3((unsigned)q_units), dim3(kBwThreads),
                               dq_smem_bytes<192>(), s, p);
        if (kv_units > 0 && am)
            hipLaunchKernelGGL((bwd_dkdv_kernel<false, 192, true>), dim3((unsigned)kv_units), dim3(kBwThreads),
                               kv_smem_bytes<192>(), s, p);
        else if (kv_units > 0)
            hipLaunchKernelGGL((bwd_dkdv_kernel<false, 192, false>), dim3((unsigned)kv_units), dim3(kBwThreads),
                               kv_smem_bytes<192>(), s, p);
        if (pl.n_hsplit > 1 && rows_kv > 0)
            hipLaunchKernelGGL(bwd_dkdv_reduce_kernel<192>, dim3((unsigned)ceil_div(rows_kv, 16)), dim3(256), 0, s,
                               p);
        if (hipGetLastError() != hipSuccess) return FGQA_ERR_HIP;
        return FGQA_OK;
    }
    if (q_units > 0 && dq_split) {
        if (swa)
            hipLaunchKernelGGL(bwd_dq_split_kernel<true>, dim3((unsigned)q_units), dim3(2 * kBwThreads),
                               kDqPpSmemBytes, s, p);
        else
            hipLaunchKernelGGL(bwd_dq_split_kernel<false>, dim3((unsigned)q_units), dim3(2 * kBwThreads),
                               kDqPpSmemBytes, s, p);
    } else if (q_units > 0) {
        const dim3 g((unsigned)q_units), t(kBwThreads);
        if (swa && am) hipLaunchKernelGGL((bwd_dq_kernel<true, 128, true>), g, t, kDqSmemBytes, s, p);
        else if (swa) hipLaunchKernelGGL((bwd_dq_kernel<true, 128, false>), g, t, kDqSmemBytes, s, p);
        else if (am) hipLaunchKernelGGL((bwd_dq_kernel<false, 128, true>), g, t, kDqSmemBytes, s, p);
        else hipLaunchKernelGGL((bwd_dq_kernel<false, 128, false>), g, t, kDqSmemBytes, s, p);
    }
    if (kv_units > 0) {
        const dim3 g((unsigned)kv_units), t(kBwThreads);
        if (swa && am) hipLaunchKernelGGL((bwd_dkdv_kernel<true, 128, true>), g, t, kKvSmemBytes, s, p);
        else if (swa) hipLaunchKernelGGL((bwd_dkdv_kernel<true, 128, false>), g, t, kKvSmemBytes, s, p);
        else if (am) hipLaunchKernelGGL((bwd_dkdv_kernel<false, 128, true>), g, t, kKvSmemBytes, s, p);
        else hipLaunchKernelGGL((bwd_dkdv_kernel<false, 128, false>), g, t, kKvSmemBytes, s, p);
    }
    if (pl.n_hsplit > 1 && rows_kv > 0)
        hipLaunchKernelGGL(bwd_dkdv_reduce_kernel<128>, dim3((unsigned)ceil_div(rows_kv, 16)), dim3(256), 0, s, p);
    if (hipGetLastError() != hipSuccess) return FGQA_ERR_HIP;
    return FGQA_OK;
}

}  // namespace
}  // namespace fgqa
