// Sparse-index GQA prefill forward for gfx950.
//
// Stands in for the reference's Triton-only flash_sgqa_forward_bf16_kernel
// (src/python/Triton/SparseGQA/flash_sgqa_kernel.py:15-137).  Query row i of
// head h attends the keys listed in idx[b][h / G][i][0 .. nsparse): an entry is
// used when 0 <= j < Skv and, if causal, j <= i (:98-102); a key listed twice
// counts twice.  Same maths as the dense prefill: fp32 scores, online softmax,
// P rounded to bf16 before P.V with the row sum kept from the fp32 P
// (:110-121), O /= rowsum and lse = max + log(rowsum), or O = 0 and
// lse = -inf for a row with no usable entry (:123-125).
//
// One wave owns one work item: a query position, a KV head and up to 16 of
// its query heads, which share the position's index list.  The heads are the
// N dimension of v_mfma_f32_16x16x32_bf16; per 32-entry step:
//   S^T (32 keys x 16 heads) = K_gathered . Q^T     8 MFMAs; K rows are gathered
//                                                    straight into A operands
//   O^T (128 x 16)          += V^T . P^T            8 MFMAs; V rows are gathered
//                                                    into registers, written to
//                                                    the wave's LDS tile and read
//                                                    transposed (ds_read_b64_tr_b16)
// The next step's K and V rows are in flight while a step is computed.  Each
// step reads 16 KB of K/V rows; the MFMA work per step is small, so the kernel
// is bound by how fast the gathers are served (mostly from L2 and the MALL:
// every position gathers rows of the same Skv x 256-byte K/V).
#include <math.h>
#include <stdint.h>

#include "fgqa_device.h"
#include "fgqa_internal.h"

namespace fgqa {

struct SparseParams {
    const __bf16* q;
    const __bf16* k;
    const __bf16* v;
    __bf16* o;
    float* lse;
    const int32_t* idx;
    int64_t q_sb, q_ss, q_sh;
    int64_t k_sb, k_ss, k_sh;
    int64_t v_sb, v_ss, v_sh;
    int64_t o_sb, o_ss, o_sh;
    int64_t i_sb, i_sh, i_ss;   // index list strides: batch, kv head, query row
    int batch, sq, skv, hq, hkv, group, nsparse, causal;
    int n_hg;                   // ceil(group / 16) head groups per position
    int n_steps;                // ceil(nsparse / 32), rounded up to even
    int64_t n_items;            // batch * hkv * sq * n_hg
    float scale_log2;           // |scale| * log2(e)
    uint32_t q_sign;            // 0x80008000 when scale < 0 (Q is negated on load)
};

constexpr int kSpWaves = 4;                  // waves (= work items) per workgroup
constexpr int kSpStep = 32;                  // index entries per step
constexpr int kSpTileBytes = kSpStep * 256;  // one step's V rows in LDS (8 KB per wave)
constexpr float kSpRescaleSlack = 8.f;       // log2 units: P <= 2^8 between rescales

// V tile layout in LDS: 16-byte chunk c (dims 8c .. 8c+7) of row r sits at
// c * 512 + (r ^ 8*(c % 2)) * 16.  A row's chunks are 512 bytes apart; the
// XOR keeps the transposed reads (4 rows x 2 chunks x 2 halves per 16 lanes,
// 8 rows per 32 lanes) and the b128 writes free of bank conflicts.

// Block -> first work item.  Blocks go round-robin over the 8 XCDs; this map
// hands each XCD one contiguous range of items (positions), so the rows its
// L2 holds are the causal prefix of nearby positions.
__device__ __forceinline__ int64_t sp_block_first_item(int64_t nblocks) {
    const int64_t bid = blockIdx.x;
    const int64_t q = nblocks / 8, r = nblocks % 8;
    const int64_t x = bid % 8, j = bid / 8;
    return (x * q + (x < r ? x : r) + j) * kSpWaves;
}

__global__ __launch_bounds__(kSpWaves * kWave, 2) void sparse_prefill_kernel(SparseParams p) {
    __shared__ __attribute__((aligned(16))) unsigned char smem[kSpWaves * kSpTileBytes];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int64_t item = sp_block_first_item(gridDim.x) + wave;
    if (item >= p.n_items) return;   // the kernel has no barrier: a finished wave may leave
    unsigned char* vl = smem + wave * kSpTileBytes;

    // (the divisions run on the VALU: readfirstlane tells the compiler the
    // results are wave-uniform, so buffer descriptors stay in SGPRs)
    int64_t rest = item;
    const int hg = __builtin_amdgcn_readfirstlane((int)(rest % p.n_hg));
    rest /= p.n_hg;
    const int pos = __builtin_amdgcn_readfirstlane((int)(rest % p.sq));
    rest /= p.sq;
    const int kvh = __builtin_amdgcn_readfirstlane((int)(rest % p.hkv));
    const int b = __builtin_amdgcn_readfirstlane((int)(rest / p.hkv));

    const int l16 = lane & 15;
    const int g = lane >> 4;          // 16-lane group
    const int l32 = lane & 31;
    const int h0 = kvh * p.group + hg * 16;
    const int nh = min(16, p.group - hg * 16);   // real heads in this item

    // Q^T as the B operand: lane (head l16, group g) holds dims 32*ks + 8g .. +7.
    bf16x8_t qop[4];
    {
        const __amdgpu_buffer_rsrc_t qrs =
            make_rsrc(p.q + b * p.q_sb + (int64_t)pos * p.q_ss + (int64_t)h0 * p.q_sh,
                      (uint32_t)((int64_t)(nh - 1) * p.q_sh * 2 + 256));
        const uint32_t qoff = (uint32_t)((int64_t)min(l16, nh - 1) * p.q_sh * 2) + g * 16;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            u32x4_t t = buf_load16(qrs, qoff + ks * 64);
            t = (l16 < nh) ? (t ^ p.q_sign) : u32x4_t{0u, 0u, 0u, 0u};
            qop[ks] = as_bf16x8(t);
        }
    }

    // The index list (entries past nsparse read as 0 and are masked below).
    const __amdgpu_buffer_rsrc_t irs =
        make_rsrc(p.idx + b * p.i_sb + kvh * p.i_sh + (int64_t)pos * p.i_ss, (uint32_t)p.nsparse * 4);
    // K/V rows of this (batch, kv head); rows are addressed by 32-bit offsets.
    const uint32_t kss = (uint32_t)(p.k_ss * 2);
    const uint32_t vss = (uint32_t)(p.v_ss * 2);
    // (Skv = 0: empty ranges, every load returns 0 and every entry is masked.
    // The select would otherwise put the descriptors in VGPRs.)
    const uint32_t kv_rows = (uint32_t)p.skv;
    const uint32_t k_bytes = __builtin_amdgcn_readfirstlane(kv_rows ? (kv_rows - 1) * kss + 256 : 0u);
    const uint32_t v_bytes = __builtin_amdgcn_readfirstlane(kv_rows ? (kv_rows - 1) * vss + 256 : 0u);
    const __amdgpu_buffer_rsrc_t krs = make_rsrc(p.k + b * p.k_sb + kvh * p.k_sh, k_bytes);
    const __amdgpu_buffer_rsrc_t vrs = make_rsrc(p.v + b * p.v_sb + kvh * p.v_sh, v_bytes);

    // Entry e of step t: lane l loads entry 32t + l % 32 (lanes 32..63 repeat
    // 0..31).  usable -> its key row, else row 0 (read, then masked).
    auto load_idx = [&](int t) -> int { return (int)__builtin_amdgcn_raw_buffer_load_b32(irs, (uint32_t)(t * kSpStep + l32) * 4, 0, 0); };
    struct StepIdx {
        uint32_t row;    // this lane's entry's key row (0 when unusable)
        uint32_t mask;   // bit e: entry 32t + e is usable
    };
    auto decode_idx = [&](int t, int j) -> StepIdx {
        const bool ok = (t * kSpStep + l32 < p.nsparse) && j >= 0 && j < p.skv && (!p.causal || j <= pos);
        const uint64_t bal = __builtin_amdgcn_ballot_w64(ok);
        return StepIdx{ok ? (uint32_t)j : 0u, (uint32_t)bal};
    };

    // K A operands of one step: tile t (entries 16t .. 16t+15), lane (key l16,
    // group g) holds dims 32*ks + 8g .. +7 of entry 16t + l16's row.
    // V: lane l gathers chunks 2i + l/32 (i = 0..7) of entry l % 32's row.
    bf16x8_t ka[2][4], kb[2][4];
    u32x4_t vreg[8];
    auto issue = [&](const StepIdx& si, bf16x8_t (&kd)[2][4]) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const uint32_t row = (uint32_t)__shfl((int)si.row, 16 * t + l16, kWave);
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) kd[t][ks] = as_bf16x8(buf_load16(krs, row * kss + ks * 64 + g * 16));
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) vreg[i] = buf_load16(vrs, si.row * vss + (2 * i + (lane >> 5)) * 16);
    };
    auto write_v = [&] {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int c = 2 * i + (lane >> 5);
            *reinterpret_cast<u32x4_t*>(vl + c * 512 + ((l32 ^ (8 * (lane >> 5))) << 4)) = vreg[i];
        }
    };
    // Transposed V reads: lane (l16, g) of half kh supplies row 16*kh + 4g + l16/4,
    // dims 16*dt + 4*(l16 % 4) .. +3, i.e. chunk 2dt + (l16/2) % 2, half l16 % 2.
    uint32_t vrd[2];
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
        const int c1 = (l16 >> 1) & 1;
        const int r = 16 * kh + 4 * g + (l16 >> 2);
        vrd[kh] = c1 * 512 + ((r ^ (8 * c1)) << 4) + 8 * (l16 & 1);
    }

    const float c = p.scale_log2;
    float m_run = -INFINITY;   // running max (log2 units) of head l16
    float m_use = 0.f;         // m_run, or 0 while m_run is -inf
    float l_run = 0.f;         // this lane's share of head l16's row sum
    f32x4_t oacc[8];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) oacc[dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // One step on entries 32t .. 32t+31, K operands in kc.  S^T C layout: lane
    // (head l16, group g) register r of tile tt = entry 16tt + 4g + r.
    auto compute = [&](const bf16x8_t (&kc)[2][4], uint32_t mask) {
        f32x4_t s[2];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            s[tt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) s[tt] = mfma16(kc[tt][ks], qop[ks], s[tt]);
        }
        float tmax = -INFINITY;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const bool ok = (mask >> (16 * tt + 4 * g + r)) & 1u;
                s[tt][r] = ok ? s[tt][r] : -INFINITY;
                tmax = fmaxf(tmax, s[tt][r]);
            }
        tmax = half_max(xor_max(tmax, 16)) * c;
        if (__builtin_amdgcn_ballot_w64(tmax > m_run + kSpRescaleSlack) != 0) {
            const float m_new = fmaxf(m_run, tmax);
            const float m_new_use = (m_new == -INFINITY) ? 0.f : m_new;
            const float alpha = fast_exp2(m_use - m_new_use);
            l_run *= alpha;
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) oacc[dt] *= alpha;
            m_run = m_new;
            m_use = m_new_use;
        }
        bf16x8_t pop;
        float psum = 0.f;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float pv = fast_exp2(__builtin_fmaf(s[tt][r], c, -m_use));
                psum += pv;
                pop[tt * 4 + r] = (__bf16)pv;
            }
        l_run += psum;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
            const bf16x4_t lo = lds_read_tr16(reinterpret_cast<const __bf16*>(vl + dt * 1024 + vrd[0]));
            const bf16x4_t hi = lds_read_tr16(reinterpret_cast<const __bf16*>(vl + dt * 1024 + vrd[1]));
            oacc[dt] = mfma16(__builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7), pop, oacc[dt]);
        }
    };

    // Step t's rows are issued during step t - 1; index lists run two steps
    // ahead.  n_steps is even, so the loop alternates the two K register sets
    // without copies; steps past nsparse are fully masked.
    // Each index list is loaded before the rows of the step in front of it, so
    // that waiting for it never waits for those rows.
    StepIdx sc = decode_idx(0, load_idx(0));
    int jn = load_idx(1);
    issue(sc, ka);
    for (int t = 0; t < p.n_steps; t += 2) {
        write_v();
        const StepIdx s1 = decode_idx(t + 1, jn);
        jn = load_idx(t + 2);
        issue(s1, kb);
        compute(ka, sc.mask);

        write_v();
        const StepIdx s2 = decode_idx(t + 2, jn);
        jn = load_idx(t + 3);
        issue(s2, ka);   // past the end on the last trip: masked rows 0, never used
        compute(kb, s1.mask);
        sc = s2;
    }

    // Row sums over the four lane groups; then O and the LSE of head l16.
    l_run = half_sum(xor_sum(l_run, 16));
    if (l16 < nh) {
        const int h = h0 + l16;
        const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
        __bf16* orow = p.o + b * p.o_sb + (int64_t)pos * p.o_ss + (int64_t)h * p.o_sh;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
            bf16x4_t w;
#pragma unroll
            for (int r = 0; r < 4; ++r) w[r] = (__bf16)(oacc[dt][r] * inv);
            *reinterpret_cast<bf16x4_t*>(orow + 16 * dt + 4 * g) = w;
        }
        if (p.lse != nullptr && g == 0)
            p.lse[((int64_t)b * p.hq + h) * p.sq + pos] = l_run > 0.f ? m_run * kLn2 + logf(l_run) : -INFINITY;
    }
}

namespace {

int validate_sparse(const fgqa_sparse_prefill_args* a) {
    if (a == nullptr) return FGQA_ERR_INVALID_ARGUMENT;
    if (a->batch < 0 || a->seqlen_q < 0 || a->seqlen_kv < 0 || a->num_q_heads <= 0 || a->num_kv_heads <= 0 ||
        a->head_dim <= 0 || a->num_sparse_kv < 1)
        return FGQA_ERR_INVALID_ARGUMENT;
    if (a->num_q_heads % a->num_kv_heads != 0) return FGQA_ERR_INVALID_ARGUMENT;
    if (!isfinite(a->scale)) return FGQA_ERR_INVALID_ARGUMENT;
    for (int i = 0; i < 3; ++i)
        if (a->q_stride[i] < 0 || a->k_stride[i] < 0 || a->v_stride[i] < 0 || a->o_stride[i] < 0 ||
            a->idx_stride[i] < 0)
            return FGQA_ERR_INVALID_ARGUMENT;
    if (a->head_dim != kHeadDim) return FGQA_ERR_UNSUPPORTED;
    const int64_t lim = (int64_t)1 << 31;
    if ((int64_t)a->seqlen_kv * a->k_stride[1] * 2 + 256 >= lim ||
        (int64_t)a->seqlen_kv * a->v_stride[1] * 2 + 256 >= lim ||
        (int64_t)a->num_q_heads * a->q_stride[2] * 2 >= lim || (int64_t)a->num_sparse_kv * 4 >= lim)
        return FGQA_ERR_UNSUPPORTED;
    if (a->batch == 0 || a->seqlen_q == 0) return FGQA_OK;
    // (with Skv = 0 no K/V row is read: k and v may be null)
    if (a->q == nullptr || a->o == nullptr || a->kv_indices == nullptr ||
        (a->seqlen_kv > 0 && (a->k == nullptr || a->v == nullptr)))
        return FGQA_ERR_INVALID_ARGUMENT;
    if (!aligned16(a->q) || !aligned16(a->k) || !aligned16(a->v) || !aligned16(a->o) ||
        (reinterpret_cast<uintptr_t>(a->kv_indices) & 3u))
        return FGQA_ERR_UNSUPPORTED;
    for (int i = 0; i < 3; ++i)
        if ((a->q_stride[i] & 7) || (a->k_stride[i] & 7) || (a->v_stride[i] & 7) || (a->o_stride[i] & 3))
            return FGQA_ERR_UNSUPPORTED;
    return FGQA_OK;
}

}  // namespace
}  // namespace fgqa

using namespace fgqa;

extern "C" int fgqa_sparse_prefill_bf16(const fgqa_sparse_prefill_args* a, void* stream) {
    int st = validate_sparse(a);
    if (st != FGQA_OK) return st;
    if (a->batch == 0 || a->seqlen_q == 0) return FGQA_OK;

    SparseParams p;
    p.q = static_cast<const __bf16*>(a->q);
    p.k = static_cast<const __bf16*>(a->k);
    p.v = static_cast<const __bf16*>(a->v);
    p.o = static_cast<__bf16*>(a->o);
    p.lse = a->lse;
    p.idx = a->kv_indices;
    p.q_sb = a->q_stride[0];
    p.q_ss = a->q_stride[1];
    p.q_sh = a->q_stride[2];
    p.k_sb = a->k_stride[0];
    p.k_ss = a->k_stride[1];
    p.k_sh = a->k_stride[2];
    p.v_sb = a->v_stride[0];
    p.v_ss = a->v_stride[1];
    p.v_sh = a->v_stride[2];
    p.o_sb = a->o_stride[0];
    p.o_ss = a->o_stride[1];
    p.o_sh = a->o_stride[2];
    p.i_sb = a->idx_stride[0];
    p.i_sh = a->idx_stride[1];
    p.i_ss = a->idx_stride[2];
    p.batch = a->batch;
    p.sq = a->seqlen_q;
    p.skv = a->seqlen_kv;
    p.hq = a->num_q_heads;
    p.hkv = a->num_kv_heads;
    p.group = a->num_q_heads / a->num_kv_heads;
    p.nsparse = a->num_sparse_kv;
    p.causal = a->causal ? 1 : 0;
    p.n_hg = (int)ceil_div(p.group, 16);
    const int steps = (int)ceil_div(p.nsparse, kSpStep);
    p.n_steps = steps + (steps & 1);
    p.n_items = (int64_t)p.batch * p.hkv * p.sq * p.n_hg;
    p.scale_log2 = fabsf(a->scale) * kLog2e;
    p.q_sign = (a->scale < 0.f) ? 0x80008000u : 0u;

    const int64_t blocks = ceil_div(p.n_items, kSpWaves);
    if (blocks >= ((int64_t)1 << 31)) return FGQA_ERR_UNSUPPORTED;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(sparse_prefill_kernel, dim3((unsigned)blocks), dim3(kSpWaves * kWave), 0, s, p);
    if (hipGetLastError() != hipSuccess) return FGQA_ERR_HIP;
    return FGQA_OK;
}
