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
//   S^T (32 keys x 16 heads) = K_gathered . Q^T     8 MFMAs, K from the wave's
//                                                    LDS tile (b128 reads)
//   O^T (128 x 16)          += V^T . P^T            8 MFMAs, V read transposed
//                                                    from its LDS tile
//                                                    (ds_read_b64_tr_b16)
// The next step's K and V rows are in flight while a step is computed.  Each
// step reads 16 KB of K/V rows; the MFMA work per step is small, so the kernel
// is bound by how fast the gathers are served (mostly from L2 and the MALL:
// every position gathers rows of the same Skv x 256-byte K/V).
#include <limits.h>
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
constexpr int kSpKRow = 288;                 // K row stride in LDS (256 + 32 bytes)
constexpr int kSpVRow = 288;                 // V row stride in LDS
constexpr int kSpKBytes = kSpStep * kSpKRow;
constexpr int kSpVBytes = kSpStep * kSpVRow;
constexpr int kSpIdxBytes = kSpStep * 4;
constexpr int kSpWaveBytes = kSpKBytes + kSpVBytes + kSpIdxBytes;   // 17.9 KB of LDS per wave
constexpr float kSpRescaleSlack = 8.f;       // log2 units: P <= 2^8 between rescales

// Gathers are row-contiguous: load instruction i of a step fetches entries
// 4i .. 4i+3, 16 lanes per 256-byte row, so every 16 lanes read two whole
// 128-byte lines (a lane-per-row gather makes the L1 handle one access per
// lane and is several times slower).  The rows then go through the wave's LDS
// tiles to reach the MFMA operand layouts.  A 288-byte row stride (256 + 32)
// keeps every LDS pattern here free of bank conflicts (SQ_LDS_BANK_CONFLICT
// reads 0 for the b128 writes of one row's 16 chunks, the b128 A-operand reads
// of 16 rows at one chunk, and the transposed reads of rows 0..7 x chunks
// {2dt, 2dt + 1} per 32 lanes; a 272-byte stride costs the b128 reads 4
// conflict cycles each).

// Block -> first work item: the last positions first.  Blocks go round-robin
// over the 8 XCDs, so every XCD works through the same positions at the same
// time: each L2 holds rows of the same causal prefix and the XCDs finish
// together.  (Handing each XCD one contiguous range of positions gives the
// XCDs with early positions a prefix that fits their L2 and the others one that
// does not; at S = 32768 the late XCDs then ran 30 % longer per item and the
// launch took 16 % longer.)  Early positions have the fewest usable entries, so
// running them last shortens the tail.
__device__ __forceinline__ int64_t sp_block_first_item(int64_t nblocks) {
    return (nblocks - 1 - (int64_t)blockIdx.x) * kSpWaves;
}

// The value of lane ^ d: DPP quad permutes for d = 1, 2, a bit-mode swizzle
// inside each half-wave for 4 <= d <= 16, the half-wave swap for 32.
__device__ __forceinline__ int sp_xor(int v, int d, int lane) {
    switch (d) {
        case 1: return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
        case 2: return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
        case 4: return __builtin_amdgcn_ds_swizzle(v, (4 << 10) | 0x1F);
        case 8: return __builtin_amdgcn_ds_swizzle(v, (8 << 10) | 0x1F);
        case 16: return __builtin_amdgcn_ds_swizzle(v, (16 << 10) | 0x1F);
        default: {
            const auto r = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
            return (int)(lane < 32 ? r[1] : r[0]);
        }
    }
}

// Ascending bitonic sort of a wave's 512 ints, value 8*lane + r in x[r]:
// distances of 8 values or more pair registers across lanes, smaller ones
// pair registers of a lane.  Deterministic (no atomics).
__device__ __forceinline__ void sp_sort512(int (&x)[8], int lane) {
#pragma unroll
    for (int k = 2; k <= 512; k <<= 1)
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
            if (j >= 8) {
                // value e pairs with e ^ j: same register of lane ^ (j / 8);
                // the block of size k holding e sorts up when (e & k) == 0
                const int d = j >> 3;
                const bool keep_min = ((lane & d) == 0) == ((lane & (k >> 3)) == 0);
#pragma unroll
                for (int r = 0; r < 8; ++r) {
                    const int o = sp_xor(x[r], d, lane);
                    x[r] = keep_min ? min(x[r], o) : max(x[r], o);
                }
            } else {
#pragma unroll
                for (int r = 0; r < 8; ++r) {
                    if (r & j) continue;
                    const bool up = ((8 * lane + r) & k) == 0;
                    const int lo = min(x[r], x[r | j]), hi = max(x[r], x[r | j]);
                    x[r] = up ? lo : hi;
                    x[r | j] = up ? hi : lo;
                }
            }
        }
}

// kSorted: lists of at most 512 entries, taken in ascending key order (see
// the loop below); otherwise in list order, streamed a step ahead.
template <bool kSorted>
__global__ __launch_bounds__(kSpWaves * kWave, 2) void sparse_prefill_kernel(SparseParams p) {
    __shared__ __attribute__((aligned(16))) unsigned char smem[kSpWaves * kSpWaveBytes];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int64_t item = sp_block_first_item(gridDim.x) + wave;
    if (item >= p.n_items) return;   // the kernel has no barrier: a finished wave may leave
    unsigned char* kl = smem + wave * kSpWaveBytes;
    unsigned char* vl = kl + kSpKBytes;
    int* il = reinterpret_cast<int*>(vl + kSpVBytes);

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
    // (Skv = 0: empty ranges, every load returns 0 and every entry is masked.
    // The select would otherwise put the descriptors in VGPRs.)
    const uint32_t kss = (uint32_t)(p.k_ss * 2);
    const uint32_t vss = (uint32_t)(p.v_ss * 2);
    const uint32_t kv_rows = (uint32_t)p.skv;
    const uint32_t k_bytes = __builtin_amdgcn_readfirstlane(kv_rows ? (kv_rows - 1) * kss + 256 : 0u);
    const uint32_t v_bytes = __builtin_amdgcn_readfirstlane(kv_rows ? (kv_rows - 1) * vss + 256 : 0u);
    const __amdgpu_buffer_rsrc_t krs = make_rsrc(p.k + b * p.k_sb + kvh * p.k_sh, k_bytes);
    const __amdgpu_buffer_rsrc_t vrs = make_rsrc(p.v + b * p.v_sb + kvh * p.v_sh, v_bytes);

    // Index lists of steps t and t + 1 (t even): lane l loads entry 32t + l.
    auto load_pair = [&](int t) -> int {
        return (int)__builtin_amdgcn_raw_buffer_load_b32(irs, (uint32_t)(t * kSpStep + lane) * 4, 0, 0);
    };
    // Usable-entry masks of the pair: bit e of the low (high) word = entry
    // 32t + e (32t + 32 + e).  Usable -> its key row, else row 0 (read, then masked).
    auto pair_mask = [&](int t, int j) -> uint64_t {
        const bool ok = (t * kSpStep + lane < p.nsparse) && j >= 0 && j < p.skv && (!p.causal || j <= pos);
        return __builtin_amdgcn_ballot_w64(ok);
    };
    // Leaves the key rows of step t (half = 0) or t + 1 (half = 1) in the index
    // area, stored so that lane l finds the rows of entries 4i + l/16 (i = 0..7)
    // in 8 consecutive words.
    auto post_rows = [&](int j, uint64_t mask, int half) {
        if ((lane >> 5) == half) il[(l32 & 3) * 8 + (l32 >> 2)] = ((mask >> lane) & 1u) ? j : 0;
    };

    // Row gathers of one step: instruction i, lane l -> entry 4i + l/16,
    // 16-byte chunk l % 16, into one of two register sets (two steps in flight).
    struct Rows {
        u32x4_t k[8], v[8];
    };
    Rows ra, rb;
    auto issue = [&](Rows& r) {
        const u32x4_t r0 = *reinterpret_cast<const u32x4_t*>(il + (lane >> 4) * 8);
        const u32x4_t r1 = *reinterpret_cast<const u32x4_t*>(il + (lane >> 4) * 8 + 4);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t row = i < 4 ? r0[i] : r1[i - 4];
            r.k[i] = buf_load16(krs, row * kss + l16 * 16);
            r.v[i] = buf_load16(vrs, row * vss + l16 * 16);
        }
    };
    const int wrow = lane >> 4;   // row within each group of 4 entries
    auto stage = [&](const Rows& r) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            *reinterpret_cast<u32x4_t*>(kl + (4 * i + wrow) * kSpKRow + l16 * 16) = r.k[i];
            *reinterpret_cast<u32x4_t*>(vl + (4 * i + wrow) * kSpVRow + l16 * 16) = r.v[i];
        }
    };
    // A operand (K) of tile tt, k-step ks: lane (key l16, group g) reads dims
    // 32*ks + 8g .. +7 of entry 16tt + l16.
    const unsigned char* krd = kl + l16 * kSpKRow + g * 16;
    // Transposed V reads: lane (l16, g) of half kh supplies entry 16kh + 4g + l16/4,
    // dims 16dt + 4*(l16 % 4) .. +3, i.e. chunk 2dt + (l16/2) % 2, half l16 % 2.
    const unsigned char* vrd = vl + (4 * g + (l16 >> 2)) * kSpVRow + ((l16 >> 1) & 1) * 16 + (l16 & 1) * 8;

    const float c = p.scale_log2;
    float m_run = -INFINITY;   // running max (log2 units) of head l16
    float m_use = 0.f;         // m_run, or 0 while m_run is -inf
    float l_run = 0.f;         // this lane's share of head l16's row sum
    f32x4_t oacc[8];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) oacc[dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // One step on the staged entries.  S^T C layout: lane (head l16, group g)
    // register r of tile tt = entry 16tt + 4g + r.
    auto compute = [&](uint32_t mask) {
        f32x4_t s[2];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            s[tt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const bf16x8_t ka = *reinterpret_cast<const bf16x8_t*>(krd + tt * 16 * kSpKRow + ks * 64);
                s[tt] = mfma16(ka, qop[ks], s[tt]);
            }
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
            const bf16x4_t lo = lds_read_tr16(reinterpret_cast<const __bf16*>(vrd + dt * 32));
            const bf16x4_t hi = lds_read_tr16(reinterpret_cast<const __bf16*>(vrd + 16 * kSpVRow + dt * 32));
            oacc[dt] = mfma16(__builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7), pop, oacc[dt]);
        }
    };

    // Step t: its rows (gathered two steps earlier) are staged into LDS, then
    // step t + 2's rows are gathered into the freed register set while step t
    // is computed.
    if constexpr (kSorted) {
        // The whole list (at most 512 entries) in ascending key order, unusable
        // entries last: every wave walks the keys of its prefix from low to high
        // at about the same pace as the other waves of its XCD, whose lists
        // overlap, so a row one wave fetches is often still in L2 when another
        // needs it (at the reference's shape 634 -> 477 us for pre-sorted lists
        // against list order).  The order of the sum changes by rounding only.
        // Lane l holds sorted entries 8l .. 8l+7; a step's 32 entries are lanes
        // 4t .. 4t+3.  Only steps holding usable entries run.
        int x[8];
        {
            const u32x4_t a0 = buf_load16(irs, (uint32_t)lane * 32);
            const u32x4_t a1 = buf_load16(irs, (uint32_t)lane * 32 + 16);
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                const int jj = (int)(r < 4 ? a0[r] : a1[r - 4]);
                const bool ok = 8 * lane + r < p.nsparse && jj >= 0 && jj < p.skv && (!p.causal || jj <= pos);
                x[r] = ok ? jj : INT_MAX;
            }
        }
        sp_sort512(x, lane);
        int n_valid = 0;
#pragma unroll
        for (int r = 0; r < 8; ++r) n_valid += __builtin_popcountll(__builtin_amdgcn_ballot_w64(x[r] != INT_MAX));
        const int steps = (n_valid + 2 * kSpStep - 1) / (2 * kSpStep) * 2;   // even
        // rows of step t into the index area (lane l then finds the rows of
        // entries 4i + l/16 in 8 consecutive words); unusable entries read row 0
        auto post = [&](int t) {
            if ((lane >> 2) == t) {
                const int q = lane & 3;
#pragma unroll
                for (int r = 0; r < 8; ++r) {
                    const int e = 8 * q + r;
                    il[(e & 3) * 8 + (e >> 2)] = x[r] == INT_MAX ? 0 : x[r];
                }
            }
        };
        auto step_mask = [&](int t) -> uint32_t {
            const int nv = min(max(n_valid - t * kSpStep, 0), kSpStep);
            return nv == kSpStep ? 0xffffffffu : ((1u << nv) - 1u);
        };
        post(0);
        issue(ra);
        post(1);
        issue(rb);
        for (int t = 0; t < steps; t += 2) {
            stage(ra);
            post(t + 2);
            issue(ra);
            compute(step_mask(t));
            stage(rb);
            post(t + 3);
            issue(rb);
            compute(step_mask(t + 1));
        }
    } else {
    // Index lists are loaded a step before their rows are
    // gathered and before the rows in front of them, so waiting for a list never
    // waits for rows.  Steps past nsparse are fully masked (their gathers read
    // row 0 and are never used); n_steps is even, so the two register sets
    // alternate without copies.
    // One index load per loop trip, issued before the rows behind it.
    int j = load_pair(0);
    uint64_t mcur = pair_mask(0, j);
    post_rows(j, mcur, 0);
    issue(ra);
    int jn = load_pair(2);
    post_rows(j, mcur, 1);
    issue(rb);
    for (int t = 0; t < p.n_steps; t += 2) {
        stage(ra);
        const uint64_t mnext = pair_mask(t + 2, jn);
        post_rows(jn, mnext, 0);
        issue(ra);
        compute((uint32_t)mcur);

        stage(rb);
        j = jn;
        jn = load_pair(t + 4);
        post_rows(j, mnext, 1);
        issue(rb);
        compute((uint32_t)(mcur >> 32));
        mcur = mnext;
    }
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

static_assert(kSpWaves == plan::kSparseWaves, "waves per sparse workgroup");

}  // namespace fgqa

using namespace fgqa;

extern "C" int fgqa_sparse_prefill_bf16(const fgqa_sparse_prefill_args* a, void* stream) {
    int st = plan::validate_sparse(a);
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
    // lists of at most 512 entries are taken in key order
    if (p.nsparse <= 512)
        hipLaunchKernelGGL(sparse_prefill_kernel<true>, dim3((unsigned)blocks), dim3(kSpWaves * kWave), 0, s, p);
    else
        hipLaunchKernelGGL(sparse_prefill_kernel<false>, dim3((unsigned)blocks), dim3(kSpWaves * kWave), 0, s, p);
    if (hipGetLastError() != hipSuccess) return FGQA_ERR_HIP;
    return FGQA_OK;
}
