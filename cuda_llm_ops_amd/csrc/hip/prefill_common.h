// Definitions shared by the prefill forward translation units: the kernel
// parameter block, the unit numbering and the merge-slot layout of units
// whose KV range runs on two workgroups.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "fgqa_device.h"
#include "../host/fgqa_plan.h"

namespace fgqa {

struct PrefillParams {
    const __bf16* q;
    const __bf16* k;
    const __bf16* v;
    __bf16* o;
    float* lse;
    int64_t q_sb, q_ss, q_sh;
    int64_t k_sb, k_ss, k_sh;
    int64_t v_sb, v_ss, v_sh;
    int64_t o_sb, o_ss, o_sh;
    int batch, sq, skv, hq, hkv, group, causal;
    int hb;          // heads per unit (1, 2 or 4; the 256-row kernels 1, 2, 4 or 8)
    int hb_log2;     // log2(hb)
    int n_hgroups;   // group / hb
    int n_qblocks;   // ceil(sq / (unit rows / hb))
    int n_streams;   // n_hgroups * hkv * batch
    FastDiv div_streams, div_hgroups, div_hkv;   // by n_streams, n_hgroups, hkv
    float scale_log2;   // |scale| * log2(e)
    uint32_t q_sign;    // 0x80008000 when scale < 0 (Q is negated on load), else 0
    int window;         // > 0: sliding window, row i sees keys [i - window + 1, i] (causal)
    const float* sink;  // nullable [Hq]: added to the softmax denominator as sink * exp(-max)
    // 256-row kernels whose unit pairs split a unit over two workgroups: tiles
    // a pair's heavy unit keeps beyond half the pair's tiles on its first
    // workgroup, and the partial-result slots and arrival counters of the
    // split units
    int wide_bias;
    float* wide_part;
    unsigned* wide_ctr;
};

// A segment of a 256-row unit: tiles [lo, hi) of its KV range.  part != null:
// the unit's other tiles run on another workgroup; whichever of the two
// finishes second merges both partial results (slot 0: the segment holding
// the unit's first tiles, slot 1: the other).
struct PfSeg {
    int lo, hi;
    int slot;          // this segment's slot (0 or 1)
    float* part;       // the unit's two slots
    unsigned* ctr;     // the unit's 4 words: arrival counter, XCD of each slot (0 between launches)
};

// f(integral_constant<int, 0>), ..., f(integral_constant<int, N-1>): an
// unrolled loop whose index is a constant expression in the body.
template <int N, int I = 0, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<N, I + 1>(f);
    }
}

constexpr int kPfTile = 64;   // KV tokens per tile
// most split units one launch may hold (two partial slots and 4 counter words each)
constexpr int kPwMaxSplit = 128;
// floats of one partial-result slot (O, running max and sum of every lane of
// the 256-row unit's waves): 8 waves x 66 or 4 waves x 132 floats per lane
constexpr int kPfPartFloats = 2 * 4 * 66 * kWave;
// (the host planner sizes the merge scratch from the same figures)
static_assert(kPwMaxSplit == plan::kPrefillMaxSplit && kPfPartFloats == plan::kPrefillPartFloats,
              "merge scratch layout");
static_assert(4 * sizeof(unsigned) * kPwMaxSplit <= FGQA_PREFILL_WORKSPACE_ZERO_BYTES, "counters");

// Rank -> unit.  Units are ranked heaviest first (the causal KV range grows
// with the query block), so the dispatcher hands long units out before short
// ones (and the persistent kernels can pair long ranks with short).  The
// stream (head group, kv head, batch) is the fastest index: with a multiple of
// 8 streams each stream's blocks share one XCD and its L2 (blocks go
// round-robin over the 8 XCDs).
__device__ __forceinline__ void pf_rank_unit(const PrefillParams& p, int r, int* qb, int* hg, int* kvh, int* b) {
    const int rank_q = fast_div(r, p.div_streams);
    const int stream = r - rank_q * p.n_streams;
    *qb = p.causal ? p.n_qblocks - 1 - rank_q : rank_q;
    const int t = fast_div(stream, p.div_hgroups);   // kv head + hkv * batch
    *hg = stream - t * p.n_hgroups;
    *b = fast_div(t, p.div_hkv);
    *kvh = t - *b * p.hkv;
}

// The kernel's parameters read again from the kernarg segment through a
// pointer the compiler cannot see through, so that a loop over units keeps
// none of them in scalar registers across a unit (they would be spilled and
// reloaded one lane read at a time).
__device__ __forceinline__ PrefillParams pf_params_reread(const PrefillParams& p) {
#if defined(__HIP_DEVICE_COMPILE__)
    (void)p;
    typedef const __attribute__((address_space(4))) PrefillParams* KernargParams;
    KernargParams pp = (KernargParams)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(pp));
    return *pp;
#else
    return p;   // the host pass never runs device code
#endif
}

// Tiles of a unit's KV range (a sliding window starts it at the tile that
// holds its first row's first key).
__device__ __forceinline__ int pf_unit_tiles(const PrefillParams& p, int qb, int qrows) {
    int kv_end = p.skv;
    if (p.causal) kv_end = min(kv_end, min((qb + 1) * qrows, p.sq));
    const int t_lo = p.window > 0 ? max(0, qb * qrows - p.window + 1) / kPfTile : 0;
    return max(0, (kv_end + kPfTile - 1) / kPfTile - t_lo);
}

// The pair of 256-row units block w of a pair grid runs (blocks w and w + 8
// of each 16, one XCD: blocks go round-robin over the 8 XCDs), and its role
// (0: the heavy unit's first tiles; 1: the rest of it, then the light unit).
__device__ __forceinline__ int pf_pair_of_block(int w) { return ((w >> 4) << 3) | (w & 7); }
__device__ __forceinline__ int pf_role_of_block(int w) { return (w >> 3) & 1; }

}  // namespace fgqa
