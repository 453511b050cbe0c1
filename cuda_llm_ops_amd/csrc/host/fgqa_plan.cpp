// Host-only argument validation and launch planning of the flash-GQA C ABI
// (see fgqa_plan.h).  Every product of caller-supplied sizes is formed in
// 128-bit arithmetic, so no shape, however large, overflows before it is
// compared with the limit it must stay under.
#include "fgqa_plan.h"

#include <math.h>

namespace fgqa {
namespace plan {

namespace {

typedef __int128 i128;

constexpr int64_t kLim31 = (int64_t)1 << 31;
// largest workspace the planners describe (larger shapes are unsupported)
constexpr i128 kMaxWorkspace = (i128)1 << 46;

// The byte span of `rows` bf16 rows `stride` elements apart reaches 2^31 (the
// kernels address one sequence of a tensor through 32-bit buffer offsets).
bool span_reaches_2g(int64_t rows, int64_t stride) { return (i128)rows * stride * 2 >= kLim31; }

size_t round256(i128 x) { return (size_t)((x + 255) / 256 * 256); }

// The element offset of a tensor's last row, the sum of (n_i - 1) * s_i over
// its dimensions, stays below 2^60: the kernels form element offsets in
// 64-bit integers.  (Strides are checked non-negative first.)
template <int K>
bool extent_ok(const int64_t (&n)[K], const int64_t* s) {
    i128 off = 0;
    for (int i = 0; i < K; ++i) off += (i128)(n[i] > 0 ? n[i] - 1 : 0) * s[i];
    return off < ((i128)1 << 60);
}

}  // namespace

// ---------------------------------------------------------------- decode

int validate_decode(const fgqa_decode_args* a) {
    if (a == nullptr) return FGQA_ERR_INVALID_ARGUMENT;
    if (a->batch < 0 || a->max_seqlen < 0 || a->num_q_heads <= 0 || a->num_kv_heads <= 0 || a->head_dim <= 0)
        return FGQA_ERR_INVALID_ARGUMENT;
    if (a->num_q_heads % a->num_kv_heads != 0) return FGQA_ERR_INVALID_ARGUMENT;
    if (!isfinite(a->scale)) return FGQA_ERR_INVALID_ARGUMENT;
    if (a->split_tokens < 0) return FGQA_ERR_INVALID_ARGUMENT;
    for (int i = 0; i < 2; ++i)
        if (a->q_stride[i] < 0 || a->o_stride[i] < 0) return FGQA_ERR_INVALID_ARGUMENT;
    for (int i = 0; i < 3; ++i)
        if (a->k_stride[i] < 0 || a->v_stride[i] < 0) return FGQA_ERR_INVALID_ARGUMENT;
    if (a->head_dim != kHeadDim) return FGQA_ERR_UNSUPPORTED;
    if (a->num_q_heads / a->num_kv_heads > 16) return FGQA_ERR_UNSUPPORTED;
    if (a->max_seqlen > kMaxTokens) return FGQA_ERR_UNSUPPORTED;
    const int64_t qn[2] = {a->batch, a->num_q_heads};
    const int64_t kn[3] = {a->batch, a->max_seqlen, a->num_kv_heads};
    if (!extent_ok(qn, a->q_stride) || !extent_ok(qn, a->o_stride) || !extent_ok(kn, a->k_stride) ||
        !extent_ok(kn, a->v_stride))
        return FGQA_ERR_UNSUPPORTED;
    // 32-bit buffer offsets: the furthest byte addressed inside one sequence
    if (span_reaches_2g((int64_t)a->max_seqlen + 64, a->k_stride[1]) ||
        span_reaches_2g((int64_t)a->max_seqlen + 64, a->v_stride[1]))
        return FGQA_ERR_UNSUPPORTED;
    return FGQA_OK;
}

int validate_decode_pointers(const fgqa_decode_args* a) {
    if (a->batch == 0) return FGQA_OK;
    if (a->q == nullptr || a->k == nullptr || a->v == nullptr || a->o == nullptr) return FGQA_ERR_INVALID_ARGUMENT;
    if (!aligned16(a->q) || !aligned16(a->k) || !aligned16(a->v) || !aligned16(a->o)) return FGQA_ERR_UNSUPPORTED;
    for (int i = 0; i < 2; ++i)
        if ((a->q_stride[i] & 7) || (a->o_stride[i] & 7)) return FGQA_ERR_UNSUPPORTED;
    for (int i = 0; i < 3; ++i)
        if ((a->k_stride[i] & 7) || (a->v_stride[i] & 7)) return FGQA_ERR_UNSUPPORTED;
    return FGQA_OK;
}

DecodeShape decode_shape(const fgqa_decode_args* a) {
    return DecodeShape{a->batch, a->max_seqlen, a->num_q_heads, a->num_kv_heads, a->split_tokens,
                       a->seqlens != nullptr};
}

// Ragged batches get a work list of their non-empty splits (built on the
// device from the lengths), so no workgroup is spent on padding.
static bool list_batch(const DecodeShape& a) { return a.ragged && a.batch < (1 << 15); }

bool decode_needs_cus(const DecodeShape& a) { return a.split_tokens == 0 && !list_batch(a); }

int plan_decode(const DecodeShape& a, int cus, DecodePlan* plan) {
    const int64_t S = a.max_seqlen > 0 ? a.max_seqlen : 1;
    plan->list = list_batch(a);
    int64_t chunk;
    if (a.split_tokens > 0) {
        chunk = ceil_div(a.split_tokens, kDecodeStepRound) * kDecodeStepRound;
    } else if (plan->list) {
        chunk = kDecodeRaggedChunk;
    } else {
        // The KV stream is HBM-bound: a split only pays when there are too
        // few (batch, kv head) streams to occupy every CU, or when sequences
        // are long enough that one workgroup per stream would leave a long
        // tail.  Splits cost a partial write/read and a combine pass.
        if (cus <= 0) return FGQA_ERR_HIP;
        const int64_t items = (int64_t)(a.batch > 0 ? a.batch : 1) * a.num_kv_heads;
        int64_t want = (items >= cus) ? 1 : ceil_div(4LL * cus, items);
        const int64_t max_splits = ceil_div(S, kDecodeStepRound);
        if (want > max_splits) want = max_splits;
        if (want < 1) want = 1;
        chunk = ceil_div(ceil_div(S, want), kDecodeStepRound) * kDecodeStepRound;
        if (chunk > kDecodeMaxAutoChunk) chunk = kDecodeMaxAutoChunk;
    }
    if (chunk < kDecodeStepRound) chunk = kDecodeStepRound;
    if (chunk > S) chunk = ceil_div(S, kDecodeStepRound) * kDecodeStepRound;
    plan->chunk = (int)chunk;
    plan->nsplit = (int)ceil_div(S, chunk);
    if (plan->nsplit >= (1 << 16)) plan->list = false;
    const i128 slots = (i128)a.batch * a.num_q_heads * plan->nsplit;
    i128 part_o = 0, part_ml = 0;
    if (plan->nsplit > 1) {
        part_o = slots * kHeadDim * 4;
        part_ml = slots * 2 * 4;
    }
    const i128 list = plan->list ? (1 + (i128)a.batch * plan->nsplit) * 4 : 0;
    if (part_o + part_ml + list > kMaxWorkspace) return FGQA_ERR_UNSUPPORTED;
    plan->part_o_bytes = round256(part_o);
    plan->part_ml_bytes = round256(part_ml);
    plan->ws_bytes = plan->part_o_bytes + plan->part_ml_bytes + (size_t)list;
    return FGQA_OK;
}

int validate_paged(const fgqa_decode_paged_args* a) {
    if (a == nullptr) return FGQA_ERR_INVALID_ARGUMENT;
    if (a->batch < 0 || a->max_seqlen < 0 || a->num_q_heads <= 0 || a->num_kv_heads <= 0 || a->head_dim <= 0 ||
        a->page_size <= 0 || a->num_pages < 0 || a->block_table_stride < 0)
        return FGQA_ERR_INVALID_ARGUMENT;
    if (a->num_q_heads % a->num_kv_heads != 0) return FGQA_ERR_INVALID_ARGUMENT;
    if (!isfinite(a->scale) || !isfinite(a->k_scale) || !isfinite(a->v_scale)) return FGQA_ERR_INVALID_ARGUMENT;
    if (a->split_tokens < 0) return FGQA_ERR_INVALID_ARGUMENT;
    if (a->kv_dtype != FGQA_KV_BF16 && a->kv_dtype != FGQA_KV_FP8_E4M3) return FGQA_ERR_INVALID_ARGUMENT;
    if ((a->page_size & (a->page_size - 1)) != 0 || a->page_size > (1 << 20)) return FGQA_ERR_UNSUPPORTED;
    // the block table row covers max_seqlen tokens
    if ((i128)a->max_seqlen > (i128)a->block_table_stride * a->page_size) return FGQA_ERR_INVALID_ARGUMENT;
    for (int i = 0; i < 2; ++i)
        if (a->q_stride[i] < 0 || a->o_stride[i] < 0) return FGQA_ERR_INVALID_ARGUMENT;
    for (int i = 0; i < 3; ++i)
        if (a->k_stride[i] < 0 || a->v_stride[i] < 0) return FGQA_ERR_INVALID_ARGUMENT;
    if (a->head_dim != kHeadDim) return FGQA_ERR_UNSUPPORTED;
    if (a->num_q_heads / a->num_kv_heads > 16) return FGQA_ERR_UNSUPPORTED;
    if (a->max_seqlen > kMaxTokens) return FGQA_ERR_UNSUPPORTED;
    const int64_t qn[2] = {a->batch, a->num_q_heads};
    const int64_t cn[3] = {a->num_pages, a->page_size, a->num_kv_heads};
    const int64_t bn[1] = {a->batch};
    if (!extent_ok(qn, a->q_stride) || !extent_ok(qn, a->o_stride) || !extent_ok(cn, a->k_stride) ||
        !extent_ok(cn, a->v_stride) || !extent_ok(bn, &a->block_table_stride))
        return FGQA_ERR_UNSUPPORTED;
    return FGQA_OK;
}

int validate_paged_pointers(const fgqa_decode_paged_args* a) {
    if (a->batch == 0) return FGQA_OK;
    if (a->q == nullptr || a->o == nullptr || a->seqlens == nullptr || a->block_table == nullptr)
        return FGQA_ERR_INVALID_ARGUMENT;
    if (a->max_seqlen > 0 && (a->k_cache == nullptr || a->v_cache == nullptr || a->num_pages == 0))
        return FGQA_ERR_INVALID_ARGUMENT;
    if (!aligned16(a->q) || !aligned16(a->o) || !aligned16(a->k_cache) || !aligned16(a->v_cache))
        return FGQA_ERR_UNSUPPORTED;
    for (int i = 0; i < 2; ++i)
        if ((a->q_stride[i] & 7) || (a->o_stride[i] & 7)) return FGQA_ERR_UNSUPPORTED;
    // 16-byte aligned rows: strides in elements of the cache type
    const int64_t m = (a->kv_dtype == FGQA_KV_FP8_E4M3) ? 15 : 7;
    for (int i = 0; i < 3; ++i)
        if ((a->k_stride[i] & m) || (a->v_stride[i] & m)) return FGQA_ERR_UNSUPPORTED;
    return FGQA_OK;
}

int plan_paged(const fgqa_decode_paged_args* a, DecodePlan* plan) {
    const DecodeShape shape{a->batch, a->max_seqlen, a->num_q_heads, a->num_kv_heads, a->split_tokens, true};
    if (!list_batch(shape)) return FGQA_ERR_UNSUPPORTED;
    const int st = plan_decode(shape, 0, plan);
    if (st != FGQA_OK) return st;
    return plan->list ? FGQA_OK : FGQA_ERR_UNSUPPORTED;
}

// ---------------------------------------------------------------- prefill

namespace {
int head_dim_v_of(const fgqa_prefill_args* a) { return a->head_dim_v == 0 ? a->head_dim : a->head_dim_v; }
// the pairs the kernels are built for: Q/K 128, 192 or 256, V/O 128
bool native_head_dims(int dqk, int dv) { return dv == kHeadDim && (dqk == kHeadDim || dqk == 192 || dqk == 256); }
}  // namespace

bool prefill_padded(const fgqa_prefill_args* a) {
    const int dv = head_dim_v_of(a);
    return a->head_dim > 0 && dv > 0 && a->head_dim <= 256 && dv <= 256 && !native_head_dims(a->head_dim, dv);
}

int padded_dk(const fgqa_prefill_args* a) {
    return a->head_dim <= kHeadDim ? kHeadDim : a->head_dim == 192 ? 192 : 256;
}

int padded_dv(const fgqa_prefill_args* a) { return head_dim_v_of(a) <= kHeadDim ? kHeadDim : 2 * kHeadDim; }

fgqa_prefill_args padded_args(const fgqa_prefill_args* a) {
    fgqa_prefill_args p = *a;
    const int dk = padded_dk(a), dv = padded_dv(a);
    p.head_dim = dk;
    p.head_dim_v = kHeadDim;
    const int64_t qs[3] = {(int64_t)a->seqlen_q * a->num_q_heads * dk, (int64_t)a->num_q_heads * dk, dk};
    const int64_t os[3] = {(int64_t)a->seqlen_q * a->num_q_heads * dv, (int64_t)a->num_q_heads * dv, dv};
    const int64_t ks[3] = {(int64_t)a->seqlen_kv * a->num_kv_heads * dk, (int64_t)a->num_kv_heads * dk, dk};
    const int64_t vs[3] = {(int64_t)a->seqlen_kv * a->num_kv_heads * dv, (int64_t)a->num_kv_heads * dv, dv};
    for (int i = 0; i < 3; ++i) {
        p.q_stride[i] = qs[i];
        p.o_stride[i] = os[i];
        p.k_stride[i] = ks[i];
        p.v_stride[i] = vs[i];
    }
    p.q = p.k = p.v = p.o = nullptr;
    p.workspace = nullptr;
    p.workspace_bytes = 0;
    return p;
}

PadLayout pad_layout(const fgqa_prefill_args* a, size_t merge_bytes) {
    const int dk = padded_dk(a), dv = padded_dv(a);
    const i128 rq = (i128)a->batch * a->seqlen_q * a->num_q_heads * 2;
    const i128 rk = (i128)a->batch * a->seqlen_kv * a->num_kv_heads * 2;
    PadLayout L;
    // the copies never touch the zeroed counter prefix, which later calls
    // on the same workspace count on even when this one merges nothing
    L.q = round256(merge_bytes > kPrefillZeroBytes ? merge_bytes : kPrefillZeroBytes);
    L.k = L.q + round256(rq * dk);
    L.v = L.k + round256(rk * dk);
    L.o = L.v + round256(rk * dv);
    L.total = L.o + round256(rq * dv);
    return L;
}

int validate_prefill(const fgqa_prefill_args* a) {
    if (a == nullptr) return FGQA_ERR_INVALID_ARGUMENT;
    if (a->batch < 0 || a->seqlen_q < 0 || a->seqlen_kv < 0 || a->num_q_heads <= 0 || a->num_kv_heads <= 0 ||
        a->head_dim <= 0)
        return FGQA_ERR_INVALID_ARGUMENT;
    if (a->num_q_heads % a->num_kv_heads != 0) return FGQA_ERR_INVALID_ARGUMENT;
    if (!isfinite(a->scale)) return FGQA_ERR_INVALID_ARGUMENT;
    // a sliding window is a causal window (flash_swa_kernel.py: kv <= q)
    if (a->window_size < 0 || (a->window_size > 0 && !a->causal)) return FGQA_ERR_INVALID_ARGUMENT;
    for (int i = 0; i < 3; ++i)
        if (a->q_stride[i] < 0 || a->k_stride[i] < 0 || a->v_stride[i] < 0 || a->o_stride[i] < 0)
            return FGQA_ERR_INVALID_ARGUMENT;
    if (a->head_dim_v < 0) return FGQA_ERR_INVALID_ARGUMENT;
    const int dv = head_dim_v_of(a);
    // (128, 128), the MLA shape (192, 128) and (256, 128); any other pair up
    // to 256 runs on zero-padded copies; the 192 kernels have no window /
    // sink form
    const bool padded = prefill_padded(a);
    if (!padded && !native_head_dims(a->head_dim, dv)) return FGQA_ERR_UNSUPPORTED;
    const int dk_run = padded ? padded_dk(a) : a->head_dim;
    if (dk_run == 192 && (a->window_size > 0 || a->sink != nullptr)) return FGQA_ERR_UNSUPPORTED;
    if (a->kernel < FGQA_KERNEL_AUTO || a->kernel > FGQA_KERNEL_TALL) return FGQA_ERR_INVALID_ARGUMENT;
    // the window / sink variant has no split form
    if (a->kernel == FGQA_KERNEL_SPLIT && (a->window_size > 0 || a->sink != nullptr)) return FGQA_ERR_UNSUPPORTED;
    // the tall kernel: head dim 128 (or padded to it), no window or sink
    if (a->kernel == FGQA_KERNEL_TALL && (dk_run != kHeadDim || a->window_size > 0 || a->sink != nullptr))
        return FGQA_ERR_UNSUPPORTED;
    // Q/K head dim 256: the whole-range kernel only
    if (dk_run == 256 && a->kernel != FGQA_KERNEL_AUTO && a->kernel != FGQA_KERNEL_WHOLE) return FGQA_ERR_UNSUPPORTED;
    if (a->seqlen_q > kMaxTokens || a->seqlen_kv > kMaxTokens) return FGQA_ERR_UNSUPPORTED;
    if (span_reaches_2g((int64_t)a->seqlen_q + 128, a->q_stride[1]) ||
        span_reaches_2g((int64_t)a->seqlen_kv + 128, a->k_stride[1]) ||
        span_reaches_2g((int64_t)a->seqlen_kv + 128, a->v_stride[1]))
        return FGQA_ERR_UNSUPPORTED;
    {
        const int64_t qn[3] = {a->batch, a->seqlen_q, a->num_q_heads};
        const int64_t kn[3] = {a->batch, a->seqlen_kv, a->num_kv_heads};
        if (!extent_ok(qn, a->q_stride) || !extent_ok(qn, a->o_stride) || !extent_ok(kn, a->k_stride) ||
            !extent_ok(kn, a->v_stride))
            return FGQA_ERR_UNSUPPORTED;
    }
    // unit indices are 32-bit: (query blocks of 32 rows) x heads x batch
    if ((i128)ceil_div(a->seqlen_q, 32) * a->num_q_heads * a->batch >= kLim31) return FGQA_ERR_UNSUPPORTED;
    if (padded) {
        // the copies must pass as a (128, 128) call themselves, and the
        // workspace that holds them stays within the planners' limit
        fgqa_prefill_args p = padded_args(a);
        const uintptr_t dummy = 256;   // validation only: aligned, non-null
        p.q = p.k = p.v = reinterpret_cast<const void*>(dummy);
        p.o = reinterpret_cast<void*>(dummy);
        if (const int st = validate_prefill(&p); st != FGQA_OK) return st;
        if ((i128)pad_layout(a, merge_scratch_bytes_for(kPrefillMaxSplit)).total >= kMaxWorkspace)
            return FGQA_ERR_UNSUPPORTED;
    }
    if (a->batch == 0 || a->seqlen_q == 0) return FGQA_OK;
    if (a->q == nullptr || a->k == nullptr || a->v == nullptr || a->o == nullptr) return FGQA_ERR_INVALID_ARGUMENT;
    // the copies are made with 2-byte accesses: any alignment and strides
    if (padded) return FGQA_OK;
    if (!aligned16(a->q) || !aligned16(a->k) || !aligned16(a->v) || !aligned16(a->o)) return FGQA_ERR_UNSUPPORTED;
    // (O rows go out as 16-byte stores, so O's strides need 8 elements too)
    for (int i = 0; i < 3; ++i)
        if ((a->q_stride[i] & 7) || (a->k_stride[i] & 7) || (a->v_stride[i] & 7) || (a->o_stride[i] & 7))
            return FGQA_ERR_UNSUPPORTED;
    return FGQA_OK;
}

int64_t wide_pairs(const fgqa_prefill_args* a) {
    const int group = a->num_q_heads / a->num_kv_heads;
    const int hbw = group % 8 == 0 ? 8 : group % 4 == 0 ? 4 : group % 2 == 0 ? 2 : 1;
    const int64_t units = ceil_div(a->seqlen_q, 256 / hbw) * (int64_t)(group / hbw) * a->num_kv_heads * a->batch;
    return (units + 1) / 2;
}

bool wide_on_pairs(const fgqa_prefill_args* a, int cus) {
    const int64_t pairs = wide_pairs(a);
    return pairs <= kPrefillMaxSplit && 2 * pairs <= cus;
}

bool tall_on_pairs(const fgqa_prefill_args* a, int cus) { return a->causal && wide_on_pairs(a, cus); }

// The caller's `kernel`, or for AUTO the choice by grid size:
//  - wide: causal, no window or sink, and the wide kernel's unit pairs fill
//    the CUs (two workgroups per pair, within 1/8 of one per CU).  Forced, it
//    also runs the window / sink form;
//  - split: fewer than 4 of the 128-row units per CU, no window or sink: each
//    unit's KV range runs on two wave groups, so a CU never runs a long unit
//    with one wave per SIMD, and each CU gets a share of the units whose tile
//    counts add up evenly;
//  - wide again for the causal grids left (at least 2 of the 128-row units
//    per CU), as whole 256-row units on a persistent grid;
//  - whole: the rest (a sliding window gives every unit about the same number
//    of tiles: nothing to balance).
// The tall kernel runs only when forced.
int prefill_choice(const fgqa_prefill_args* a, int cus) {
    if (a->kernel != FGQA_KERNEL_AUTO) return a->kernel;
    if (a->head_dim == 256) return FGQA_KERNEL_WHOLE;
    const int group = a->num_q_heads / a->num_kv_heads;
    const int hb = group % 4 == 0 ? 4 : group % 2 == 0 ? 2 : 1;
    const bool win = a->window_size > 0;
    const bool swa = win || a->sink != nullptr;
    const int64_t units = ceil_div(a->seqlen_q, 128 / hb) * (int64_t)(group / hb) * a->num_kv_heads * a->batch;
    const int64_t pairs = wide_pairs(a);
    const int64_t wide_grid = 16 * ceil_div(pairs, 8);
    if (!swa && a->causal && pairs <= kPrefillMaxSplit && wide_grid <= cus && 8 * wide_grid >= 7 * (int64_t)cus)
        return FGQA_KERNEL_WIDE;
    if (!swa && a->causal) return units < 2 * (int64_t)cus ? FGQA_KERNEL_SPLIT : FGQA_KERNEL_WIDE;
    // A window of at least 1536 keys (24 tiles per unit), or a sink without a
    // window over a grid of a 128-row unit per CU: the 256-row kernels'
    // shared tiles pay for their fewer, longer units.  Measured on four
    // shapes (S = 4096 to 16384, Hkv 1 and 8): windows of 1536-3072 keys 3-8 %
    // faster than the whole-range kernel (at 512-1024 keys its two workgroups
    // per CU win or tie); a sink alone 4-20 % faster (config 4's shape: 87.5
    // against 70.1 us).
    if (swa && a->causal && (win ? a->window_size >= 1536 : units >= (int64_t)cus)) return FGQA_KERNEL_WIDE;
    if (units < 4 * (int64_t)cus && !swa) return FGQA_KERNEL_SPLIT;
    return FGQA_KERNEL_WHOLE;
}

size_t prefill_workspace_bytes(const fgqa_prefill_args* a, int cus) {
    if (!prefill_padded(a)) return merge_scratch_bytes(a, prefill_choice(a, cus), cus);
    const fgqa_prefill_args p = padded_args(a);
    return pad_layout(a, merge_scratch_bytes(&p, prefill_choice(&p, cus), cus)).total;
}

size_t merge_scratch_bytes(const fgqa_prefill_args* a, int choice, int cus) {
    if ((choice != FGQA_KERNEL_WIDE && choice != FGQA_KERNEL_TALL) || !a->causal) return 0;
    if (a->batch == 0 || a->seqlen_q == 0 || !wide_on_pairs(a, cus)) return 0;
    return merge_scratch_bytes_for(wide_pairs(a));
}

const char* prefill_kernel_name(const fgqa_prefill_args* a, int cus) {
    switch (prefill_choice(a, cus)) {
        case FGQA_KERNEL_WHOLE: return "prefill_kernel";
        case FGQA_KERNEL_SPLIT: return "prefill_split_kernel";
        case FGQA_KERNEL_WIDE: return wide_on_pairs(a, cus) ? "prefill_wide_kernel" : "prefill_wide_persistent_kernel";
        default: return tall_on_pairs(a, cus) ? "prefill_tall_pairs_kernel" : "prefill_tall_persistent_kernel";
    }
}

// ---------------------------------------------------------------- backward

bool backward_padded(const fgqa_prefill_backward_args* a) {
    const int dv = a->head_dim_v == 0 ? a->head_dim : a->head_dim_v;
    const bool dk_ok = (a->head_dim > 0 && a->head_dim <= kHeadDim) || a->head_dim == 192;
    const bool built = dv == kHeadDim && (a->head_dim == kHeadDim || a->head_dim == 192);
    return dk_ok && dv > 0 && dv <= kHeadDim && !built;
}

int backward_padded_dk(const fgqa_prefill_backward_args* a) { return a->head_dim <= kHeadDim ? kHeadDim : 192; }

fgqa_prefill_backward_args backward_padded_args(const fgqa_prefill_backward_args* a) {
    fgqa_prefill_backward_args p = *a;
    const int dk = backward_padded_dk(a);
    p.head_dim = dk;
    p.head_dim_v = kHeadDim;
    const int64_t sq = a->seqlen_q, skv = a->seqlen_kv, hq = a->num_q_heads, hkv = a->num_kv_heads;
    const int64_t qs[3] = {sq * hq * dk, hq * dk, dk}, os[3] = {sq * hq * kHeadDim, hq * kHeadDim, kHeadDim};
    const int64_t ks[3] = {skv * hkv * dk, hkv * dk, dk}, vs[3] = {skv * hkv * kHeadDim, hkv * kHeadDim, kHeadDim};
    for (int i = 0; i < 3; ++i) {
        p.q_stride[i] = p.grad_q_stride[i] = qs[i];
        p.o_stride[i] = p.grad_o_stride[i] = os[i];
        p.k_stride[i] = p.grad_k_stride[i] = ks[i];
        p.v_stride[i] = p.grad_v_stride[i] = vs[i];
    }
    p.q = p.k = p.v = p.o = p.grad_o = nullptr;
    p.grad_q = p.grad_k = p.grad_v = nullptr;
    p.workspace = nullptr;
    p.workspace_bytes = 0;
    return p;
}

BwdPadLayout backward_pad_layout(const fgqa_prefill_backward_args* a, size_t ws_bytes) {
    const int dk = backward_padded_dk(a);
    const i128 rq = (i128)a->batch * a->seqlen_q * a->num_q_heads * 2;
    const i128 rk = (i128)a->batch * a->seqlen_kv * a->num_kv_heads * 2;
    BwdPadLayout L;
    L.q = round256(ws_bytes);
    L.k = L.q + round256(rq * dk);
    L.v = L.k + round256(rk * dk);
    L.o = L.v + round256(rk * kHeadDim);
    L.dout = L.o + round256(rq * kHeadDim);
    L.dq = L.dout + round256(rq * kHeadDim);
    L.dk = L.dq + round256(rq * dk);
    L.dv = L.dk + round256(rk * dk);
    L.total = L.dv + round256(rk * kHeadDim);
    return L;
}

int validate_backward(const fgqa_prefill_backward_args* a) {
    if (a == nullptr) return FGQA_ERR_INVALID_ARGUMENT;
    if (a->batch < 0 || a->seqlen_q < 0 || a->seqlen_kv < 0 || a->num_q_heads <= 0 || a->num_kv_heads <= 0 ||
        a->head_dim <= 0)
        return FGQA_ERR_INVALID_ARGUMENT;
    if (a->num_q_heads % a->num_kv_heads != 0) return FGQA_ERR_INVALID_ARGUMENT;
    if (!isfinite(a->scale)) return FGQA_ERR_INVALID_ARGUMENT;
    // a sliding window is a causal window (flash_swa_backward_kernel.py:278-282)
    if (a->window_size < 0 || (a->window_size > 0 && !a->causal)) return FGQA_ERR_INVALID_ARGUMENT;
    const int64_t* strides[8] = {a->q_stride,      a->k_stride,      a->v_stride,      a->o_stride,
                                 a->grad_o_stride, a->grad_q_stride, a->grad_k_stride, a->grad_v_stride};
    for (const int64_t* s : strides)
        for (int i = 0; i < 3; ++i)
            if (s[i] < 0) return FGQA_ERR_INVALID_ARGUMENT;
    // (128, 128) and the MLA shape (192, 128) (flash_mla_backward_kernel.py);
    // MLA has no sliding-window form
    if (a->head_dim_v < 0) return FGQA_ERR_INVALID_ARGUMENT;
    const int dv = a->head_dim_v == 0 ? a->head_dim : a->head_dim_v;
    // other head dims up to 128 (Q/K up to 128 or 192, V/O up to 128) run on
    // zero-padded copies
    const bool padded = backward_padded(a);
    if (!padded && (dv != kHeadDim || (a->head_dim != kHeadDim && a->head_dim != 192))) return FGQA_ERR_UNSUPPORTED;
    const int dk_run = padded ? backward_padded_dk(a) : a->head_dim;
    if (dk_run == 192 && a->window_size > 0) return FGQA_ERR_UNSUPPORTED;
    const int group = a->num_q_heads / a->num_kv_heads;
    if (a->kv_head_split < 0 || a->kv_head_split > group || (a->kv_head_split > 0 && group % a->kv_head_split != 0))
        return FGQA_ERR_INVALID_ARGUMENT;
    if (a->dq_kernel < FGQA_KERNEL_AUTO || a->dq_kernel > FGQA_KERNEL_SPLIT) return FGQA_ERR_INVALID_ARGUMENT;
    // the 192-wide dQ kernel needs one wave per SIMD: it has no split form
    if (a->dq_kernel == FGQA_KERNEL_SPLIT && dk_run == 192) return FGQA_ERR_UNSUPPORTED;
    // query rows past sq must read as zero (rows may not overlap; the
    // padded copies are contiguous)
    if (!padded && (a->q_stride[1] < a->head_dim || a->grad_o_stride[1] < kHeadDim)) return FGQA_ERR_UNSUPPORTED;
    if (a->seqlen_q > kMaxTokens || a->seqlen_kv > kMaxTokens) return FGQA_ERR_UNSUPPORTED;
    if (span_reaches_2g((int64_t)a->seqlen_q + 128, a->q_stride[1]) ||
        span_reaches_2g((int64_t)a->seqlen_q + 128, a->grad_o_stride[1]) ||
        span_reaches_2g((int64_t)a->seqlen_kv + 128, a->k_stride[1]) ||
        span_reaches_2g((int64_t)a->seqlen_kv + 128, a->v_stride[1]))
        return FGQA_ERR_UNSUPPORTED;
    {
        const int64_t qn[3] = {a->batch, a->seqlen_q, a->num_q_heads};
        const int64_t kn[3] = {a->batch, a->seqlen_kv, a->num_kv_heads};
        const int64_t* qs[4] = {a->q_stride, a->o_stride, a->grad_o_stride, a->grad_q_stride};
        const int64_t* ks[4] = {a->k_stride, a->v_stride, a->grad_k_stride, a->grad_v_stride};
        for (int i = 0; i < 4; ++i)
            if (!extent_ok(qn, qs[i]) || !extent_ok(kn, ks[i])) return FGQA_ERR_UNSUPPORTED;
    }
    // the row statistics are addressed through one buffer resource
    if ((i128)a->batch * a->num_q_heads * a->seqlen_q * 8 >= kLim31) return FGQA_ERR_UNSUPPORTED;
    // the dK/dV partials of a full head split stay describable
    if ((i128)a->batch * a->num_q_heads * a->seqlen_kv * (dk_run + kHeadDim) * 4 > kMaxWorkspace)
        return FGQA_ERR_UNSUPPORTED;
    if (padded) {
        // the copies must pass as a built call themselves, and the workspace
        // that holds them stays within the planners' limit
        const fgqa_prefill_backward_args p = backward_padded_args(a);
        if (const int st = validate_backward(&p); st != FGQA_OK) return st;
        if ((i128)backward_pad_layout(a, 0).total >= kMaxWorkspace) return FGQA_ERR_UNSUPPORTED;
    }
    return FGQA_OK;
}

int validate_backward_pointers(const fgqa_prefill_backward_args* a) {
    if (a->seqlen_q > 0 &&
        (a->q == nullptr || a->o == nullptr || a->lse == nullptr || a->grad_o == nullptr || a->grad_q == nullptr))
        return FGQA_ERR_INVALID_ARGUMENT;
    if (a->seqlen_kv > 0 && (a->k == nullptr || a->v == nullptr || a->grad_k == nullptr || a->grad_v == nullptr))
        return FGQA_ERR_INVALID_ARGUMENT;
    // padded head dims: the copies are made with 2-byte accesses
    if (backward_padded(a)) return FGQA_OK;
    const void* ptrs[8] = {a->q, a->k, a->v, a->o, a->grad_o, a->grad_q, a->grad_k, a->grad_v};
    for (const void* ptr : ptrs)
        if (!aligned16(ptr)) return FGQA_ERR_UNSUPPORTED;
    const int64_t* strides[8] = {a->q_stride,      a->k_stride,      a->v_stride,      a->o_stride,
                                 a->grad_o_stride, a->grad_q_stride, a->grad_k_stride, a->grad_v_stride};
    for (const int64_t* s : strides)
        for (int i = 0; i < 3; ++i)
            if (s[i] & 7) return FGQA_ERR_UNSUPPORTED;
    return FGQA_OK;
}

// Query heads per dK/dV workgroup: all G query heads of a KV head (dK/dV
// written once, straight from registers) unless that leaves fewer than 2
// workgroups per CU; then the heads are split over workgroups, each writing
// an fp32 partial that a reduce pass sums.  Under a sliding window every key
// block carries the same work, so one workgroup per CU (the kernel's
// occupancy) is enough and halves the partials.  The caller's kv_head_split
// field, when nonzero, sets n (a divisor of G, validated).
BwdPlan plan_backward(const fgqa_prefill_backward_args* a, int cus) {
    BwdPlan pl;
    const int group = a->num_q_heads / a->num_kv_heads;
    const i128 base = (i128)ceil_div(a->seqlen_kv, kBackwardKvKeys) * a->num_kv_heads * a->batch;
    const i128 want = (i128)(a->window_size > 0 ? 1 : 2) * cus;
    pl.n_hsplit = group;
    for (int d = 1; d <= group; ++d)
        if (group % d == 0 && base * d >= want) {
            pl.n_hsplit = d;
            break;
        }
    if (a->kv_head_split > 0) pl.n_hsplit = a->kv_head_split;
    const i128 rows_q = (i128)a->batch * a->num_q_heads * a->seqlen_q;
    const i128 rows_kv = (i128)a->batch * a->num_kv_heads * a->seqlen_kv;
    pl.stat_bytes = round256(2 * rows_q * 4);
    const i128 parts = pl.n_hsplit > 1 ? (i128)pl.n_hsplit * rows_kv * 4 : 0;
    pl.part_k_bytes = round256(parts * a->head_dim);
    pl.part_v_bytes = round256(parts * kHeadDim);
    pl.ws_bytes = pl.stat_bytes + pl.part_k_bytes + pl.part_v_bytes;
    return pl;
}

size_t backward_workspace_bytes(const fgqa_prefill_backward_args* a, int cus) {
    if (!backward_padded(a)) return plan_backward(a, cus).ws_bytes;
    const fgqa_prefill_backward_args p = backward_padded_args(a);
    return backward_pad_layout(a, plan_backward(&p, cus).ws_bytes).total;
}

int check_backward_grid(const fgqa_prefill_backward_args* a, const BwdPlan& pl) {
    const int group = a->num_q_heads / a->num_kv_heads;
    const int hb = group % 4 == 0 ? 4 : group % 2 == 0 ? 2 : 1;
    const i128 kv_streams = (i128)pl.n_hsplit * a->num_kv_heads * a->batch;
    const i128 q_streams = (i128)(group / hb) * a->num_kv_heads * a->batch;
    const i128 rows_q = (i128)a->batch * a->num_q_heads * a->seqlen_q;
    const i128 rows_kv = (i128)a->batch * a->num_kv_heads * a->seqlen_kv;
    const i128 kv_units = (i128)ceil_div(a->seqlen_kv, kBackwardKvKeys) * kv_streams;
    const i128 q_units = (i128)ceil_div(a->seqlen_q, 128 / hb) * q_streams;
    if (kv_streams >= kLim31 || q_streams >= kLim31 || (rows_q + 15) / 16 >= kLim31 ||
        (rows_kv + 15) / 16 >= kLim31 || kv_units >= kLim31 || q_units >= kLim31)
        return FGQA_ERR_UNSUPPORTED;
    return FGQA_OK;
}

// ---------------------------------------------------------------- sparse

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
    if ((i128)a->seqlen_kv * a->k_stride[1] * 2 + 256 >= kLim31 ||
        (i128)a->seqlen_kv * a->v_stride[1] * 2 + 256 >= kLim31 ||
        (i128)a->num_q_heads * a->q_stride[2] * 2 >= kLim31 || (i128)a->num_sparse_kv * 4 >= kLim31)
        return FGQA_ERR_UNSUPPORTED;
    if (a->seqlen_q > kMaxTokens || a->seqlen_kv > kMaxTokens || a->num_sparse_kv > kMaxTokens)
        return FGQA_ERR_UNSUPPORTED;
    {
        const int64_t qn[3] = {a->batch, a->seqlen_q, a->num_q_heads};
        const int64_t kn[3] = {a->batch, a->seqlen_kv, a->num_kv_heads};
        const int64_t in[3] = {a->batch, a->num_kv_heads, a->seqlen_q};
        if (!extent_ok(qn, a->q_stride) || !extent_ok(qn, a->o_stride) || !extent_ok(kn, a->k_stride) ||
            !extent_ok(kn, a->v_stride) || !extent_ok(in, a->idx_stride))
            return FGQA_ERR_UNSUPPORTED;
    }
    // one wave per (batch, KV head, query row, group of 16 query heads)
    const i128 items = (i128)a->batch * a->num_kv_heads * a->seqlen_q * ceil_div(a->num_q_heads / a->num_kv_heads, 16);
    if ((items + kSparseWaves - 1) / kSparseWaves >= kLim31) return FGQA_ERR_UNSUPPORTED;
    if (a->batch == 0 || a->seqlen_q == 0) return FGQA_OK;
    // (with Skv = 0 no K/V row is read: k and v may be null)
    if (a->q == nullptr || a->o == nullptr || a->kv_indices == nullptr ||
        (a->seqlen_kv > 0 && (a->k == nullptr || a->v == nullptr)))
        return FGQA_ERR_INVALID_ARGUMENT;
    if (!aligned16(a->q) || !aligned16(a->k) || !aligned16(a->v) || !aligned16(a->o) ||
        (reinterpret_cast<uintptr_t>(a->kv_indices) & 3u))
        return FGQA_ERR_UNSUPPORTED;
    for (int i = 0; i < 3; ++i)
        if ((a->q_stride[i] & 7) || (a->k_stride[i] & 7) || (a->v_stride[i] & 7) || (a->o_stride[i] & 7))
            return FGQA_ERR_UNSUPPORTED;
    return FGQA_OK;
}

}  // namespace plan
}  // namespace fgqa
