// Host-only validation and launch planning (cuda_llm_ops_amd/csrc/host) driven
// with the benchmark shapes, invalid arguments and extreme sizes.  Built by
// tests/test_host_sanitizers.py with g++ and AddressSanitizer +
// UndefinedBehaviorSanitizer (no recovery), so a signed overflow, an
// out-of-bounds access or any other undefined behaviour in the planner ends
// the run as a failure.  No GPU and no HIP: the CU count is an argument.
//
// Output: one line per failed check, then "N checks, M failed"; exit status 1
// when a check failed.
#include <limits.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <random>

#include "fgqa_plan.h"

using namespace fgqa;

static long g_checks = 0, g_failed = 0;

#define CHECK(cond)                                                                 \
    do {                                                                            \
        ++g_checks;                                                                 \
        if (!(cond)) {                                                              \
            ++g_failed;                                                             \
            if (g_failed < 50) fprintf(stderr, "%s:%d: %s\n", __FILE__, __LINE__, #cond); \
        }                                                                           \
    } while (0)

// 16-byte aligned stand-ins: nothing here dereferences an argument pointer.
static void* fake(uintptr_t n) { return reinterpret_cast<void*>(0x100000 + 256 * n); }

static const int kCus = 256;   // MI355X

// ---------------------------------------------------------------- decode

static fgqa_decode_args decode_args(int B, int S, int hq, int hkv) {
    fgqa_decode_args a;
    memset(&a, 0, sizeof a);
    a.q = fake(1);
    a.k = fake(2);
    a.v = fake(3);
    a.o = fake(4);
    a.batch = B;
    a.max_seqlen = S;
    a.num_q_heads = hq;
    a.num_kv_heads = hkv;
    a.head_dim = 128;
    a.scale = 0.08838834764831845f;
    // contiguous q [B, Hq, D], k / v [B, S, Hkv, D], o [B, Hq, D]
    a.q_stride[0] = (int64_t)hq * 128;
    a.q_stride[1] = 128;
    a.k_stride[0] = (int64_t)S * hkv * 128;
    a.k_stride[1] = (int64_t)hkv * 128;
    a.k_stride[2] = 128;
    for (int i = 0; i < 3; ++i) a.v_stride[i] = a.k_stride[i];
    a.o_stride[0] = a.q_stride[0];
    a.o_stride[1] = 128;
    return a;
}

// What any plan must give: splits of whole 128-token passes that cover the
// longest sequence with no empty split, and a workspace that holds what the
// kernels write (fp32 O and (max, sum) per split slot, the work list).
static void check_decode_plan(const plan::DecodeShape& s, const plan::DecodePlan& pl) {
    const int64_t S = s.max_seqlen > 0 ? s.max_seqlen : 1;
    CHECK(pl.chunk >= 128 && pl.chunk % 128 == 0);
    CHECK(pl.nsplit >= 1);
    CHECK((int64_t)pl.chunk * pl.nsplit >= S);
    CHECK((int64_t)pl.chunk * (pl.nsplit - 1) < S);
    if (s.split_tokens > 0 && (int64_t)s.split_tokens < S) CHECK(pl.chunk == (s.split_tokens + 127) / 128 * 128);
    const __int128 slots = (__int128)s.batch * s.num_q_heads * pl.nsplit;
    if (pl.nsplit > 1) {
        CHECK((__int128)pl.part_o_bytes >= slots * 128 * 4);
        CHECK((__int128)pl.part_ml_bytes >= slots * 8);
        CHECK(pl.part_o_bytes % 256 == 0 && pl.part_ml_bytes % 256 == 0);
    } else {
        CHECK(pl.part_o_bytes == 0 && pl.part_ml_bytes == 0);
    }
    if (pl.list) {
        CHECK(s.ragged && s.batch < (1 << 15) && pl.nsplit < (1 << 16));
        CHECK((__int128)pl.ws_bytes >= (__int128)pl.part_o_bytes + pl.part_ml_bytes + (1 + (__int128)s.batch * pl.nsplit) * 4);
    } else {
        CHECK(pl.ws_bytes == pl.part_o_bytes + pl.part_ml_bytes);
    }
}

static void test_decode_known_shapes() {
    // config 2: B=60, S=4096, Hq=128, Hkv=8.  480 (batch, KV head) streams
    // already fill 256 CUs: one split each, no combine, no workspace.
    {
        fgqa_decode_args a = decode_args(60, 4096, 128, 8);
        CHECK(plan::validate_decode(&a) == FGQA_OK);
        CHECK(plan::validate_decode_pointers(&a) == FGQA_OK);
        plan::DecodePlan pl;
        CHECK(plan::decode_needs_cus(plan::decode_shape(&a)));
        CHECK(plan::plan_decode(plan::decode_shape(&a), kCus, &pl) == FGQA_OK);
        CHECK(pl.nsplit == 1 && pl.chunk == 4096 && !pl.list && pl.ws_bytes == 0);
        // without a CU count the automatic split cannot be planned
        CHECK(plan::plan_decode(plan::decode_shape(&a), 0, &pl) == FGQA_ERR_HIP);
    }
    // config 1: B=2, S=512, Hq=16, Hkv=2: 4 streams on 256 CUs split as far
    // as 128-token passes go: 4 splits of 128.
    {
        fgqa_decode_args a = decode_args(2, 512, 16, 2);
        plan::DecodePlan pl;
        CHECK(plan::plan_decode(plan::decode_shape(&a), kCus, &pl) == FGQA_OK);
        CHECK(pl.nsplit == 4 && pl.chunk == 128 && !pl.list);
        CHECK(pl.part_o_bytes == 2u * 16 * 4 * 128 * 4);   // B * Hq * splits * D fp32
        CHECK(pl.part_ml_bytes == 2u * 16 * 4 * 2 * 4);    // (max, sum) fp32 per slot
    }
    // config 3: ragged B=64 up to 32768 tokens, Hq=64, Hkv=8: a work list of
    // 4096-token splits, 8 per sequence.
    {
        fgqa_decode_args a = decode_args(64, 32768, 64, 8);
        int32_t lens[1];
        a.seqlens = lens;
        plan::DecodePlan pl;
        CHECK(!plan::decode_needs_cus(plan::decode_shape(&a)));
        CHECK(plan::plan_decode(plan::decode_shape(&a), 0, &pl) == FGQA_OK);
        CHECK(pl.list && pl.chunk == 4096 && pl.nsplit == 8);
        CHECK(pl.part_o_bytes == 64u * 64 * 8 * 128 * 4);   // 16 MiB
        CHECK(pl.part_ml_bytes == 64u * 64 * 8 * 2 * 4);    // 256 KiB
        CHECK(pl.ws_bytes == pl.part_o_bytes + pl.part_ml_bytes + (1 + 64 * 8) * 4);
    }
}

static void test_decode_rejections() {
    fgqa_decode_args a = decode_args(2, 512, 16, 2);
    CHECK(plan::validate_decode(nullptr) == FGQA_ERR_INVALID_ARGUMENT);
    fgqa_decode_args b = a;
    b.batch = -1;
    CHECK(plan::validate_decode(&b) == FGQA_ERR_INVALID_ARGUMENT);
    b = a;
    b.num_kv_heads = 3;   // 16 % 3
    CHECK(plan::validate_decode(&b) == FGQA_ERR_INVALID_ARGUMENT);
    b = a;
    b.head_dim = 64;
    CHECK(plan::validate_decode(&b) == FGQA_ERR_UNSUPPORTED);
    b = decode_args(2, 512, 34, 2);   // 17 query heads per KV head
    CHECK(plan::validate_decode(&b) == FGQA_ERR_UNSUPPORTED);
    b = a;
    b.scale = 1.f / 0.f;
    CHECK(plan::validate_decode(&b) == FGQA_ERR_INVALID_ARGUMENT);
    b = a;
    b.k_stride[1] = -8;
    CHECK(plan::validate_decode(&b) == FGQA_ERR_INVALID_ARGUMENT);
    b = a;
    b.k = reinterpret_cast<const char*>(b.k) + 8;
    CHECK(plan::validate_decode_pointers(&b) == FGQA_ERR_UNSUPPORTED);
    b = a;
    b.v_stride[1] = 1028;   // rows not 16-byte aligned
    CHECK(plan::validate_decode_pointers(&b) == FGQA_ERR_UNSUPPORTED);
    b = a;
    b.o = nullptr;
    CHECK(plan::validate_decode_pointers(&b) == FGQA_ERR_INVALID_ARGUMENT);
    b.batch = 0;   // nothing is read or written
    CHECK(plan::validate_decode_pointers(&b) == FGQA_OK);
    // one sequence's K span reaches 2 GiB: (S + 64) * row bytes
    b = a;
    b.k_stride[1] = 8;
    b.v_stride[1] = 8;
    b.max_seqlen = (1 << 27) - 64;   // (2^27) * 16 B = 2^31
    CHECK(plan::validate_decode(&b) == FGQA_ERR_UNSUPPORTED);
    b.max_seqlen = (1 << 27) - 65;
    CHECK(plan::validate_decode(&b) == FGQA_OK);
    b.v_stride[1] = 16;              // V's span decides alone
    CHECK(plan::validate_decode(&b) == FGQA_ERR_UNSUPPORTED);
    // sequence length limit (stride 0: every token reads one row)
    b = a;
    b.k_stride[1] = 0;
    b.v_stride[1] = 0;
    b.max_seqlen = plan::kMaxTokens;
    CHECK(plan::validate_decode(&b) == FGQA_OK);
    b.max_seqlen = plan::kMaxTokens + 1;
    CHECK(plan::validate_decode(&b) == FGQA_ERR_UNSUPPORTED);
    b.max_seqlen = INT_MAX;
    CHECK(plan::validate_decode(&b) == FGQA_ERR_UNSUPPORTED);
    // huge strides: products formed without overflow
    b = a;
    b.k_stride[1] = INT64_MAX - 7;
    CHECK(plan::validate_decode(&b) == FGQA_ERR_UNSUPPORTED);
}

static void test_decode_extremes() {
    // the longest sequence in 128-token splits: 2^23 splits, no work list
    plan::DecodeShape s{1, plan::kMaxTokens, 16, 2, 128, true};
    plan::DecodePlan pl;
    CHECK(plan::plan_decode(s, kCus, &pl) == FGQA_OK);
    CHECK(pl.nsplit == (1 << 23) && !pl.list);
    check_decode_plan(s, pl);
    // batch 2^31 - 1 with 16 heads and 2^23 splits: 2^58 partial slots
    s = plan::DecodeShape{INT_MAX, plan::kMaxTokens, 16, 1, 128, false};
    CHECK(plan::plan_decode(s, kCus, &pl) == FGQA_ERR_UNSUPPORTED);
    // batch 2^15 (ragged): too many sequences for the list
    s = plan::DecodeShape{1 << 15, 8192, 8, 8, 0, true};
    CHECK(plan::decode_needs_cus(s));
    CHECK(plan::plan_decode(s, kCus, &pl) == FGQA_OK);
    CHECK(!pl.list);
    check_decode_plan(s, pl);
    s.batch = (1 << 15) - 1;
    CHECK(plan::plan_decode(s, kCus, &pl) == FGQA_OK);
    CHECK(pl.list);
    check_decode_plan(s, pl);
    // split_tokens near INT_MAX (rounded up past 2^31 - 1 in 64 bits)
    s = plan::DecodeShape{4, plan::kMaxTokens, 8, 8, INT_MAX, false};
    CHECK(plan::plan_decode(s, kCus, &pl) == FGQA_OK);
    CHECK(pl.nsplit == 1 && pl.chunk == plan::kMaxTokens);
    check_decode_plan(s, pl);
    // S = 0: one (empty) pass
    s = plan::DecodeShape{4, 0, 8, 8, 0, false};
    CHECK(plan::plan_decode(s, kCus, &pl) == FGQA_OK);
    CHECK(pl.nsplit == 1 && pl.chunk == 128);
}

static void test_paged() {
    fgqa_decode_paged_args a;
    memset(&a, 0, sizeof a);
    a.q = fake(1);
    a.o = fake(2);
    a.k_cache = fake(3);
    a.v_cache = fake(4);
    static int32_t dummy[4];
    a.seqlens = dummy;
    a.block_table = dummy;
    a.batch = 64;
    a.max_seqlen = 32768;
    a.num_q_heads = 64;
    a.num_kv_heads = 8;
    a.head_dim = 128;
    a.scale = 0.088f;
    a.k_scale = a.v_scale = 1.f;
    a.page_size = 16;
    a.num_pages = 64 * 2048;
    a.block_table_stride = 2048;
    a.kv_dtype = FGQA_KV_BF16;
    a.q_stride[0] = 64 * 128;
    a.q_stride[1] = 128;
    a.o_stride[0] = 64 * 128;
    a.o_stride[1] = 128;
    a.k_stride[0] = 16 * 8 * 128;
    a.k_stride[1] = 8 * 128;
    a.k_stride[2] = 128;
    memcpy(a.v_stride, a.k_stride, sizeof a.k_stride);
    CHECK(plan::validate_paged(&a) == FGQA_OK);
    CHECK(plan::validate_paged_pointers(&a) == FGQA_OK);
    plan::DecodePlan pl;
    CHECK(plan::plan_paged(&a, &pl) == FGQA_OK);
    CHECK(pl.list && pl.nsplit == 8);
    // the block table row must cover max_seqlen
    fgqa_decode_paged_args b = a;
    b.block_table_stride = 2047;
    CHECK(plan::validate_paged(&b) == FGQA_ERR_INVALID_ARGUMENT);
    b = a;
    b.block_table_stride = INT64_MAX;
    b.page_size = 1 << 20;
    b.batch = 1;
    CHECK(plan::validate_paged(&b) == FGQA_OK);   // INT64_MAX * 2^20 formed without overflow
    b.batch = 2;                                  // row 1 of the table at 2^63 - 1 entries
    CHECK(plan::validate_paged(&b) == FGQA_ERR_UNSUPPORTED);
    b.page_size = 24;
    CHECK(plan::validate_paged(&b) == FGQA_ERR_UNSUPPORTED);
    b = a;
    b.kv_dtype = 7;
    CHECK(plan::validate_paged(&b) == FGQA_ERR_INVALID_ARGUMENT);
    // fp8 rows: strides in multiples of 16 elements
    b = a;
    b.kv_dtype = FGQA_KV_FP8_E4M3;
    b.k_stride[1] = 8;
    CHECK(plan::validate_paged_pointers(&b) == FGQA_ERR_UNSUPPORTED);
    // the list's limits
    b = a;
    b.batch = 1 << 15;
    CHECK(plan::plan_paged(&b, &pl) == FGQA_ERR_UNSUPPORTED);
    b = a;
    b.split_tokens = 128;
    b.max_seqlen = plan::kMaxTokens;
    b.block_table_stride = plan::kMaxTokens / 16;
    CHECK(plan::validate_paged(&b) == FGQA_OK);
    CHECK(plan::plan_paged(&b, &pl) == FGQA_ERR_UNSUPPORTED);   // 2^23 splits
    b.max_seqlen = plan::kMaxTokens + 1;
    b.block_table_stride = INT64_MAX;
    CHECK(plan::validate_paged(&b) == FGQA_ERR_UNSUPPORTED);
}

// ---------------------------------------------------------------- prefill

static fgqa_prefill_args prefill_args(int B, int S, int hq, int hkv, bool causal) {
    fgqa_prefill_args a;
    memset(&a, 0, sizeof a);
    a.q = fake(1);
    a.k = fake(2);
    a.v = fake(3);
    a.o = fake(4);
    a.batch = B;
    a.seqlen_q = S;
    a.seqlen_kv = S;
    a.num_q_heads = hq;
    a.num_kv_heads = hkv;
    a.head_dim = 128;
    a.scale = 0.088f;
    a.causal = causal ? 1 : 0;
    // [B, S, H, D]
    a.q_stride[0] = (int64_t)S * hq * 128;
    a.q_stride[1] = (int64_t)hq * 128;
    a.q_stride[2] = 128;
    a.k_stride[0] = (int64_t)S * hkv * 128;
    a.k_stride[1] = (int64_t)hkv * 128;
    a.k_stride[2] = 128;
    memcpy(a.v_stride, a.k_stride, sizeof a.k_stride);
    memcpy(a.o_stride, a.q_stride, sizeof a.q_stride);
    return a;
}

static void test_prefill_known_shapes() {
    // config 4: B=1, S=4096, Hq=16, Hkv=1, causal.  Units of 32 query rows x
    // 8 heads: 128 row blocks x 2 head groups = 256 units, 128 pairs, two
    // workgroups per pair: exactly 256 CUs.
    fgqa_prefill_args a = prefill_args(1, 4096, 16, 1, true);
    CHECK(plan::validate_prefill(&a) == FGQA_OK);
    CHECK(plan::wide_pairs(&a) == 128);
    CHECK(plan::wide_on_pairs(&a, kCus));
    CHECK(plan::prefill_choice(&a, kCus) == FGQA_KERNEL_WIDE);
    CHECK(strcmp(plan::prefill_kernel_name(&a, kCus), "prefill_wide_kernel") == 0);
    // counters, then two slots of 2*4*66*64 floats per pair
    CHECK(plan::merge_scratch_bytes(&a, FGQA_KERNEL_WIDE, kCus) == 4096u + 128u * 2 * 33792 * 4);
    CHECK(plan::merge_scratch_bytes_for(plan::kPrefillMaxSplit) == plan::merge_scratch_bytes(&a, FGQA_KERNEL_WIDE, kCus));
    // fewer CUs: the pairs no longer fit, whole units on a persistent grid,
    // and no merge scratch
    CHECK(!plan::wide_on_pairs(&a, 255));
    CHECK(plan::merge_scratch_bytes(&a, FGQA_KERNEL_WIDE, 255) == 0);
    // forced kernels come back as given
    for (int k = FGQA_KERNEL_WHOLE; k <= FGQA_KERNEL_TALL; ++k) {
        fgqa_prefill_args f = a;
        f.kernel = k;
        CHECK(plan::validate_prefill(&f) == FGQA_OK);
        CHECK(plan::prefill_choice(&f, kCus) == k);
    }
    a.kernel = FGQA_KERNEL_TALL;
    CHECK(strcmp(plan::prefill_kernel_name(&a, kCus), "prefill_tall_pairs_kernel") == 0);
    CHECK(strcmp(plan::prefill_kernel_name(&a, 100), "prefill_tall_persistent_kernel") == 0);
    // config 5: B=4, S=16384, Hq=32, Hkv=8: 16384 128-row units (64 per CU):
    // the persistent wide kernel
    fgqa_prefill_args c5 = prefill_args(4, 16384, 32, 8, true);
    CHECK(plan::prefill_choice(&c5, kCus) == FGQA_KERNEL_WIDE);
    CHECK(strcmp(plan::prefill_kernel_name(&c5, kCus), "prefill_wide_persistent_kernel") == 0);
    CHECK(plan::merge_scratch_bytes(&c5, FGQA_KERNEL_WIDE, kCus) == 0);
    // non-causal, few units: the split kernel; a window: the whole-range kernel
    fgqa_prefill_args nc = prefill_args(1, 1024, 16, 1, false);
    CHECK(plan::prefill_choice(&nc, kCus) == FGQA_KERNEL_SPLIT);
    CHECK(plan::merge_scratch_bytes(&nc, FGQA_KERNEL_SPLIT, kCus) == 0);
    fgqa_prefill_args w = prefill_args(1, 4096, 16, 1, true);
    w.window_size = 512;
    CHECK(plan::prefill_choice(&w, kCus) == FGQA_KERNEL_WHOLE);
    w.window_size = 1024;
    CHECK(plan::prefill_choice(&w, kCus) == FGQA_KERNEL_WHOLE);
    // long windows, and a sink without a window over 2 units per CU: the
    // 256-row kernels (no split form with a window or sink)
    w.window_size = 1536;
    CHECK(plan::prefill_choice(&w, kCus) == FGQA_KERNEL_WIDE);
    w.window_size = 0;
    w.sink = reinterpret_cast<const float*>(fake(9));
    CHECK(plan::prefill_choice(&w, kCus) == FGQA_KERNEL_WIDE);
    fgqa_prefill_args ws = prefill_args(1, 2048, 16, 1, true);   // 256 units of 128 rows
    ws.sink = w.sink;
    CHECK(plan::prefill_choice(&ws, kCus) == FGQA_KERNEL_WIDE);
    ws = prefill_args(1, 1024, 16, 1, true);
    ws.sink = w.sink;
    CHECK(plan::prefill_choice(&ws, kCus) == FGQA_KERNEL_WHOLE);
}

static void test_prefill_rejections() {
    const fgqa_prefill_args a = prefill_args(1, 4096, 16, 1, true);
    fgqa_prefill_args b = a;
    CHECK(plan::validate_prefill(nullptr) == FGQA_ERR_INVALID_ARGUMENT);
    b.window_size = 16;
    b.causal = 0;   // a window is causal
    CHECK(plan::validate_prefill(&b) == FGQA_ERR_INVALID_ARGUMENT);
    b = a;
    b.kernel = FGQA_KERNEL_TALL + 1;
    CHECK(plan::validate_prefill(&b) == FGQA_ERR_INVALID_ARGUMENT);
    b.kernel = -1;
    CHECK(plan::validate_prefill(&b) == FGQA_ERR_INVALID_ARGUMENT);
    b = a;
    b.kernel = FGQA_KERNEL_TALL;
    b.window_size = 64;
    CHECK(plan::validate_prefill(&b) == FGQA_ERR_UNSUPPORTED);
    b = a;
    b.kernel = FGQA_KERNEL_SPLIT;
    b.sink = reinterpret_cast<const float*>(fake(9));
    CHECK(plan::validate_prefill(&b) == FGQA_ERR_UNSUPPORTED);
    b = a;
    b.head_dim = 192;   // MLA shape (V stays 128)
    b.head_dim_v = 128;
    CHECK(plan::validate_prefill(&b) == FGQA_OK);
    b.head_dim_v = 320;
    CHECK(plan::validate_prefill(&b) == FGQA_ERR_UNSUPPORTED);
    b = a;
    b.o_stride[1] = 2052;
    CHECK(plan::validate_prefill(&b) == FGQA_ERR_UNSUPPORTED);
    b = a;
    b.seqlen_q = plan::kMaxTokens + 1;
    CHECK(plan::validate_prefill(&b) == FGQA_ERR_UNSUPPORTED);
    b = a;
    b.q_stride[1] = INT64_MAX - 7;
    CHECK(plan::validate_prefill(&b) == FGQA_ERR_UNSUPPORTED);
    // 2^31 - 1 sequences of 32 query rows x 16 heads: unit indices overflow 32 bits
    b = a;
    b.batch = INT_MAX;
    b.seqlen_q = b.seqlen_kv = 32;
    CHECK(plan::validate_prefill(&b) == FGQA_ERR_UNSUPPORTED);
    b.batch = (1 << 27) - 1;   // (2^27 - 1) * 16 row blocks: under 2^31
    CHECK(plan::validate_prefill(&b) == FGQA_OK);
    // empty calls need no pointers
    b = a;
    b.q = b.k = b.v = nullptr;
    b.o = nullptr;
    b.seqlen_q = 0;
    CHECK(plan::validate_prefill(&b) == FGQA_OK);
    b.seqlen_q = 1;
    CHECK(plan::validate_prefill(&b) == FGQA_ERR_INVALID_ARGUMENT);
}

// Head dims up to 128 other than (128, 128) run on zero-padded copies.
static fgqa_prefill_args with_head_dims(fgqa_prefill_args a, int dqk, int dv) {
    a.head_dim = dqk;
    a.head_dim_v = dv;
    a.q_stride[0] = (int64_t)a.seqlen_q * a.num_q_heads * dqk;
    a.q_stride[1] = (int64_t)a.num_q_heads * dqk;
    a.q_stride[2] = dqk;
    a.k_stride[0] = (int64_t)a.seqlen_kv * a.num_kv_heads * dqk;
    a.k_stride[1] = (int64_t)a.num_kv_heads * dqk;
    a.k_stride[2] = dqk;
    a.v_stride[0] = (int64_t)a.seqlen_kv * a.num_kv_heads * dv;
    a.v_stride[1] = (int64_t)a.num_kv_heads * dv;
    a.v_stride[2] = dv;
    a.o_stride[0] = (int64_t)a.seqlen_q * a.num_q_heads * dv;
    a.o_stride[1] = (int64_t)a.num_q_heads * dv;
    a.o_stride[2] = dv;
    return a;
}

static void test_prefill_padded_head_dims() {
    const fgqa_prefill_args c4 = prefill_args(1, 4096, 16, 1, true);
    CHECK(!plan::prefill_padded(&c4));
    fgqa_prefill_args m = c4;
    m.head_dim = 192;
    m.head_dim_v = 128;
    CHECK(!plan::prefill_padded(&m));
    // config 4's shape at D = 64: the (128, 128) call on copies, whose
    // workspace is the wide kernel's merge scratch, then Q, K, V and O
    // padded to 128 (16 MiB, 1 MiB, 1 MiB, 16 MiB)
    fgqa_prefill_args a = with_head_dims(c4, 64, 64);
    CHECK(plan::prefill_padded(&a));
    CHECK(plan::validate_prefill(&a) == FGQA_OK);
    const fgqa_prefill_args p = plan::padded_args(&a);
    CHECK(p.head_dim == 128 && p.head_dim_v == 128 && p.q == nullptr && p.workspace == nullptr);
    CHECK(p.q_stride[0] == 4096 * 16 * 128 && p.q_stride[1] == 16 * 128 && p.q_stride[2] == 128);
    CHECK(p.k_stride[1] == 128 && p.v_stride[1] == 128 && p.o_stride[1] == 16 * 128);
    CHECK(p.causal == 1 && p.scale == a.scale && p.kernel == a.kernel);
    CHECK(plan::prefill_choice(&p, kCus) == FGQA_KERNEL_WIDE);
    const size_t merge = 4096u + 128u * 2 * 33792 * 4;
    const plan::PadLayout L = plan::pad_layout(&a, merge);
    CHECK(L.q == merge && L.k == L.q + (16u << 20) && L.v == L.k + (1u << 20) && L.o == L.v + (1u << 20));
    CHECK(L.total == L.o + (16u << 20));
    CHECK(plan::prefill_workspace_bytes(&a, kCus) == L.total);
    CHECK(plan::prefill_workspace_bytes(&c4, kCus) == merge);
    // no merge scratch: the copies still start after the zeroed counter
    // prefix, which a later call on the same workspace may merge through
    CHECK(plan::pad_layout(&a, 0).q == FGQA_PREFILL_WORKSPACE_ZERO_BYTES);
    CHECK(plan::pad_layout(&a, 100).q == FGQA_PREFILL_WORKSPACE_ZERO_BYTES);
    CHECK(plan::prefill_workspace_bytes(&a, 255) == plan::pad_layout(&a, 0).total);
    // every pair with both dims in [1, 128]; odd dims, rows at any alignment
    // (the copies are made with 2-byte accesses)
    const int dims[][2] = {{64, 128}, {128, 64}, {1, 1}, {100, 36}, {8, 128}, {127, 127}};
    for (const auto& d : dims) {
        fgqa_prefill_args b = with_head_dims(c4, d[0], d[1]);
        b.q = static_cast<const char*>(fake(1)) + 2;   // 2-byte aligned only
        CHECK(plan::prefill_padded(&b));
        CHECK(plan::validate_prefill(&b) == FGQA_OK);
    }
    // up to 256: Q/K padded to 128, 192 (MLA's kernels) or 256 (the
    // whole-range kernel), V/O to 128 or 256 (two launches of 128 columns)
    struct Pad { int dqk, dv, dk_run, dv_run; };
    const Pad pads[] = {{129, 129, 256, 256}, {64, 129, 128, 256}, {256, 256, 256, 256}, {192, 64, 192, 128},
                        {128, 192, 128, 256}, {200, 72, 256, 128}, {192, 192, 192, 256}, {1, 256, 128, 256}};
    for (const Pad& d : pads) {
        fgqa_prefill_args b = with_head_dims(c4, d.dqk, d.dv);
        CHECK(plan::prefill_padded(&b));
        CHECK(plan::validate_prefill(&b) == FGQA_OK);
        CHECK(plan::padded_dk(&b) == d.dk_run && plan::padded_dv(&b) == d.dv_run);
        const fgqa_prefill_args p2 = plan::padded_args(&b);
        CHECK(p2.head_dim == d.dk_run && p2.head_dim_v == 128);
        CHECK(p2.q_stride[2] == d.dk_run && p2.k_stride[2] == d.dk_run);
        CHECK(p2.v_stride[2] == d.dv_run && p2.o_stride[2] == d.dv_run && p2.o_stride[1] == 16 * d.dv_run);
        // Q/K 256 runs the whole-range kernel, which merges nothing
        if (d.dk_run == 256) CHECK(plan::prefill_choice(&p2, kCus) == FGQA_KERNEL_WHOLE);
        const plan::PadLayout Lb = plan::pad_layout(&b, 0);
        CHECK(Lb.k - Lb.q == (size_t)4096 * 16 * d.dk_run * 2 && Lb.v - Lb.k == (size_t)4096 * d.dk_run * 2);
        CHECK(Lb.o - Lb.v == (size_t)4096 * d.dv_run * 2 && Lb.total - Lb.o == (size_t)4096 * 16 * d.dv_run * 2);
    }
    // (256, 128) is built: no copies
    fgqa_prefill_args n256 = with_head_dims(c4, 256, 128);
    CHECK(!plan::prefill_padded(&n256));
    CHECK(plan::validate_prefill(&n256) == FGQA_OK);
    CHECK(plan::prefill_choice(&n256, kCus) == FGQA_KERNEL_WHOLE);
    CHECK(plan::prefill_workspace_bytes(&n256, kCus) == 0);
    n256.kernel = FGQA_KERNEL_SPLIT;
    CHECK(plan::validate_prefill(&n256) == FGQA_ERR_UNSUPPORTED);
    n256.kernel = FGQA_KERNEL_WHOLE;
    CHECK(plan::validate_prefill(&n256) == FGQA_OK);
    n256.window_size = 64;   // the whole-range kernel has the window form
    CHECK(plan::validate_prefill(&n256) == FGQA_OK);
    // above 256: not built
    const int bad[][2] = {{257, 257}, {64, 257}, {300, 128}, {1000, 8}};
    for (const auto& d : bad) {
        fgqa_prefill_args b = with_head_dims(c4, d[0], d[1]);
        CHECK(!plan::prefill_padded(&b));
        CHECK(plan::validate_prefill(&b) == FGQA_ERR_UNSUPPORTED);
    }
    // the 192 kernels have no window form, padded or not
    fgqa_prefill_args w192 = with_head_dims(c4, 192, 64);
    w192.window_size = 64;
    CHECK(plan::validate_prefill(&w192) == FGQA_ERR_UNSUPPORTED);
    // forced shapes the 256 kernel lacks
    fgqa_prefill_args f256 = with_head_dims(c4, 160, 96);
    f256.kernel = FGQA_KERNEL_WIDE;
    CHECK(plan::validate_prefill(&f256) == FGQA_ERR_UNSUPPORTED);
    f256.kernel = FGQA_KERNEL_TALL;
    CHECK(plan::validate_prefill(&f256) == FGQA_ERR_UNSUPPORTED);
    // the window and sink forms, and a forced tall kernel, take padded dims
    fgqa_prefill_args w = a;
    w.window_size = 512;
    w.sink = reinterpret_cast<const float*>(fake(9));
    CHECK(plan::validate_prefill(&w) == FGQA_OK);
    w = a;
    w.kernel = FGQA_KERNEL_TALL;
    CHECK(plan::validate_prefill(&w) == FGQA_OK);
    // a shape whose rows fit 32-bit offsets at D = 64 but whose copies at
    // 128 do not: (2^20 - 72) rows of 16 x 128 elements reach 2^31 bytes
    fgqa_prefill_args big = with_head_dims(prefill_args(1, (1 << 20) - 200, 16, 1, true), 64, 64);
    fgqa_prefill_args big128 = prefill_args(1, (1 << 20) - 200, 16, 1, true);
    CHECK(plan::validate_prefill(&big128) == FGQA_ERR_UNSUPPORTED);
    CHECK(plan::validate_prefill(&big) == FGQA_ERR_UNSUPPORTED);
    big = with_head_dims(prefill_args(1, (1 << 19) - 200, 16, 1, true), 64, 64);
    CHECK(plan::validate_prefill(&big) == FGQA_OK);
}

// ---------------------------------------------------------------- backward

static fgqa_prefill_backward_args backward_args(int B, int S, int hq, int hkv) {
    fgqa_prefill_backward_args a;
    memset(&a, 0, sizeof a);
    a.q = fake(1);
    a.k = fake(2);
    a.v = fake(3);
    a.o = fake(4);
    a.grad_o = fake(5);
    a.grad_q = fake(6);
    a.grad_k = fake(7);
    a.grad_v = fake(8);
    static float lse[1];
    a.lse = lse;
    a.batch = B;
    a.seqlen_q = S;
    a.seqlen_kv = S;
    a.num_q_heads = hq;
    a.num_kv_heads = hkv;
    a.head_dim = 128;
    a.scale = 0.088f;
    a.causal = 1;
    int64_t qs[3] = {(int64_t)S * hq * 128, (int64_t)hq * 128, 128};
    int64_t ks[3] = {(int64_t)S * hkv * 128, (int64_t)hkv * 128, 128};
    memcpy(a.q_stride, qs, sizeof qs);
    memcpy(a.o_stride, qs, sizeof qs);
    memcpy(a.grad_o_stride, qs, sizeof qs);
    memcpy(a.grad_q_stride, qs, sizeof qs);
    memcpy(a.k_stride, ks, sizeof ks);
    memcpy(a.v_stride, ks, sizeof ks);
    memcpy(a.grad_k_stride, ks, sizeof ks);
    memcpy(a.grad_v_stride, ks, sizeof ks);
    return a;
}

static void test_backward() {
    // config 4 backward: 32 key blocks x 1 KV head = 32 dK/dV workgroups with
    // all 16 heads; 512 workgroups wanted on 256 CUs: split the 16 heads in 16
    fgqa_prefill_backward_args a = backward_args(1, 4096, 16, 1);
    CHECK(plan::validate_backward(&a) == FGQA_OK);
    CHECK(plan::validate_backward_pointers(&a) == FGQA_OK);
    plan::BwdPlan pl = plan::plan_backward(&a, kCus);
    CHECK(pl.n_hsplit == 16);
    CHECK(pl.stat_bytes == 16u * 4096 * 2 * 4);
    CHECK(pl.part_k_bytes == 16u * 4096 * 128 * 4 && pl.part_v_bytes == pl.part_k_bytes);
    CHECK(plan::check_backward_grid(&a, pl) == FGQA_OK);
    // config 5 backward: 128 key blocks x 8 KV heads x 4 = 4096 workgroups: no split
    a = backward_args(4, 16384, 32, 8);
    pl = plan::plan_backward(&a, kCus);
    CHECK(pl.n_hsplit == 1 && pl.part_k_bytes == 0 && pl.part_v_bytes == 0);
    // a window wants one workgroup per CU: 32 blocks x 2 = 64 < 256 -> 8 of 16
    a = backward_args(1, 4096, 16, 1);
    a.window_size = 512;
    pl = plan::plan_backward(&a, kCus);
    CHECK(pl.n_hsplit == 8);
    a.kv_head_split = 4;
    CHECK(plan::validate_backward(&a) == FGQA_OK);
    CHECK(plan::plan_backward(&a, kCus).n_hsplit == 4);
    a.kv_head_split = 3;   // not a divisor of 16
    CHECK(plan::validate_backward(&a) == FGQA_ERR_INVALID_ARGUMENT);
    a.kv_head_split = 17;
    CHECK(plan::validate_backward(&a) == FGQA_ERR_INVALID_ARGUMENT);
    // the 192-wide dQ has no split form
    a = backward_args(1, 4096, 16, 1);
    a.head_dim = 192;
    a.head_dim_v = 128;
    a.q_stride[1] = 16 * 192;
    CHECK(plan::validate_backward(&a) == FGQA_OK);
    a.dq_kernel = FGQA_KERNEL_SPLIT;
    CHECK(plan::validate_backward(&a) == FGQA_ERR_UNSUPPORTED);
    // overlapping query rows
    a = backward_args(1, 4096, 16, 1);
    a.q_stride[1] = 64;
    CHECK(plan::validate_backward(&a) == FGQA_ERR_UNSUPPORTED);
    // padded head dims: Q/K up to 128 (run at 128) or 192 (run at 192), V/O
    // up to 128 (run at 128); any alignment
    {
        struct Pad { int dqk, dv, dk_run; bool ok; };
        const Pad pads[] = {{64, 64, 128, true},   {1, 1, 128, true},    {100, 36, 128, true}, {192, 64, 192, true},
                            {128, 64, 128, true},  {64, 128, 128, true}, {200, 128, 0, false}, {64, 129, 0, false},
                            {256, 128, 0, false}, {128, 192, 0, false}};
        for (const Pad& d : pads) {
            fgqa_prefill_backward_args b = backward_args(1, 4096, 16, 1);
            b.head_dim = d.dqk;
            b.head_dim_v = d.dv;
            const int64_t qs[3] = {4096LL * 16 * d.dqk, 16LL * d.dqk, d.dqk}, os[3] = {4096LL * 16 * d.dv, 16LL * d.dv, d.dv};
            const int64_t ks[3] = {4096LL * d.dqk, d.dqk, d.dqk}, vs[3] = {4096LL * d.dv, d.dv, d.dv};
            memcpy(b.q_stride, qs, sizeof qs);
            memcpy(b.grad_q_stride, qs, sizeof qs);
            memcpy(b.o_stride, os, sizeof os);
            memcpy(b.grad_o_stride, os, sizeof os);
            memcpy(b.k_stride, ks, sizeof ks);
            memcpy(b.grad_k_stride, ks, sizeof ks);
            memcpy(b.v_stride, vs, sizeof vs);
            memcpy(b.grad_v_stride, vs, sizeof vs);
            b.grad_v = static_cast<char*>(b.grad_v) + 2;   // 2-byte aligned only
            CHECK(plan::backward_padded(&b) == d.ok);
            CHECK(plan::validate_backward(&b) == (d.ok ? FGQA_OK : FGQA_ERR_UNSUPPORTED));
            if (!d.ok) continue;
            CHECK(plan::validate_backward_pointers(&b) == FGQA_OK);
            CHECK(plan::backward_padded_dk(&b) == d.dk_run);
            const fgqa_prefill_backward_args p = plan::backward_padded_args(&b);
            CHECK(p.head_dim == d.dk_run && p.head_dim_v == 128 && p.q == nullptr && p.workspace == nullptr);
            CHECK(p.q_stride[1] == 16 * d.dk_run && p.grad_k_stride[1] == d.dk_run && p.o_stride[1] == 16 * 128);
            CHECK(!plan::backward_padded(&p) && plan::validate_backward(&p) == FGQA_OK);
            const size_t inner = plan::plan_backward(&p, kCus).ws_bytes;
            const plan::BwdPadLayout L = plan::backward_pad_layout(&b, inner);
            const size_t rq = 4096u * 16 * 2, rk = 4096u * 2;
            CHECK(L.q == inner && L.k - L.q == rq * d.dk_run && L.v - L.k == rk * d.dk_run);
            CHECK(L.o - L.v == rk * 128 && L.dout - L.o == rq * 128 && L.dq - L.dout == rq * 128);
            CHECK(L.dk - L.dq == rq * d.dk_run && L.dv - L.dk == rk * d.dk_run && L.total - L.dv == rk * 128);
            CHECK(plan::backward_workspace_bytes(&b, kCus) == L.total);
            fgqa_prefill_backward_args w = b;
            w.window_size = 64;
            CHECK(plan::validate_backward(&w) == (d.dk_run == 192 ? FGQA_ERR_UNSUPPORTED : FGQA_OK));
            w = b;
            w.dq_kernel = FGQA_KERNEL_SPLIT;
            CHECK(plan::validate_backward(&w) == (d.dk_run == 192 ? FGQA_ERR_UNSUPPORTED : FGQA_OK));
        }
        const fgqa_prefill_backward_args built = backward_args(1, 4096, 16, 1);
        CHECK(!plan::backward_padded(&built));
        CHECK(plan::backward_workspace_bytes(&built, kCus) == plan::plan_backward(&built, kCus).ws_bytes);
    }
    // a huge batch without query rows: the row statistics are empty, but the
    // dK/dV grid of 2^31 - 1 batches x 2^12 heads cannot be indexed
    a = backward_args(INT_MAX, 0, 4096, 4096);
    a.seqlen_kv = 1;
    memset(a.k_stride, 0, sizeof a.k_stride);
    memset(a.v_stride, 0, sizeof a.v_stride);
    CHECK(plan::validate_backward(&a) == FGQA_ERR_UNSUPPORTED);   // partials beyond 2^46 bytes
    a.num_q_heads = a.num_kv_heads = 64;
    a.batch = 1 << 26;
    CHECK(plan::validate_backward(&a) == FGQA_OK);
    pl = plan::plan_backward(&a, kCus);
    CHECK(plan::check_backward_grid(&a, pl) == FGQA_ERR_UNSUPPORTED);   // 2^32 KV streams
    a.batch = 1 << 20;
    pl = plan::plan_backward(&a, kCus);
    CHECK(plan::check_backward_grid(&a, pl) == FGQA_OK);
    // the row statistics of 2^31 / 8 rows
    a = backward_args(1 << 14, 1 << 10, 16, 16);
    CHECK(plan::validate_backward(&a) == FGQA_ERR_UNSUPPORTED);
    a = backward_args((1 << 14) - 1, 1 << 10, 16, 16);
    CHECK(plan::validate_backward(&a) == FGQA_OK);
}

// ---------------------------------------------------------------- sparse

static void test_sparse() {
    fgqa_sparse_prefill_args a;
    memset(&a, 0, sizeof a);
    a.q = fake(1);
    a.k = fake(2);
    a.v = fake(3);
    a.o = fake(4);
    static int32_t idx[4];
    a.kv_indices = idx;
    a.batch = 1;
    a.seqlen_q = 4096;
    a.seqlen_kv = 4096;
    a.num_q_heads = 16;
    a.num_kv_heads = 1;
    a.head_dim = 128;
    a.num_sparse_kv = 2048;
    a.scale = 0.088f;
    int64_t qs[3] = {4096 * 16 * 128, 16 * 128, 128};
    int64_t ks[3] = {4096 * 128, 128, 128};
    memcpy(a.q_stride, qs, sizeof qs);
    memcpy(a.o_stride, qs, sizeof qs);
    memcpy(a.k_stride, ks, sizeof ks);
    memcpy(a.v_stride, ks, sizeof ks);
    CHECK(plan::validate_sparse(&a) == FGQA_OK);
    fgqa_sparse_prefill_args b = a;
    b.num_sparse_kv = 0;
    CHECK(plan::validate_sparse(&b) == FGQA_ERR_INVALID_ARGUMENT);
    b = a;
    b.kv_indices = reinterpret_cast<const int32_t*>(reinterpret_cast<const char*>(idx) + 2);
    CHECK(plan::validate_sparse(&b) == FGQA_ERR_UNSUPPORTED);
    b = a;
    b.seqlen_kv = 0;   // no K/V row is read
    b.k = b.v = nullptr;
    CHECK(plan::validate_sparse(&b) == FGQA_OK);
    // 2^31 - 1 batches x 2^20 rows: the wave count is formed without overflow
    b = a;
    b.batch = INT_MAX;
    b.seqlen_q = 1 << 20;
    b.num_q_heads = b.num_kv_heads = 1 << 10;
    b.q_stride[2] = 128;
    CHECK(plan::validate_sparse(&b) == FGQA_ERR_UNSUPPORTED);
    // 2^15 batches x 4 KV heads x 2^16 rows = 2^33 waves: 2^31 workgroups of 4
    b = a;
    b.batch = 1 << 15;
    b.seqlen_q = 1 << 16;
    b.num_q_heads = 64;
    b.num_kv_heads = 4;
    CHECK(plan::validate_sparse(&b) == FGQA_ERR_UNSUPPORTED);
    b.batch = (1 << 15) - 1;
    CHECK(plan::validate_sparse(&b) == FGQA_OK);
}

// ---------------------------------------------------------------- fuzz

// Every entry over arguments drawn from edge values: the validators and, for
// what they accept, the planners must run without undefined behaviour and
// give plans that hold the invariants above.
static void fuzz(unsigned seed, int rounds) {
    std::mt19937_64 rng(seed);
    const int64_t ints[] = {0, 1, 2, 7, 8, 15, 16, 17, 31, 32, 33, 127, 128, 129, 192, 4096, 32768,
                            1 << 15, 1 << 16, (1 << 20) + 1, 1 << 30, (1 << 30) + 1, INT_MAX, -1, INT_MIN};
    const int64_t strides[] = {0, 8, 16, 128, 136, 1024, 1 << 20, (int64_t)1 << 31, (int64_t)1 << 40,
                               (int64_t)1 << 62, INT64_MAX - 7, INT64_MAX, -8, INT64_MIN, 12};
    const int64_t sane_strides[] = {0, 8, 128, 1024, 2048, 16384, 1 << 20};
    const int heads[] = {1, 2, 4, 8, 16, 32, 64, 128};
    auto I = [&]() { return (int)ints[rng() % (sizeof ints / sizeof ints[0])]; };
    // three draws in four from values a caller would pass, one from the edges
    auto S = [&]() {
        return (rng() % 4) ? sane_strides[rng() % 7] : strides[rng() % (sizeof strides / sizeof strides[0])];
    };
    auto H = [&]() { return (rng() % 4) ? heads[rng() % 8] : I(); };
    auto Hq = [&](int hkv) { return (rng() % 4) ? (int)((int64_t)hkv * heads[rng() % 5] & INT_MAX) : I(); };
    long accepted[5] = {0, 0, 0, 0, 0};
    auto P = [&]() -> void* { return (rng() % 8) == 0 ? nullptr : fake(rng() % 4); };
    const int cus_choices[] = {0, 1, 80, 255, 256, 304, 1 << 20};
    auto C = [&]() { return cus_choices[rng() % 7]; };
    for (int r = 0; r < rounds; ++r) {
        {
            fgqa_decode_args a;
            memset(&a, 0, sizeof a);
            a.q = P(); a.k = P(); a.v = P(); a.o = P();
            a.batch = I(); a.max_seqlen = I(); a.num_kv_heads = H(); a.num_q_heads = Hq(a.num_kv_heads);
            a.head_dim = (rng() % 4) ? 128 : I();
            a.split_tokens = (rng() & 1) ? 0 : I();
            a.scale = 0.1f;
            for (int i = 0; i < 2; ++i) { a.q_stride[i] = S(); a.o_stride[i] = S(); }
            for (int i = 0; i < 3; ++i) { a.k_stride[i] = S(); a.v_stride[i] = S(); }
            static int32_t lens[1];
            a.seqlens = (rng() & 1) ? lens : nullptr;
            if (plan::validate_decode(&a) == FGQA_OK) {
                ++accepted[0];
                (void)plan::validate_decode_pointers(&a);
                plan::DecodePlan pl;
                const plan::DecodeShape sh = plan::decode_shape(&a);
                const int st = plan::plan_decode(sh, C(), &pl);
                CHECK(st == FGQA_OK || st == FGQA_ERR_HIP || st == FGQA_ERR_UNSUPPORTED);
                if (st == FGQA_OK) check_decode_plan(sh, pl);
            }
        }
        {
            fgqa_decode_paged_args a;
            memset(&a, 0, sizeof a);
            a.q = P(); a.o = P(); a.k_cache = P(); a.v_cache = P();
            static int32_t t[1];
            a.seqlens = t;
            a.block_table = t;
            a.batch = I(); a.max_seqlen = I(); a.num_kv_heads = H(); a.num_q_heads = Hq(a.num_kv_heads);
            a.head_dim = (rng() % 4) ? 128 : I();
            a.page_size = (rng() % 4) ? 16 : I();
            a.num_pages = I();
            a.block_table_stride = S();
            a.split_tokens = (rng() & 1) ? 0 : I();
            a.kv_dtype = (int)(rng() % 3);
            a.scale = a.k_scale = a.v_scale = 1.f;
            for (int i = 0; i < 2; ++i) { a.q_stride[i] = S(); a.o_stride[i] = S(); }
            for (int i = 0; i < 3; ++i) { a.k_stride[i] = S(); a.v_stride[i] = S(); }
            if (plan::validate_paged(&a) == FGQA_OK) {
                ++accepted[1];
                (void)plan::validate_paged_pointers(&a);
                plan::DecodePlan pl;
                const int st = plan::plan_paged(&a, &pl);
                CHECK(st == FGQA_OK || st == FGQA_ERR_UNSUPPORTED);
                if (st == FGQA_OK) {
                    CHECK(pl.list);
                    check_decode_plan(plan::DecodeShape{a.batch, a.max_seqlen, a.num_q_heads, a.num_kv_heads,
                                                        a.split_tokens, true}, pl);
                }
            }
        }
        {
            fgqa_prefill_args a;
            memset(&a, 0, sizeof a);
            a.q = P(); a.k = P(); a.v = P(); a.o = P();
            a.batch = I(); a.seqlen_q = I(); a.seqlen_kv = I(); a.num_kv_heads = H(); a.num_q_heads = Hq(a.num_kv_heads);
            a.head_dim = (rng() % 3) ? 128 : I();
            a.head_dim_v = (rng() & 1) ? 0 : I();
            a.scale = 0.1f;
            a.causal = (int)(rng() & 1);
            a.window_size = (rng() % 4) ? 0 : I();
            a.kernel = (rng() & 1) ? 0 : (rng() & 1) ? (int)(rng() % 5) : I();
            if ((rng() % 4) == 0) a.sink = reinterpret_cast<const float*>(fake(5));
            for (int i = 0; i < 3; ++i) {
                a.q_stride[i] = S(); a.k_stride[i] = S(); a.v_stride[i] = S(); a.o_stride[i] = S();
            }
            if (plan::validate_prefill(&a) == FGQA_OK) {
                ++accepted[2];
                const int cus = C() | 1;
                const int ch = plan::prefill_choice(&a, cus);
                CHECK(ch >= FGQA_KERNEL_WHOLE && ch <= FGQA_KERNEL_TALL);
                const size_t m = plan::merge_scratch_bytes(&a, ch, cus);
                CHECK(m == 0 || (m >= plan::kPrefillZeroBytes && m <= plan::merge_scratch_bytes_for(plan::kPrefillMaxSplit)));
                CHECK(plan::prefill_kernel_name(&a, cus) != nullptr);
            }
        }
        {
            fgqa_prefill_backward_args a;
            memset(&a, 0, sizeof a);
            a.q = P(); a.k = P(); a.v = P(); a.o = P(); a.grad_o = P(); a.grad_q = P(); a.grad_k = P(); a.grad_v = P();
            static float l[1];
            a.lse = l;
            a.batch = I(); a.seqlen_q = I(); a.seqlen_kv = I(); a.num_kv_heads = H(); a.num_q_heads = Hq(a.num_kv_heads);
            a.head_dim = (rng() % 3) ? 128 : I();
            a.head_dim_v = (rng() & 1) ? 0 : I();
            a.scale = 0.1f;
            a.causal = (int)(rng() & 1);
            a.window_size = (rng() % 4) ? 0 : I();
            a.kv_head_split = (rng() % 4) ? 0 : (rng() & 1) ? heads[rng() % 5] : I();
            a.dq_kernel = (rng() & 1) ? 0 : I();
            int64_t* st[8] = {a.q_stride, a.k_stride, a.v_stride, a.o_stride,
                              a.grad_o_stride, a.grad_q_stride, a.grad_k_stride, a.grad_v_stride};
            for (int64_t* s : st)
                for (int i = 0; i < 3; ++i) s[i] = S();
            if (rng() & 1) a.q_stride[1] = a.grad_o_stride[1] = 2048;   // rows that do not overlap
            if (plan::validate_backward(&a) == FGQA_OK) {
                ++accepted[3];
                (void)plan::validate_backward_pointers(&a);
                const plan::BwdPlan pl = plan::plan_backward(&a, C());
                const int group = a.num_q_heads / a.num_kv_heads;
                CHECK(pl.n_hsplit >= 1 && pl.n_hsplit <= group && group % pl.n_hsplit == 0);
                CHECK(pl.ws_bytes == pl.stat_bytes + pl.part_k_bytes + pl.part_v_bytes);
                (void)plan::check_backward_grid(&a, pl);
            }
        }
        {
            fgqa_sparse_prefill_args a;
            memset(&a, 0, sizeof a);
            a.q = P(); a.k = P(); a.v = P(); a.o = P();
            static int32_t idx[1];
            a.kv_indices = idx;
            a.batch = I(); a.seqlen_q = I(); a.seqlen_kv = I(); a.num_kv_heads = H(); a.num_q_heads = Hq(a.num_kv_heads);
            a.head_dim = (rng() % 4) ? 128 : I();
            a.num_sparse_kv = I();
            a.scale = 0.1f;
            for (int i = 0; i < 3; ++i) {
                a.q_stride[i] = S(); a.k_stride[i] = S(); a.v_stride[i] = S(); a.o_stride[i] = S(); a.idx_stride[i] = S();
            }
            if (plan::validate_sparse(&a) == FGQA_OK) ++accepted[4];
        }
    }
    printf("fuzz: accepted decode %ld, paged %ld, prefill %ld, backward %ld, sparse %ld of %d each\n", accepted[0],
           accepted[1], accepted[2], accepted[3], accepted[4], rounds);
    // the planners saw many accepted calls
    for (long n : accepted) CHECK(n >= rounds / 400);
}

int main() {
    test_decode_known_shapes();
    test_decode_rejections();
    test_decode_extremes();
    test_paged();
    test_prefill_known_shapes();
    test_prefill_rejections();
    test_prefill_padded_head_dims();
    test_backward();
    test_sparse();
    fuzz(20261202u, 200000);
    printf("%ld checks, %ld failed\n", g_checks, g_failed);
    return g_failed ? 1 : 0;
}
