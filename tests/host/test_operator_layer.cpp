// The C++ operator layer (src/cplusplus/FlashGQA/flash_gqa.cpp) over a
// recording stand-in of the C ABI, built by tests/test_host_sanitizers.py with
// g++ and AddressSanitizer + UndefinedBehaviorSanitizer (no recovery).  The
// stand-in validates each call with the library's own host planner
// (cuda_llm_ops_amd/csrc/host/fgqa_plan.cpp, CU count 256) and records the
// argument struct instead of launching, so the test checks what the operator
// entry points hand to the C ABI: tensor strides, the choice between the
// allocation-free and the allocating decode entry, the refusals the layer
// makes itself, and that no argument, however large, overflows on the way.
//
// Output: failed checks, then "N checks, M failed"; exit status 1 on failure.
#include <limits.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <random>

#include "FlashGQA/decode_flash_gqa_kernel.h"
#include "FlashGQA/flash_gqa_backward_kernel.h"
#include "FlashGQA/flash_gqa_forward_kernel.h"
#include "fgqa.h"
#include "fgqa_plan.h"

static long g_checks = 0, g_failed = 0;

#define CHECK(cond)                                                                 \
    do {                                                                            \
        ++g_checks;                                                                 \
        if (!(cond)) {                                                              \
            ++g_failed;                                                             \
            if (g_failed < 50) fprintf(stderr, "%s:%d: %s\n", __FILE__, __LINE__, #cond); \
        }                                                                           \
    } while (0)

// ---------------------------------------------------------------- recording C ABI

static const int kCus = 256;

enum Entry { kNone, kDecode, kDecodeNoalloc, kPaged, kPrefill, kBackward, kSparse };
static Entry g_entry = kNone;
static fgqa_decode_args g_dec;
static fgqa_decode_paged_args g_paged;
static fgqa_prefill_args g_pre;
static fgqa_prefill_backward_args g_bwd;
static fgqa_sparse_prefill_args g_sp;

static void reset() { g_entry = kNone; }

extern "C" {
int fgqa_decode_workspace_bytes(const fgqa_decode_args* a, size_t* bytes) {
    int st = fgqa::plan::validate_decode(a);
    if (st != FGQA_OK) return st;
    fgqa::plan::DecodePlan pl;
    st = fgqa::plan::plan_decode(fgqa::plan::decode_shape(a), kCus, &pl);
    if (st == FGQA_OK) *bytes = pl.ws_bytes;
    return st;
}
static int decode_common(const fgqa_decode_args* a, Entry e) {
    int st = fgqa::plan::validate_decode(a);
    if (st == FGQA_OK) st = fgqa::plan::validate_decode_pointers(a);
    if (st != FGQA_OK) return st;
    g_entry = e;
    g_dec = *a;
    return FGQA_OK;
}
int fgqa_decode_bf16(const fgqa_decode_args* a, void*) { return decode_common(a, kDecode); }
int fgqa_decode_bf16_noalloc(const fgqa_decode_args* a, void*) {
    size_t need = 0;
    const int st = fgqa_decode_workspace_bytes(a, &need);
    if (st != FGQA_OK) return st;
    if (need > FGQA_DECODE_NOALLOC_SCRATCH_BYTES) return FGQA_ERR_WORKSPACE;
    return decode_common(a, kDecodeNoalloc);
}
int fgqa_decode_paged(const fgqa_decode_paged_args* a, void*) {
    int st = fgqa::plan::validate_paged(a);
    if (st == FGQA_OK) st = fgqa::plan::validate_paged_pointers(a);
    if (st != FGQA_OK) return st;
    g_entry = kPaged;
    g_paged = *a;
    return FGQA_OK;
}
int fgqa_prefill_bf16(const fgqa_prefill_args* a, void*) {
    const int st = fgqa::plan::validate_prefill(a);
    if (st != FGQA_OK) return st;
    (void)fgqa::plan::prefill_choice(a, kCus);
    g_entry = kPrefill;
    g_pre = *a;
    return FGQA_OK;
}
int fgqa_prefill_backward_bf16(const fgqa_prefill_backward_args* a, void*) {
    int st = fgqa::plan::validate_backward(a);
    if (st != FGQA_OK) return st;
    st = fgqa::plan::validate_backward_pointers(a);
    if (st != FGQA_OK) return st;
    st = fgqa::plan::check_backward_grid(a, fgqa::plan::plan_backward(a, kCus));
    if (st != FGQA_OK) return st;
    g_entry = kBackward;
    g_bwd = *a;
    return FGQA_OK;
}
int fgqa_sparse_prefill_bf16(const fgqa_sparse_prefill_args* a, void*) {
    const int st = fgqa::plan::validate_sparse(a);
    if (st != FGQA_OK) return st;
    g_entry = kSparse;
    g_sp = *a;
    return FGQA_OK;
}
}

// 16-byte aligned stand-ins: nothing here dereferences a tensor pointer.
template <class T>
static T* fake(uintptr_t n) { return reinterpret_cast<T*>(0x100000 + 256 * n); }

static bool eq3(const int64_t* s, int64_t a, int64_t b, int64_t c) { return s[0] == a && s[1] == b && s[2] == c; }

// ---------------------------------------------------------------- decode

static void test_decode() {
    const bf16_t *q = fake<const bf16_t>(1), *k = fake<const bf16_t>(2), *v = fake<const bf16_t>(3);
    bf16_t* o = fake<bf16_t>(4);
    float* oi = fake<float>(5);
    // config 2: one split per (batch, KV head), no partials: the allocation-free entry
    reset();
    LaunchFlashGqaBf16Kernel(q, k, v, 0.088f, o, oi, 60, 4096, 128, 8, 128);
    CHECK(FlashGqaGetLastStatus() == FGQA_OK);
    CHECK(g_entry == kDecodeNoalloc);
    CHECK(g_dec.batch == 60 && g_dec.max_seqlen == 4096 && g_dec.num_q_heads == 128 && g_dec.num_kv_heads == 8);
    CHECK(g_dec.q_stride[0] == 128 * 128 && g_dec.q_stride[1] == 128);
    CHECK(eq3(g_dec.k_stride, 4096 * 8 * 128, 8 * 128, 128) && eq3(g_dec.v_stride, 4096 * 8 * 128, 8 * 128, 128));
    CHECK(g_dec.o_stride[0] == 128 * 128 && g_dec.o_stride[1] == 128);
    CHECK(g_dec.seqlens == nullptr && g_dec.workspace == nullptr && g_dec.workspace_bytes == 0);
    CHECK(g_dec.q == q && g_dec.k == k && g_dec.v == v && g_dec.o == o);
    // ragged, config 3 (17 MB of partials): still the fixed scratch
    const int32_t* lens = fake<const int32_t>(6);
    reset();
    LaunchFlashGqaBf16KernelVarlen(q, k, v, 0.088f, o, lens, 64, 32768, 64, 8, 128);
    CHECK(FlashGqaGetLastStatus() == FGQA_OK && g_entry == kDecodeNoalloc && g_dec.seqlens == lens);
    // ragged 256 x 16384 x 64 heads: 4 splits x 256 x 64 x 512 B = 32 MiB of
    // partial O, with (max, sum) and the list beyond the 32 MiB scratch: the
    // allocating entry
    reset();
    LaunchFlashGqaBf16KernelVarlen(q, k, v, 0.088f, o, lens, 256, 16384, 64, 8, 128);
    CHECK(FlashGqaGetLastStatus() == FGQA_OK && g_entry == kDecode);
    // the reference's early return: no launch, no error for empty shapes
    reset();
    LaunchFlashGqaBf16Kernel(q, k, v, 0.088f, o, oi, 0, 4096, 128, 8, 128);
    CHECK(FlashGqaGetLastStatus() == FGQA_OK && g_entry == kNone);
    LaunchFlashGqaBf16Kernel(q, k, v, 0.088f, o, oi, -1, 4096, 128, 8, 128);
    CHECK(FlashGqaGetLastStatus() == FGQA_ERR_INVALID_ARGUMENT && g_entry == kNone);
    // unsupported head dim: refused by validation
    LaunchFlashGqaBf16Kernel(q, k, v, 0.088f, o, oi, 2, 512, 16, 2, 64);
    CHECK(FlashGqaGetLastStatus() == FGQA_ERR_UNSUPPORTED && g_entry == kNone);
    // INT_MAX sizes: the stride product saturates, validation refuses
    LaunchFlashGqaBf16Kernel(q, k, v, 0.088f, o, oi, 2, INT_MAX, 16, INT_MAX / 128 * 128, 128);
    CHECK(FlashGqaGetLastStatus() != FGQA_OK && g_entry == kNone);
}

static void test_paged() {
    const bf16_t* q = fake<const bf16_t>(1);
    bf16_t* o = fake<bf16_t>(2);
    const void *kc = fake<const void>(3), *vc = fake<const void>(4);
    const int32_t *bt = fake<const int32_t>(5), *lens = fake<const int32_t>(6);
    reset();
    LaunchFlashGqaBf16KernelPaged(q, kc, vc, true, 0.088f, 0.5f, 0.25f, o, bt, lens, 64, 2048, 16, 64 * 2048, 64, 8,
                                  128);
    CHECK(FlashGqaGetLastStatus() == FGQA_OK && g_entry == kPaged);
    CHECK(g_paged.max_seqlen == 32768 && g_paged.block_table_stride == 2048 && g_paged.page_size == 16);
    CHECK(g_paged.kv_dtype == FGQA_KV_FP8_E4M3 && g_paged.k_scale == 0.5f && g_paged.v_scale == 0.25f);
    CHECK(eq3(g_paged.k_stride, 16 * 8 * 128, 8 * 128, 128) && eq3(g_paged.v_stride, 16 * 8 * 128, 8 * 128, 128));
    // pages x page size past INT_MAX tokens: refused here, nothing called
    reset();
    LaunchFlashGqaBf16KernelPaged(q, kc, vc, false, 0.088f, 1.f, 1.f, o, bt, lens, 4, 1 << 20, 1 << 12, 1 << 20, 16,
                                  2, 128);
    CHECK(FlashGqaGetLastStatus() == FGQA_ERR_UNSUPPORTED && g_entry == kNone);
    LaunchFlashGqaBf16KernelPaged(q, kc, vc, false, 0.088f, 1.f, 1.f, o, bt, lens, 4, INT_MAX, INT_MAX, INT_MAX, 16,
                                  2, 128);
    CHECK(FlashGqaGetLastStatus() == FGQA_ERR_UNSUPPORTED && g_entry == kNone);
}

// ---------------------------------------------------------------- prefill, backward, sparse

static void test_prefill() {
    const bf16_t *q = fake<const bf16_t>(1), *k = fake<const bf16_t>(2), *v = fake<const bf16_t>(3);
    bf16_t* o = fake<bf16_t>(4);
    float* lse = fake<float>(5);
    // config 4, BSHD
    reset();
    LaunchFlashGqaForwardBf16Kernel(q, k, v, 0.088f, o, lse, 1, 4096, 4096, 16, 1, 128, true);
    CHECK(FlashGqaGetLastStatus() == FGQA_OK && g_entry == kPrefill);
    CHECK(eq3(g_pre.q_stride, 4096 * 16 * 128, 16 * 128, 128) && eq3(g_pre.o_stride, 4096 * 16 * 128, 16 * 128, 128));
    CHECK(eq3(g_pre.k_stride, 4096 * 128, 128, 128) && eq3(g_pre.v_stride, 4096 * 128, 128, 128));
    CHECK(g_pre.causal == 1 && g_pre.window_size == 0 && g_pre.sink == nullptr && g_pre.kernel == FGQA_KERNEL_AUTO);
    CHECK(g_pre.workspace == nullptr && g_pre.workspace_bytes == 0 && g_pre.lse == lse);
    // config 5
    reset();
    LaunchFlashGqaForwardBf16Kernel(q, k, v, 0.088f, o, lse, 4, 16384, 16384, 32, 8, 128, true);
    CHECK(FlashGqaGetLastStatus() == FGQA_OK && g_entry == kPrefill);
    CHECK(eq3(g_pre.k_stride, (int64_t)16384 * 8 * 128, 8 * 128, 128));
    // strided: null stride arrays are refused here
    reset();
    LaunchFlashGqaForwardBf16KernelStrided(q, k, v, 0.088f, o, lse, 1, 64, 64, 2, 1, 128, false, nullptr, nullptr,
                                           nullptr, nullptr);
    CHECK(FlashGqaGetLastStatus() == FGQA_ERR_INVALID_ARGUMENT && g_entry == kNone);
    // sliding window: window 0 is refused (0 means "none" in the C ABI)
    const float* sink = fake<const float>(6);
    reset();
    LaunchFlashSwaForwardBf16Kernel(q, k, v, 0.088f, o, lse, 1, 4096, 4096, 16, 1, 128, 512, sink);
    CHECK(FlashGqaGetLastStatus() == FGQA_OK && g_entry == kPrefill && g_pre.window_size == 512 && g_pre.sink == sink);
    reset();
    LaunchFlashSwaForwardBf16Kernel(q, k, v, 0.088f, o, lse, 1, 4096, 4096, 16, 1, 128, 0, nullptr);
    CHECK(FlashGqaGetLastStatus() == FGQA_ERR_INVALID_ARGUMENT && g_entry == kNone);
    // MLA (192, 128)
    reset();
    LaunchFlashMlaForwardBf16Kernel(q, k, v, 0.088f, o, lse, 1, 4096, 4096, 16, 1, 192, 128, true);
    CHECK(FlashGqaGetLastStatus() == FGQA_OK && g_entry == kPrefill);
    CHECK(eq3(g_pre.q_stride, 4096 * 16 * 192, 16 * 192, 192) && eq3(g_pre.k_stride, 4096 * 192, 192, 192));
    CHECK(eq3(g_pre.v_stride, 4096 * 128, 128, 128) && eq3(g_pre.o_stride, 4096 * 16 * 128, 16 * 128, 128));
    CHECK(g_pre.head_dim == 192 && g_pre.head_dim_v == 128);
    reset();
    LaunchFlashMlaForwardBf16Kernel(q, k, v, 0.088f, o, lse, 1, 4096, 4096, 16, 1, 192, 0, true);
    CHECK(FlashGqaGetLastStatus() == FGQA_ERR_INVALID_ARGUMENT && g_entry == kNone);
    // INT_MAX sizes: saturated strides, refused
    reset();
    LaunchFlashGqaForwardBf16Kernel(q, k, v, 0.088f, o, lse, 1, INT_MAX, INT_MAX, INT_MAX, 1, 128, true);
    CHECK(FlashGqaGetLastStatus() != FGQA_OK && g_entry == kNone);
}

static void test_backward_and_sparse() {
    const bf16_t *q = fake<const bf16_t>(1), *k = fake<const bf16_t>(2), *v = fake<const bf16_t>(3),
                 *o = fake<const bf16_t>(4), *go = fake<const bf16_t>(5);
    bf16_t *gq = fake<bf16_t>(6), *gk = fake<bf16_t>(7), *gv = fake<bf16_t>(8);
    const float* lse = fake<const float>(9);
    reset();
    LaunchFlashGqaBackwardBf16Kernel(q, k, v, o, lse, go, 0.088f, gq, gk, gv, 1, 4096, 4096, 16, 1, 128, true);
    CHECK(FlashGqaGetLastStatus() == FGQA_OK && g_entry == kBackward);
    CHECK(eq3(g_bwd.q_stride, 4096 * 16 * 128, 16 * 128, 128) && eq3(g_bwd.grad_q_stride, 4096 * 16 * 128, 16 * 128, 128));
    CHECK(eq3(g_bwd.grad_k_stride, 4096 * 128, 128, 128) && eq3(g_bwd.grad_v_stride, 4096 * 128, 128, 128));
    CHECK(g_bwd.window_size == 0 && g_bwd.head_dim_v == 128);
    reset();
    LaunchFlashSwaBackwardBf16Kernel(q, k, v, o, lse, go, 0.088f, gq, gk, gv, 1, 4096, 4096, 16, 1, 128, 512);
    CHECK(FlashGqaGetLastStatus() == FGQA_OK && g_entry == kBackward && g_bwd.window_size == 512 && g_bwd.causal == 1);
    reset();
    LaunchFlashMlaBackwardBf16Kernel(q, k, v, o, lse, go, 0.088f, gq, gk, gv, 1, 4096, 4096, 16, 1, 192, 128, true);
    CHECK(FlashGqaGetLastStatus() == FGQA_OK && g_entry == kBackward);
    CHECK(eq3(g_bwd.o_stride, 4096 * 16 * 128, 16 * 128, 128) && eq3(g_bwd.k_stride, 4096 * 192, 192, 192));
    reset();
    LaunchFlashGqaBackwardBf16Kernel(q, k, v, o, lse, go, 0.088f, gq, gk, gv, INT_MAX, INT_MAX, INT_MAX, INT_MAX, 1,
                                     128, true);
    CHECK(FlashGqaGetLastStatus() != FGQA_OK && g_entry == kNone);

    const int32_t* idx = fake<const int32_t>(10);
    bf16_t* os = fake<bf16_t>(11);
    float* ls = fake<float>(12);
    reset();
    LaunchFlashSgqaForwardBf16Kernel(q, k, v, idx, 2048, 0.088f, os, ls, 1, 4096, 4096, 16, 1, 128, true);
    CHECK(FlashGqaGetLastStatus() == FGQA_OK && g_entry == kSparse);
    CHECK(eq3(g_sp.idx_stride, 4096 * 2048, 4096 * 2048, 2048) && g_sp.num_sparse_kv == 2048);
    reset();
    LaunchFlashSgqaForwardBf16Kernel(q, k, v, idx, INT_MAX, 0.088f, os, ls, 1, INT_MAX, 4096, 16, INT_MAX, 128, true);
    CHECK(FlashGqaGetLastStatus() != FGQA_OK && g_entry == kNone);
}

// ---------------------------------------------------------------- fuzz

static void fuzz(unsigned seed, int rounds) {
    std::mt19937_64 rng(seed);
    const int ints[] = {0, 1, 2, 8, 16, 64, 127, 128, 129, 192, 4096, 32768, 1 << 20, 1 << 30, INT_MAX, -1, INT_MIN};
    auto I = [&]() { return ints[rng() % (sizeof ints / sizeof ints[0])]; };
    const bf16_t* t = fake<const bf16_t>(1);
    bf16_t* w = fake<bf16_t>(2);
    float* f = fake<float>(3);
    const int32_t* ii = fake<const int32_t>(4);
    long accepted = 0;
    for (int r = 0; r < rounds; ++r) {
        reset();
        switch (rng() % 9) {
            case 0: LaunchFlashGqaBf16Kernel(t, t, t, 0.1f, w, f, I(), I(), I(), I(), I()); break;
            case 1: LaunchFlashGqaBf16KernelVarlen(t, t, t, 0.1f, w, ii, I(), I(), I(), I(), I()); break;
            case 2:
                LaunchFlashGqaBf16KernelPaged(t, t, t, rng() & 1, 0.1f, 1.f, 1.f, w, ii, ii, I(), I(), I(), I(), I(),
                                              I(), I());
                break;
            case 3: LaunchFlashGqaForwardBf16Kernel(t, t, t, 0.1f, w, f, I(), I(), I(), I(), I(), I(), rng() & 1); break;
            case 4: LaunchFlashSwaForwardBf16Kernel(t, t, t, 0.1f, w, f, I(), I(), I(), I(), I(), I(), I(), nullptr); break;
            case 5:
                LaunchFlashMlaForwardBf16Kernel(t, t, t, 0.1f, w, f, I(), I(), I(), I(), I(), I(), I(), rng() & 1);
                break;
            case 6:
                LaunchFlashGqaBackwardBf16Kernel(t, t, t, t, f, t, 0.1f, w, w, w, I(), I(), I(), I(), I(), I(),
                                                 rng() & 1);
                break;
            case 7:
                LaunchFlashMlaBackwardBf16Kernel(t, t, t, t, f, t, 0.1f, w, w, w, I(), I(), I(), I(), I(), I(), I(),
                                                 rng() & 1);
                break;
            default:
                LaunchFlashSgqaForwardBf16Kernel(t, t, t, ii, I(), 0.1f, w, f, I(), I(), I(), I(), I(), I(), rng() & 1);
                break;
        }
        const int st = FlashGqaGetLastStatus();
        CHECK(st == FGQA_OK || st == FGQA_ERR_INVALID_ARGUMENT || st == FGQA_ERR_UNSUPPORTED);
        // a call reaches the C ABI's launch only when it returns OK
        CHECK((st == FGQA_OK) || g_entry == kNone);
        accepted += g_entry != kNone;
    }
    printf("fuzz: %ld of %d operator calls reached a launch\n", accepted, rounds);
    CHECK(accepted > 0);
}

int main() {
    test_decode();
    test_paged();
    test_prefill();
    test_backward_and_sparse();
    fuzz(7u, 200000);
    printf("%ld checks, %ld failed\n", g_checks, g_failed);
    return g_failed ? 1 : 0;
}
