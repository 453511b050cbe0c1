// C++ operator entry points of the FlashGQA path, implemented over the C ABI
// (include/fgqa.h).  Host-only C++: no HIP types or calls in this file.
#include <climits>
#include <cstdint>
#include <cstring>

#include "FlashGQA/decode_flash_gqa_kernel.h"
#include "FlashGQA/flash_gqa_backward_kernel.h"
#include "FlashGQA/flash_gqa_forward_kernel.h"
#include "fgqa.h"

namespace {
thread_local int g_last_status = FGQA_OK;

// a * b * c, or INT64_MAX when the product overflows: the C ABI refuses such
// a stride (FGQA_ERR_UNSUPPORTED) instead of the product wrapping around.
int64_t mul3(int64_t a, int64_t b, int64_t c) {
    int64_t ab = 0, abc = 0;
    if (__builtin_mul_overflow(a, b, &ab) || __builtin_mul_overflow(ab, c, &abc)) return INT64_MAX;
    return abc;
}

fgqa_decode_args contiguous_decode(const bf16_t* q, const bf16_t* k, const bf16_t* v, float scale, bf16_t* o,
                                   int batchSize, int seqLength, int numQueryHeads, int numKvHeads, int headDim) {
    fgqa_decode_args a;
    std::memset(&a, 0, sizeof(a));
    a.q = q;
    a.k = k;
    a.v = v;
    a.o = o;
    a.batch = batchSize;
    a.max_seqlen = seqLength;
    a.num_q_heads = numQueryHeads;
    a.num_kv_heads = numKvHeads;
    a.head_dim = headDim;
    a.scale = scale;
    // q, o: [B, Hq, D];  k, v: [B, S, Hkv, D]
    a.q_stride[0] = (int64_t)numQueryHeads * headDim;
    a.q_stride[1] = headDim;
    a.o_stride[0] = a.q_stride[0];
    a.o_stride[1] = a.q_stride[1];
    a.k_stride[0] = mul3(seqLength, numKvHeads, headDim);
    a.k_stride[1] = (int64_t)numKvHeads * headDim;
    a.k_stride[2] = headDim;
    for (int i = 0; i < 3; ++i) a.v_stride[i] = a.k_stride[i];
    return a;
}
}  // namespace

void LaunchFlashGqaBf16Kernel(const bf16_t* q, const bf16_t* k, const bf16_t* v, float scale, bf16_t* o,
                              float* oIntermediate, int batchSize, int seqLength, int numQueryHeads,
                              int numKvHeads, int headDim) {
    // The reference returns before launching when batchSize or seqLength is
    // not positive (decode_flash_gqa_kernel.cu:416-418); so does the drop-in.
    if (batchSize <= 0 || seqLength <= 0) {
        g_last_status = (batchSize < 0 || seqLength < 0) ? FGQA_ERR_INVALID_ARGUMENT : FGQA_OK;
        return;
    }
    fgqa_decode_args a =
        contiguous_decode(q, k, v, scale, o, batchSize, seqLength, numQueryHeads, numKvHeads, headDim);
    // The split partials (two or more fp32 rows per query head, with their
    // max and sum) never fit in oIntermediate's batchSize * numQueryHeads *
    // headDim floats, so they go to the library's fixed device scratch: the
    // call allocates nothing and does not synchronize.  Only a plan beyond
    // that scratch falls back to the library's cached buffer.
    (void)oIntermediate;
    size_t need = 0;
    int st = fgqa_decode_workspace_bytes(&a, &need);
    if (st == FGQA_OK)
        st = need <= FGQA_DECODE_NOALLOC_SCRATCH_BYTES ? fgqa_decode_bf16_noalloc(&a, nullptr)
                                                        : fgqa_decode_bf16(&a, nullptr);
    g_last_status = st;
}

void LaunchFlashGqaBf16KernelVarlen(const bf16_t* q, const bf16_t* k, const bf16_t* v, float scale, bf16_t* o,
                                    const int32_t* seqLengths, int batchSize, int maxSeqLength, int numQueryHeads,
                                    int numKvHeads, int headDim) {
    fgqa_decode_args a =
        contiguous_decode(q, k, v, scale, o, batchSize, maxSeqLength, numQueryHeads, numKvHeads, headDim);
    a.seqlens = seqLengths;
    // split partials and the ragged work list in the fixed device scratch, as above
    size_t need = 0;
    int st = fgqa_decode_workspace_bytes(&a, &need);
    if (st == FGQA_OK)
        st = need <= FGQA_DECODE_NOALLOC_SCRATCH_BYTES ? fgqa_decode_bf16_noalloc(&a, nullptr)
                                                        : fgqa_decode_bf16(&a, nullptr);
    g_last_status = st;
}

void LaunchFlashGqaBf16KernelPaged(const bf16_t* q, const void* kCache, const void* vCache, bool kvFp8, float scale,
                                   float kScale, float vScale, bf16_t* o, const int32_t* blockTable,
                                   const int32_t* seqLengths, int batchSize, int maxPagesPerSeq, int pageSize,
                                   int numPages, int numQueryHeads, int numKvHeads, int headDim) {
    fgqa_decode_paged_args a;
    std::memset(&a, 0, sizeof(a));
    a.q = q;
    a.k_cache = kCache;
    a.v_cache = vCache;
    a.o = o;
    a.block_table = blockTable;
    a.seqlens = seqLengths;
    a.batch = batchSize;
    const int64_t max_tokens = (maxPagesPerSeq > 0 && pageSize > 0) ? (int64_t)maxPagesPerSeq * pageSize : 0;
    if (max_tokens > INT_MAX) {   // the C ABI's max_seqlen is an int
        g_last_status = FGQA_ERR_UNSUPPORTED;
        return;
    }
    a.max_seqlen = (int)max_tokens;
    a.num_q_heads = numQueryHeads;
    a.num_kv_heads = numKvHeads;
    a.head_dim = headDim;
    a.page_size = pageSize;
    a.num_pages = numPages;
    a.kv_dtype = kvFp8 ? FGQA_KV_FP8_E4M3 : FGQA_KV_BF16;
    a.scale = scale;
    a.k_scale = kScale;
    a.v_scale = vScale;
    // q, o: [B, Hq, D];  caches: [numPages, pageSize, Hkv, D]
    a.q_stride[0] = (int64_t)numQueryHeads * headDim;
    a.q_stride[1] = headDim;
    a.o_stride[0] = a.q_stride[0];
    a.o_stride[1] = a.q_stride[1];
    a.k_stride[0] = mul3(pageSize, numKvHeads, headDim);
    a.k_stride[1] = (int64_t)numKvHeads * headDim;
    a.k_stride[2] = headDim;
    for (int i = 0; i < 3; ++i) a.v_stride[i] = a.k_stride[i];
    a.block_table_stride = maxPagesPerSeq;
    g_last_status = fgqa_decode_paged(&a, nullptr);
}

void LaunchFlashGqaForwardBf16KernelStrided(const bf16_t* q, const bf16_t* k, const bf16_t* v, float scale,
                                            bf16_t* o, float* lse, int batchSize, int seqLengthQ, int seqLengthKv,
                                            int numQueryHeads, int numKvHeads, int headDim, bool causal,
                                            const int64_t qStride[3], const int64_t kStride[3],
                                            const int64_t vStride[3], const int64_t oStride[3]) {
    if (qStride == nullptr || kStride == nullptr || vStride == nullptr || oStride == nullptr) {
        g_last_status = FGQA_ERR_INVALID_ARGUMENT;
        return;
    }
    fgqa_prefill_args a;
    std::memset(&a, 0, sizeof(a));
    a.q = q;
    a.k = k;
    a.v = v;
    a.o = o;
    a.lse = lse;
    a.batch = batchSize;
    a.seqlen_q = seqLengthQ;
    a.seqlen_kv = seqLengthKv;
    a.num_q_heads = numQueryHeads;
    a.num_kv_heads = numKvHeads;
    a.head_dim = headDim;
    a.causal = causal ? 1 : 0;
    a.scale = scale;
    for (int i = 0; i < 3; ++i) {
        a.q_stride[i] = qStride[i];
        a.k_stride[i] = kStride[i];
        a.v_stride[i] = vStride[i];
        a.o_stride[i] = oStride[i];
    }
    g_last_status = fgqa_prefill_bf16(&a, nullptr);
}

void LaunchFlashGqaForwardBf16Kernel(const bf16_t* q, const bf16_t* k, const bf16_t* v, float scale, bf16_t* o,
                                     float* lse, int batchSize, int seqLengthQ, int seqLengthKv, int numQueryHeads,
                                     int numKvHeads, int headDim, bool causal) {
    // BSHD: q, o [B, Sq, Hq, D]; k, v [B, Skv, Hkv, D]
    const int64_t qs[3] = {mul3(seqLengthQ, numQueryHeads, headDim), (int64_t)numQueryHeads * headDim, headDim};
    const int64_t ks[3] = {mul3(seqLengthKv, numKvHeads, headDim), (int64_t)numKvHeads * headDim, headDim};
    LaunchFlashGqaForwardBf16KernelStrided(q, k, v, scale, o, lse, batchSize, seqLengthQ, seqLengthKv,
                                           numQueryHeads, numKvHeads, headDim, causal, qs, ks, ks, qs);
}

static void backward_bshd(const bf16_t* q, const bf16_t* k, const bf16_t* v, const bf16_t* o, const float* lse,
                          const bf16_t* gradO, float scale, bf16_t* gradQ, bf16_t* gradK, bf16_t* gradV,
                          int batchSize, int seqLengthQ, int seqLengthKv, int numQueryHeads, int numKvHeads,
                          int headDim, int headDimV, bool causal, int windowSize) {
    fgqa_prefill_backward_args a;
    std::memset(&a, 0, sizeof(a));
    a.q = q;
    a.k = k;
    a.v = v;
    a.o = o;
    a.lse = lse;
    a.grad_o = gradO;
    a.grad_q = gradQ;
    a.grad_k = gradK;
    a.grad_v = gradV;
    a.batch = batchSize;
    a.seqlen_q = seqLengthQ;
    a.seqlen_kv = seqLengthKv;
    a.num_q_heads = numQueryHeads;
    a.num_kv_heads = numKvHeads;
    a.head_dim = headDim;
    a.causal = causal ? 1 : 0;
    a.scale = scale;
    a.window_size = windowSize;
    a.head_dim_v = headDimV;
    // BSHD: q, gradQ [B, Sq, Hq, D]; o, gradO [B, Sq, Hq, Dv]; k, gradK [B, Skv, Hkv, D];
    // v, gradV [B, Skv, Hkv, Dv]
    const int64_t qs[3] = {mul3(seqLengthQ, numQueryHeads, headDim), (int64_t)numQueryHeads * headDim, headDim};
    const int64_t os[3] = {mul3(seqLengthQ, numQueryHeads, headDimV), (int64_t)numQueryHeads * headDimV, headDimV};
    const int64_t ks[3] = {mul3(seqLengthKv, numKvHeads, headDim), (int64_t)numKvHeads * headDim, headDim};
    const int64_t vs[3] = {mul3(seqLengthKv, numKvHeads, headDimV), (int64_t)numKvHeads * headDimV, headDimV};
    for (int i = 0; i < 3; ++i) {
        a.q_stride[i] = a.grad_q_stride[i] = qs[i];
        a.o_stride[i] = a.grad_o_stride[i] = os[i];
        a.k_stride[i] = a.grad_k_stride[i] = ks[i];
        a.v_stride[i] = a.grad_v_stride[i] = vs[i];
    }
    g_last_status = fgqa_prefill_backward_bf16(&a, nullptr);
}

void LaunchFlashGqaBackwardBf16Kernel(const bf16_t* q, const bf16_t* k, const bf16_t* v, const bf16_t* o,
                                      const float* lse, const bf16_t* gradO, float scale, bf16_t* gradQ,
                                      bf16_t* gradK, bf16_t* gradV, int batchSize, int seqLengthQ, int seqLengthKv,
                                      int numQueryHeads, int numKvHeads, int headDim, bool causal) {
    backward_bshd(q, k, v, o, lse, gradO, scale, gradQ, gradK, gradV, batchSize, seqLengthQ, seqLengthKv,
                  numQueryHeads, numKvHeads, headDim, headDim, causal, 0);
}

void LaunchFlashMlaBackwardBf16Kernel(const bf16_t* q, const bf16_t* k, const bf16_t* v, const bf16_t* o,
                                      const float* lse, const bf16_t* gradO, float scale, bf16_t* gradQ,
                                      bf16_t* gradK, bf16_t* gradV, int batchSize, int seqLengthQ, int seqLengthKv,
                                      int numQueryHeads, int numKvHeads, int headDimQk, int headDimV, bool causal) {
    backward_bshd(q, k, v, o, lse, gradO, scale, gradQ, gradK, gradV, batchSize, seqLengthQ, seqLengthKv,
                  numQueryHeads, numKvHeads, headDimQk, headDimV, causal, 0);
}

void LaunchFlashSwaBackwardBf16Kernel(const bf16_t* q, const bf16_t* k, const bf16_t* v, const bf16_t* o,
                                      const float* lse, const bf16_t* gradO, float scale, bf16_t* gradQ,
                                      bf16_t* gradK, bf16_t* gradV, int batchSize, int seqLengthQ, int seqLengthKv,
                                      int numQueryHeads, int numKvHeads, int headDim, int windowSize) {
    backward_bshd(q, k, v, o, lse, gradO, scale, gradQ, gradK, gradV, batchSize, seqLengthQ, seqLengthKv,
                  numQueryHeads, numKvHeads, headDim, headDim, true, windowSize);
}

void LaunchFlashSwaForwardBf16Kernel(const bf16_t* q, const bf16_t* k, const bf16_t* v, float scale, bf16_t* o,
                                     float* lse, int batchSize, int seqLengthQ, int seqLengthKv, int numQueryHeads,
                                     int numKvHeads, int headDim, int windowSize, const float* sink) {
    fgqa_prefill_args a;
    std::memset(&a, 0, sizeof(a));
    a.q = q;
    a.k = k;
    a.v = v;
    a.o = o;
    a.lse = lse;
    a.batch = batchSize;
    a.seqlen_q = seqLengthQ;
    a.seqlen_kv = seqLengthKv;
    a.num_q_heads = numQueryHeads;
    a.num_kv_heads = numKvHeads;
    a.head_dim = headDim;
    a.causal = 1;
    a.scale = scale;
    const int64_t qs[3] = {mul3(seqLengthQ, numQueryHeads, headDim), (int64_t)numQueryHeads * headDim, headDim};
    const int64_t ks[3] = {mul3(seqLengthKv, numKvHeads, headDim), (int64_t)numKvHeads * headDim, headDim};
    for (int i = 0; i < 3; ++i) {
        a.q_stride[i] = a.o_stride[i] = qs[i];
        a.k_stride[i] = a.v_stride[i] = ks[i];
    }
    // the window must be positive here (0 means "no window" in the C ABI)
    if (windowSize <= 0) {
        g_last_status = FGQA_ERR_INVALID_ARGUMENT;
        return;
    }
    a.window_size = windowSize;
    a.sink = sink;
    g_last_status = fgqa_prefill_bf16(&a, nullptr);
}

void LaunchFlashMlaForwardBf16Kernel(const bf16_t* q, const bf16_t* k, const bf16_t* v, float scale, bf16_t* o,
                                     float* lse, int batchSize, int seqLengthQ, int seqLengthKv, int numQueryHeads,
                                     int numKvHeads, int headDimQk, int headDimV, bool causal) {
    fgqa_prefill_args a;
    std::memset(&a, 0, sizeof(a));
    a.q = q;
    a.k = k;
    a.v = v;
    a.o = o;
    a.lse = lse;
    a.batch = batchSize;
    a.seqlen_q = seqLengthQ;
    a.seqlen_kv = seqLengthKv;
    a.num_q_heads = numQueryHeads;
    a.num_kv_heads = numKvHeads;
    a.head_dim = headDimQk;
    a.head_dim_v = headDimV;
    a.causal = causal ? 1 : 0;
    a.scale = scale;
    if (headDimV <= 0) {   // 0 would mean "same as headDimQk" in the C ABI
        g_last_status = FGQA_ERR_INVALID_ARGUMENT;
        return;
    }
    a.q_stride[0] = mul3(seqLengthQ, numQueryHeads, headDimQk);
    a.q_stride[1] = (int64_t)numQueryHeads * headDimQk;
    a.q_stride[2] = headDimQk;
    a.k_stride[0] = mul3(seqLengthKv, numKvHeads, headDimQk);
    a.k_stride[1] = (int64_t)numKvHeads * headDimQk;
    a.k_stride[2] = headDimQk;
    a.v_stride[0] = mul3(seqLengthKv, numKvHeads, headDimV);
    a.v_stride[1] = (int64_t)numKvHeads * headDimV;
    a.v_stride[2] = headDimV;
    a.o_stride[0] = mul3(seqLengthQ, numQueryHeads, headDimV);
    a.o_stride[1] = (int64_t)numQueryHeads * headDimV;
    a.o_stride[2] = headDimV;
    g_last_status = fgqa_prefill_bf16(&a, nullptr);
}

void LaunchFlashSgqaForwardBf16Kernel(const bf16_t* q, const bf16_t* k, const bf16_t* v, const int32_t* kvIndices,
                                      int numSparseKv, float scale, bf16_t* o, float* lse, int batchSize,
                                      int seqLengthQ, int seqLengthKv, int numQueryHeads, int numKvHeads, int headDim,
                                      bool causal) {
    fgqa_sparse_prefill_args a;
    std::memset(&a, 0, sizeof(a));
    a.q = q;
    a.k = k;
    a.v = v;
    a.o = o;
    a.lse = lse;
    a.kv_indices = kvIndices;
    a.batch = batchSize;
    a.seqlen_q = seqLengthQ;
    a.seqlen_kv = seqLengthKv;
    a.num_q_heads = numQueryHeads;
    a.num_kv_heads = numKvHeads;
    a.head_dim = headDim;
    a.num_sparse_kv = numSparseKv;
    a.causal = causal ? 1 : 0;
    a.scale = scale;
    const int64_t qs[3] = {mul3(seqLengthQ, numQueryHeads, headDim), (int64_t)numQueryHeads * headDim, headDim};
    const int64_t ks[3] = {mul3(seqLengthKv, numKvHeads, headDim), (int64_t)numKvHeads * headDim, headDim};
    for (int i = 0; i < 3; ++i) {
        a.q_stride[i] = a.o_stride[i] = qs[i];
        a.k_stride[i] = a.v_stride[i] = ks[i];
    }
    a.idx_stride[0] = mul3(numKvHeads, seqLengthQ, numSparseKv);
    a.idx_stride[1] = (int64_t)seqLengthQ * numSparseKv;
    a.idx_stride[2] = numSparseKv;
    g_last_status = fgqa_sparse_prefill_bf16(&a, nullptr);
}

int FlashGqaGetLastStatus() { return g_last_status; }
