/*
 * fgqa.h -- C ABI of the MI355X (gfx950) flash grouped-query attention library
 * (libfgqa.so).  Plain pointers, sizes and a status code; no C++ or HIP types.
 *
 * The C++ operator entry points in include/cplusplus/ are thin wrappers over
 * these functions.  An FFI (ctypes, cgo, JNI, N-API) binds these directly.
 *
 * Conventions
 *   - bf16 tensors are passed as `const void*` / `void*` device pointers to
 *     bfloat16 values (2 bytes, upper half of IEEE binary32).
 *   - Strides are in ELEMENTS; the head dimension is always contiguous.
 *     Base pointers must be 16-byte aligned and every stride a multiple of 8.
 *   - `stream` is a hipStream_t (NULL = the default stream).  Launches are
 *     asynchronous; the functions never synchronise the device.
 *   - Supported: head_dim == 128; decode needs num_q_heads / num_kv_heads <= 16.
 *     Sequence strides should be at least head_dim (rows do not overlap).
 *   - Every entry point returns FGQA_OK (0) or a negative fgqa_status; nothing
 *     is launched when the status is not FGQA_OK.  No exception crosses the ABI.
 */
#ifndef FGQA_H
#define FGQA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum fgqa_status {
    FGQA_OK = 0,
    FGQA_ERR_INVALID_ARGUMENT = -1, /* null pointer, negative size, Hq % Hkv != 0 ... */
    FGQA_ERR_UNSUPPORTED = -2,      /* valid but not implemented: head_dim, group size, alignment,
                                       sequence lengths above 2^30, grids of 2^31 workgroups or more,
                                       one sequence's K/V/Q span reaching 2 GiB */
    FGQA_ERR_WORKSPACE = -3,        /* caller workspace smaller than fgqa_decode_workspace_bytes */
    FGQA_ERR_HIP = -4               /* a HIP runtime call or kernel launch failed */
};

/*
 * Kernel choice of the prefill and backward calls (fields `kernel` and
 * `dq_kernel`).  AUTO picks by grid size; the others force one kernel shape,
 * for tuning and tests.  Callers that zero the argument struct get AUTO.
 *   FGQA_KERNEL_WHOLE  one workgroup runs a 128-row unit over its whole KV range
 *   FGQA_KERNEL_SPLIT  two wave groups run the two halves of a unit's KV range
 *                      and merge (the choice for causal grids under 2 units
 *                      per CU and non-causal grids under 4)
 *   FGQA_KERNEL_WIDE   (prefill forward) two wave groups
 *                      share each K/V tile of a 256-row unit.  With at most
 *                      one unit pair per two CUs (and at most 128 pairs) a
 *                      unit's KV range may be split over two workgroups that
 *                      merge through device memory the library holds (calls
 *                      that overlap on one device must not both use it);
 *                      larger grids run whole units on a persistent grid
 *                      (AUTO's choice for causal grids without a window or
 *                      sink from 2 units per CU)
 *   FGQA_KERNEL_TALL   (prefill forward, head_dim 128, no window or sink) the
 *                      256-row units of FGQA_KERNEL_WIDE on four waves of 64
 *                      rows each, one wave per SIMD, each K/V operand read
 *                      from LDS feeding two MFMAs; the same unit pairs and
 *                      merge scratch, or whole units on a persistent grid
 */
enum fgqa_kernel_choice {
    FGQA_KERNEL_AUTO = 0,
    FGQA_KERNEL_WHOLE = 1,
    FGQA_KERNEL_SPLIT = 2,
    FGQA_KERNEL_WIDE = 3,
    FGQA_KERNEL_TALL = 4
};

/*
 * Single-token decode (flash-decoding: split-KV pass + log-sum-exp combine).
 * Replaces LaunchFlashGqaBf16Kernel, reference
 * include/cplusplus/FlashGQA/decode_flash_gqa_kernel.cuh:28-38
 * (definition src/cplusplus/FlashGQA/decode_flash_gqa_kernel.cu:405-470).
 *
 *   q  [B, Hq, D]           strides q_stride  = {b, h}
 *   k  [B, S_max, Hkv, D]   strides k_stride  = {b, s, h}   (reference layout)
 *   v  [B, S_max, Hkv, D]   strides v_stride  = {b, s, h}
 *   o  [B, Hq, D]           strides o_stride  = {b, h}
 *   lse  fp32 [B, Hq] contiguous, natural log (nullable)
 *   seqlens  device int32 [B] valid lengths, each clamped to [0, max_seqlen]
 *            (nullable: every sequence has max_seqlen tokens).  Keys at
 *            positions >= seqlens[b] are never read.  A zero-length sequence
 *            yields O = 0 and lse = -inf.
 *   scale  multiplies q.k (the reference passes 1/sqrt(D)).
 *   split_tokens  KV tokens per split (rounded up to 128); 0 = automatic.
 *   workspace / workspace_bytes  device scratch of at least
 *            fgqa_decode_workspace_bytes(); pass NULL/0 to let the library use
 *            its own per-device cached buffer (allocated on first use).  Calls
 *            that share that buffer must not run at the same time on the GPU:
 *            concurrent calls on different streams of one device each pass
 *            their own workspace.  (Host threads may call concurrently.)
 */
typedef struct fgqa_decode_args {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    float* lse;
    const int32_t* seqlens;
    int32_t batch;
    int32_t max_seqlen;
    int32_t num_q_heads;
    int32_t num_kv_heads;
    int32_t head_dim;
    float scale;
    int64_t q_stride[2];
    int64_t k_stride[3];
    int64_t v_stride[3];
    int64_t o_stride[2];
    int32_t split_tokens;
    void* workspace;
    size_t workspace_bytes;
} fgqa_decode_args;

/* Bytes of workspace fgqa_decode_bf16 needs for these arguments (pointers unused). */
int fgqa_decode_workspace_bytes(const fgqa_decode_args* args, size_t* bytes);

/* Launch the decode on `stream`. */
int fgqa_decode_bf16(const fgqa_decode_args* args, void* stream);

/*
 * fgqa_decode_bf16 that allocates nothing.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments and results as fgqa_decode_bf16, except that `workspace` must be
 * NULL and `workspace_bytes` 0 (else FGQA_ERR_INVALID_ARGUMENT): the split
 * partials and the ragged work list go to a device array built into the
 * library, FGQA_DECODE_NOALLOC_SCRATCH_BYTES on every device it runs on,
 * held until the process ends.  A call whose plan needs more
 * (fgqa_decode_workspace_bytes() above that size) returns FGQA_ERR_WORKSPACE
 * and launches nothing; BASELINE-size ragged batches (64 x 64 heads, 32 K
 * tokens) need about half of it.  All calls on one device share that array:
 * calls that overlap on the GPU (different streams, or host threads racing)
 * corrupt each other's results; calls on one stream are safe.
 */
#define FGQA_DECODE_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int fgqa_decode_bf16_noalloc(const fgqa_decode_args* args, void* stream);

/*
 * Decode over a paged KV cache (block table), in bf16 or fp8.  No counterpart
 * in the reference: it extends the decode above (and its per-sequence
 * lengths) to the paged layout serving engines keep their KV cache in.
 *
 *   q, o       bf16 [B, Hq, D], strides {b, h} (as fgqa_decode_bf16)
 *   k_cache    [num_pages, page_size, Hkv, D] of kv_dtype, strides
 *   v_cache      {page, slot, head} in elements of kv_dtype
 *   block_table  device int32 [B, block_table_stride]: token t of sequence b
 *              is slot t % page_size of page block_table[b][t / page_size].
 *              Entries are clamped to [0, num_pages) on the device.
 *   seqlens    device int32 [B] (required), each clamped to [0, max_seqlen];
 *              max_seqlen <= block_table_stride * page_size.
 *   page_size  a power of two.
 *   kv_dtype   FGQA_KV_BF16 or FGQA_KV_FP8_E4M3 (OCP e4m3, as torch.float8_e4m3fn);
 *              the cache holds K/k_scale and V/v_scale: scores use
 *              q.k * k_scale * scale and O is multiplied by v_scale.
 *   lse        nullable fp32 [B, Hq], natural log.
 * Alignment: q, o, caches 16-byte aligned; cache strides multiples of 16 bytes.
 */
enum fgqa_kv_dtype { FGQA_KV_BF16 = 0, FGQA_KV_FP8_E4M3 = 1 };

typedef struct fgqa_decode_paged_args {
    const void* q;
    const void* k_cache;
    const void* v_cache;
    void* o;
    float* lse;
    const int32_t* block_table;
    const int32_t* seqlens;
    int32_t batch;
    int32_t max_seqlen;
    int32_t num_q_heads;
    int32_t num_kv_heads;
    int32_t head_dim;
    int32_t page_size;
    int32_t num_pages;
    int32_t kv_dtype;
    float scale;
    float k_scale;
    float v_scale;
    int64_t q_stride[2];
    int64_t o_stride[2];
    int64_t k_stride[3];
    int64_t v_stride[3];
    int64_t block_table_stride;
    int32_t split_tokens;
    void* workspace;
    size_t workspace_bytes;
} fgqa_decode_paged_args;

int fgqa_decode_paged_workspace_bytes(const fgqa_decode_paged_args* args, size_t* bytes);

int fgqa_decode_paged(const fgqa_decode_paged_args* args, void* stream);

/*
 * Causal (or full) prefill forward.  Replaces the Triton-only
 * launch_flash_gqa_forward_bf16_kernel, reference
 * src/python/Triton/flash_gqa_kernel.py:185-338 (kernel :15-138), which has no
 * C++ counterpart in the reference.
 *
 *   q  [B, Sq, Hq, D]  (BSHD) or any layout expressible by q_stride = {b, s, h}
 *   k  [B, Skv, Hkv, D]        k_stride = {b, s, h}
 *   v  [B, Skv, Hkv, D]        v_stride = {b, s, h}
 *   o  [B, Sq, Hq, D]          o_stride = {b, s, h}
 *   lse  fp32 [B, Hq, Sq] contiguous, natural log (nullable) -- the Triton layout
 *   causal  nonzero: query i sees keys j <= i (top-left aligned, as the
 *           reference's q_idx >= kv_idx mask).  A row with no visible key
 *           (Skv == 0) yields O = 0 and lse = -inf.
 * BHSD (the Triton layout) is q_stride = {Hq*Sq*D, D, Sq*D} etc.
 *   window_size  0: none.  > 0 (causal only): sliding window, row i sees keys
 *           [i - window_size + 1, i], as the reference's
 *           src/python/Triton/SWA/flash_swa_kernel.py:15-160.
 *   sink    nullable device fp32 [Hq]: per-head sink added to the softmax
 *           denominator, sum_j exp(s_j - m) + sink * exp(-m); lse includes it.
 *           A row with no visible key then gives O = 0, lse = log(max(sink, 1e-9)).
 *   Callers that zero the struct get neither.
 *   head_dim_v  V/O head dim; 0 means head_dim.  head_dim = 192 with
 *           head_dim_v = 128 is the MLA prefill, replacing the Triton-only
 *           launch_flash_mla_forward_bf16_kernel, reference
 *           src/python/Triton/flash_mla_kernel.py:315-508 (kernel :16-270):
 *           q/k rows hold head_dim elements, v/o rows head_dim_v.  Built:
 *           (128, 128); (192, 128) without window or sink; (256, 128) (the
 *           whole-range kernel only: FGQA_KERNEL_AUTO or _WHOLE).  Any other
 *           pair with both dims in [1, 256] runs on copies of q and k
 *           zero-padded to 128, 192 (for head_dim 192) or 256, and of v to
 *           128 or 256 (then one launch per 128 columns, each recomputing the
 *           scores), before the first head_dim_v columns of O are copied
 *           out, as the reference's Triton launcher pads its head-dim blocks
 *           to a power of two (src/python/Triton/flash_gqa_kernel.py:
 *           266-269); zero columns add nothing to q.k^T.  Those copies are
 *           made element by element, so such calls need neither 16-byte
 *           alignment nor strides in multiples of 8.  Head dims above 256
 *           return FGQA_ERR_UNSUPPORTED, and so do a window or sink with
 *           head_dim 192 and FGQA_KERNEL_SPLIT / _WIDE / _TALL with q/k
 *           padded to 256.
 *   kernel  an fgqa_kernel_choice (0 = AUTO).  The window / sink variant has
 *           no split form: FGQA_KERNEL_SPLIT with either returns
 *           FGQA_ERR_UNSUPPORTED (FGQA_KERNEL_WIDE runs it).
 *   workspace / workspace_bytes  device scratch of at least
 *           fgqa_prefill_workspace_bytes() bytes, 256-byte aligned, for the
 *           kernels that split a unit's KV range over two workgroups (the
 *           wide and tall kernels on causal grids whose unit pairs fill the
 *           CUs, such as S=4096, Hq=16, Hkv=1), and for the padded copies
 *           of head dims below 128 (after the counters and merge slots); the
 *           other shapes need none.  With NULL / 0, head dims below 128 keep
 *           their copies in the library's per-device cached buffer (the
 *           decode's, grown with hipMalloc when too small).
 *           Its first FGQA_PREFILL_WORKSPACE_ZERO_BYTES bytes (the arrival
 *           counters) must be zero before its first use; every call leaves
 *           them zero when it completes, so the workspace can be reused
 *           (graph replays included) without clearing.  Calls that overlap
 *           on the GPU must not share a workspace: concurrent calls on
 *           different streams each pass their own.  NULL / 0 uses the
 *           library's per-device scratch, which every such NULL call on
 *           that device shares.  Callers that zero the struct get NULL / 0.
 */
#define FGQA_PREFILL_WORKSPACE_ZERO_BYTES 4096

typedef struct fgqa_prefill_args {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    float* lse;
    int32_t batch;
    int32_t seqlen_q;
    int32_t seqlen_kv;
    int32_t num_q_heads;
    int32_t num_kv_heads;
    int32_t head_dim;
    int32_t causal;
    float scale;
    int64_t q_stride[3];
    int64_t k_stride[3];
    int64_t v_stride[3];
    int64_t o_stride[3];
    int32_t window_size;
    const float* sink;
    int32_t head_dim_v;
    int32_t kernel;
    void* workspace;
    size_t workspace_bytes;
} fgqa_prefill_args;

int fgqa_prefill_bf16(const fgqa_prefill_args* args, void* stream);

/* Bytes of workspace fgqa_prefill_bf16 needs for these arguments on the
 * current device (0: the chosen kernel needs none).  Same validation as the
 * call; launches nothing.  (No counterpart in the reference, whose Triton
 * launcher keeps no state between its kernel's workgroups.) */
int fgqa_prefill_workspace_bytes(const fgqa_prefill_args* args, size_t* bytes);

/* The kernel shape (FGQA_KERNEL_WHOLE, _SPLIT or _WIDE) fgqa_prefill_bf16
 * runs for these arguments on the current device: `kernel`, or what AUTO
 * picks.  Same validation and status codes as the call; launches nothing.
 * (No counterpart in the reference, whose prefill has one kernel shape.) */
int fgqa_prefill_kernel_choice(const fgqa_prefill_args* args, int32_t* kernel);

/* The name of the kernel function fgqa_prefill_bf16 launches for these
 * arguments on the current device (static storage), which also tells apart
 * the grid forms of one kernel shape: "prefill_kernel",
 * "prefill_split_kernel", "prefill_wide_kernel" (unit pairs),
 * "prefill_wide_persistent_kernel", "prefill_tall_pairs_kernel" or
 * "prefill_tall_persistent_kernel".  Same validation as the call; launches
 * nothing.  (No counterpart in the reference.) */
int fgqa_prefill_kernel_name(const fgqa_prefill_args* args, const char** name);

/*
 * Prefill backward: dQ, dK, dV of the causal (or full) forward above.
 * Replaces the Triton-only launch_flash_gqa_backward_bf16_kernel, reference
 * src/python/Triton/flash_gqa_backward_kernel.py:312-478 (kernels :16-50 and
 * :159-310), which has no C++ counterpart in the reference.
 *
 *   q, o, grad_o, grad_q  [B, Sq, Hq, D]   strides {b, s, h} each
 *   k, v, grad_k, grad_v  [B, Skv, Hkv, D] strides {b, s, h} each
 *   lse  fp32 [B, Hq, Sq] contiguous, natural log, as fgqa_prefill_bf16
 *        writes it
 *   causal, scale  as in the forward call that produced o and lse.
 * grad_* are written (not accumulated); a key that no query row sees gets
 * zero gradients.  Gradients are accumulated in fp32 in the workspace and
 * rounded to bf16 once.
 * workspace / workspace_bytes  device scratch of at least
 *   fgqa_prefill_backward_workspace_bytes() bytes, 256-byte aligned; NULL/0
 *   uses the library's per-device cached buffer (same rule as for decode:
 *   concurrent calls on different streams each pass their own workspace).
 * window_size  0: none.  > 0 (causal only): the sliding-window backward,
 *   replacing the Triton-only launch_flash_swa_backward_bf16_kernel,
 *   reference src/python/Triton/SWA/flash_swa_backward_kernel.py:323-489
 *   (kernel :157-321): row i uses keys [i - window_size + 1, i].  A sink
 *   needs nothing here: it is in the lse the forward wrote (the reference
 *   computes no sink gradient).
 * head_dim_v  0 (= head_dim) or the V / O / grad_o head dim.  head_dim 192
 *   with head_dim_v 128 is the MLA backward, replacing the Triton-only
 *   launch_flash_mla_backward_bf16_kernel (src/python/Triton/
 *   flash_mla_backward_kernel.py:788-969, kernel :202-786): q, k, grad_q,
 *   grad_k have 192-element rows, v, o, grad_o, grad_v 128-element rows.
 *   Built: (128, 128), and (192, 128) without a window.  Q/K head dims up to
 *   128 (or 192, without a window) with V/O head dims up to 128 run on copies
 *   of q, k, v, o, grad_o zero-padded to a built pair (element by element:
 *   no alignment needed), the first columns of the padded gradients copied
 *   out; the copies live in the workspace after the built call's own bytes
 *   (fgqa_prefill_backward_workspace_bytes includes them).  Other head dims
 *   return FGQA_ERR_UNSUPPORTED.
 * kv_head_split  0: automatic.  n >= 1 (a divisor of Hq / Hkv): the dK/dV pass
 *   splits each KV head's query heads over n workgroups whose fp32 partials a
 *   reduction sums (n = 1: no partials).  It changes the workspace size.
 *   Other values return FGQA_ERR_INVALID_ARGUMENT.
 * dq_kernel  an fgqa_kernel_choice for the dQ pass (0 = AUTO).  The MLA shape
 *   has no split dQ kernel: FGQA_KERNEL_SPLIT with head_dim 192 returns
 *   FGQA_ERR_UNSUPPORTED.
 */
typedef struct fgqa_prefill_backward_args {
    const void* q;
    const void* k;
    const void* v;
    const void* o;
    const float* lse;
    const void* grad_o;
    void* grad_q;
    void* grad_k;
    void* grad_v;
    int32_t batch;
    int32_t seqlen_q;
    int32_t seqlen_kv;
    int32_t num_q_heads;
    int32_t num_kv_heads;
    int32_t head_dim;
    int32_t causal;
    float scale;
    int64_t q_stride[3];
    int64_t k_stride[3];
    int64_t v_stride[3];
    int64_t o_stride[3];
    int64_t grad_o_stride[3];
    int64_t grad_q_stride[3];
    int64_t grad_k_stride[3];
    int64_t grad_v_stride[3];
    void* workspace;
    size_t workspace_bytes;
    int32_t window_size;
    int32_t head_dim_v;
    int32_t kv_head_split;
    int32_t dq_kernel;
} fgqa_prefill_backward_args;

/* Bytes of workspace fgqa_prefill_backward_bf16 needs (pointers unused; the
 * sizes, causal and window_size decide it). */
int fgqa_prefill_backward_workspace_bytes(const fgqa_prefill_backward_args* args, size_t* bytes);

int fgqa_prefill_backward_bf16(const fgqa_prefill_backward_args* args, void* stream);

/*
 * Sparse-index GQA prefill forward.  Replaces the Triton-only
 * launch_flash_sgqa_forward_bf16_kernel, reference
 * src/python/Triton/SparseGQA/flash_sgqa_kernel.py:202-396 (kernel :15-137).
 *
 *   q  [B, Sq, Hq, D], k/v [B, Skv, Hkv, D], o [B, Sq, Hq, D]: strides
 *      {batch, sequence, head} as in fgqa_prefill_args; D = 128.
 *   kv_indices  int32, entry e of query row i of kv head h at
 *      kv_indices + b*idx_stride[0] + h*idx_stride[1] + i*idx_stride[2] + e,
 *      e < num_sparse_kv (the reference's [B, Hkv, Sq, num_sparse_kv]).
 *      Query row i of every query head of kv head h attends the listed keys:
 *      an entry j is used when 0 <= j < seqlen_kv and, if causal, j <= i
 *      (others, e.g. -1 padding, are skipped); a key listed twice counts twice.
 *   lse  fp32 [B, Hq, Sq] contiguous, natural log (nullable).  A row with no
 *      usable entry gives O = 0 and lse = -inf.
 */
typedef struct fgqa_sparse_prefill_args {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    float* lse;
    const int32_t* kv_indices;
    int32_t batch;
    int32_t seqlen_q;
    int32_t seqlen_kv;
    int32_t num_q_heads;
    int32_t num_kv_heads;
    int32_t head_dim;
    int32_t num_sparse_kv;
    int32_t causal;
    float scale;
    int64_t q_stride[3];
    int64_t k_stride[3];
    int64_t v_stride[3];
    int64_t o_stride[3];
    int64_t idx_stride[3];
} fgqa_sparse_prefill_args;

int fgqa_sparse_prefill_bf16(const fgqa_sparse_prefill_args* args, void* stream);

/* Static, human-readable text for a status code. */
const char* fgqa_status_string(int status);

/* Library version as MAJOR*10000 + MINOR*100 + PATCH. */
int fgqa_version(void);

/* Measurement helper (no counterpart in the reference): enqueues on `stream`
 * `samples` (1 .. 65536) one-wave workgroups; workgroup w stores to the
 * device array out[3w .. 3w+2] (8-byte aligned) its CU's shader-clock
 * counter (s_memtime), the 100 MHz real-time counter (s_memrealtime) and
 * (xcd << 8) | the SE, SH and CU fields of HW_ID, which names the CU.  Two
 * such launches on one stream around a run of launches give, for each CU
 * sampled by both, the average shader clock over the run:
 * (t1 - t0) / (r1 - r0) * 100 MHz (the counters of different CUs are not
 * aligned, so only samples of one CU are differenced).  Used by bench.py to
 * record the clock the MFMA-bound kernels sustain. */
int fgqa_clock_sample(unsigned long long* out, int samples, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FGQA_H */
