/*
 * fgqa_oracle.h -- CPU restatement of the reference's flash grouped-query
 * attention (decode + causal prefill), used ONLY as a parity checker.
 *
 * TEST INFRASTRUCTURE.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the checker (or, for
 * cpu_baseline, as the timed CPU reference).  The product path
 * (cuda_llm_ops_amd, include/) never links, loads or calls it.
 *
 * bf16 values travel as uint16_t bit patterns (upper half of IEEE binary32).
 * All sizes are element counts; strides are element strides.
 *
 * Parity status of each function (how it is pinned, see tests/test_oracle.py):
 *   fgqa_oracle_f32_to_bf16 / bf16_to_f32   exhaustive 2^16 round trip + IEEE-754
 *                                            RNE tie cases + numpy restatement
 *   fgqa_oracle_decode_bf16                 fp64 brute force (fgqa_oracle_attention_f64)
 *                                            at the stated tolerance, closed forms
 *                                            (len=1, constant V, equal K), invariants;
 *                                            the fp32-P variant (p_bf16 = 0) sits closer
 *                                            to the fp64 answer than the bf16-P one
 *   fgqa_oracle_prefill_bf16                fp64 brute force, closed forms (row 0 = V[0],
 *                                            LSE of equal logits = log n), invariants
 *   fgqa_oracle_prefill_mla_bf16            bit-identical to fgqa_oracle_prefill_bf16 when
 *                                            dqk = dv; a float64 numpy restatement with
 *                                            dqk = 192, dv = 128; closed forms (causal row 0
 *                                            = V[0]; Q = 0 gives the running mean of V)
 *   fgqa_oracle_prefill_backward_bf16       fp64 backward (fgqa_oracle_attention_backward_f64,
 *                                            the torch-reference form) at the stated tolerance,
 *                                            closed forms (one key: dQ = dK = 0, dV = sum dO),
 *                                            invariants (sum_j dK_j = 0, sum_j dV_j = sum dO)
 *   fgqa_oracle_attention_backward_f64      central finite differences of a float64
 *                                            numpy forward on tiny inputs
 *   fgqa_oracle_prefill_mla_backward_bf16   bit-identical to fgqa_oracle_prefill_backward_bf16
 *                                            when dqk = dvd; the float64 MLA gradient below
 *                                            at the stated tolerance; planted mistakes
 *   fgqa_oracle_attention_mla_backward_f64  central finite differences of a float64 numpy
 *                                            forward with dqk != dvd
 *   fgqa_oracle_fp8e4m3_to_f32              all 256 codes against torch.float8_e4m3fn
 *   fgqa_oracle_decode_paged                bit-identical to fgqa_oracle_decode_bf16 on a
 *                                            contiguous bf16 cache; page-permutation
 *                                            invariance; fp8 path vs the fp64 brute force
 *                                            on the decoded values
 *   fgqa_oracle_prefill_swa_backward_bf16   bit-identical to fgqa_oracle_prefill_backward_bf16
 *                                            for a window >= Sq; the float64 SWA gradient
 *                                            below at the stated tolerance
 *   fgqa_oracle_attention_swa_backward_f64  central finite differences of a float64 numpy
 *                                            forward with window and sink
 *   fgqa_oracle_prefill_swa_bf16            bit-identical to fgqa_oracle_prefill_bf16 for a
 *                                            window >= Sq and no sink; a float64 numpy
 *                                            restatement with the window and sink; closed
 *                                            forms (window 1: O = V[i] / (1 + sink e^-s_ii))
 *   fgqa_oracle_sparse_prefill_bf16         bit-identical to fgqa_oracle_prefill_bf16 when
 *                                            every row lists keys 0..Skv-1 in order; a
 *                                            float64 numpy restatement; closed forms (one
 *                                            valid entry: O = V[j]; none: O = 0, lse = -inf;
 *                                            a key listed twice = its score + ln 2)
 *   fgqa_oracle_attention_f64               textbook softmax attention in double;
 *                                            pinned by numpy float64 restatement and
 *                                            closed forms on tiny inputs
 */
#ifndef FGQA_ORACLE_H
#define FGQA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* IEEE-754 binary32 -> bfloat16, round to nearest even; NaN stays NaN (quiet). */
uint16_t fgqa_oracle_f32_to_bf16(float x);
float fgqa_oracle_bf16_to_f32(uint16_t h);
void fgqa_oracle_f32_to_bf16_array(const float* src, uint16_t* dst, size_t n);
void fgqa_oracle_bf16_to_f32_array(const uint16_t* src, float* dst, size_t n);

/*
 * Decode (one query token per sequence), restating the reference's C++ CPU
 * reference examples/cplusplus/test_decode_flash_gqa.cu:184-255:
 * 128-token flash tiles (tile = 128 there), fp32 q.k dot, running max in
 * scaled units, fp32 rowsum, P rounded to bf16 before P.V, O/rowsum -> bf16.
 * Generalised (as the new kernel is) to any group size, a partial last tile
 * and per-sequence lengths.
 *
 * Layouts (the reference's, decode_flash_gqa_kernel.cu:144-148):
 *   q, o : [B, Hq, D]         k, v : [B, S_max, Hkv, D]
 * seqlens: host array of B lengths (each 0..S_max) or NULL (= S_max for all).
 * lse (nullable): fp32 [B, Hq], natural log; a length-0 row gives O = 0, lse = -inf.
 * tile: flash tile length (the reference uses 128).
 * p_bf16: 1 rounds P to bf16 before P.V, as the C++ reference does; 0 keeps P
 * in fp32, which restates the torch tiled decode reference
 * examples/python/Triton/test_decode_flash_gqa_kernel.py:26-79 (tile 128,
 * online softmax, fp32 throughout).  nthreads <= 0: OpenMP default.
 * Returns 0, or -1 on invalid arguments.
 */
int fgqa_oracle_decode_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                            float scale, uint16_t* o, float* lse,
                            int batch, int s_max, int hq, int hkv, int d,
                            const int32_t* seqlens, int tile, int p_bf16, int nthreads);

/*
 * OCP FP8 E4M3 (torch.float8_e4m3fn) -> float, from the format definition:
 * bias 7, 3 mantissa bits, subnormals m/8 * 2^-6, S.1111.111 = NaN, no inf.
 */
float fgqa_oracle_fp8e4m3_to_f32(uint8_t c);

/*
 * Decode over a paged KV cache (no counterpart in the reference): the loop of
 * fgqa_oracle_decode_bf16 (p_bf16 = 1) with each K/V row fetched through the
 * block table and, for kv_fp8, decoded from e4m3.  Scores use
 * q.k * (scale * k_scale); the output is bf16((O / l) * v_scale).  With bf16
 * caches holding a contiguous sequence, k_scale = v_scale = 1, the results
 * are bit-identical to fgqa_oracle_decode_bf16.
 *   q, o: [B, Hq, D] contiguous; k_cache / v_cache: uint16 bf16 bits or uint8
 *   e4m3 codes, element strides {page, slot, head}; token t of sequence b is
 *   slot t % page_size of page block_table[b * bt_stride + t / page_size].
 *   seqlens: host int32 [B] (required).
 */
int fgqa_oracle_decode_paged(const uint16_t* q, const void* k_cache, const void* v_cache, int kv_fp8,
                             const int32_t* block_table, int64_t bt_stride, int page_size,
                             const int64_t* k_strides, const int64_t* v_strides,
                             float scale, float k_scale, float v_scale, uint16_t* o, float* lse,
                             int batch, int hq, int hkv, int d, const int32_t* seqlens, int tile,
                             int nthreads);

/*
 * Prefill forward, restating the reference's torch reference
 * examples/python/Triton/test_flash_gqa_kernel.py:60-90 (fp32 scores, causal
 * triu(diagonal=1) mask = top-left aligned, q_idx >= kv_idx as in
 * src/python/Triton/flash_gqa_kernel.py:113-117, full softmax, fp32 P.V,
 * lse = log(sum exp) + max) with BSHD-or-any strides.
 *   q: (b, s, h) strides qs[3]; k: ks[3]; v: vs[3]; o: os[3]; head dim contiguous.
 *   lse (nullable): fp32, contiguous [B, Hq, Sq].
 * q_offset: query row i sits at absolute position i + q_offset, so a causal
 * row sees keys j <= i + q_offset (0 for the reference's square Sq = Skv case;
 * a nonzero offset lets a test check a slice of rows of a long sequence).
 * A row with no visible key gives O = 0 and lse = -inf.
 */
int fgqa_oracle_prefill_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                             float scale, uint16_t* o, float* lse,
                             int batch, int sq, int skv, int hq, int hkv, int d,
                             const int64_t* q_strides, const int64_t* k_strides,
                             const int64_t* v_strides, const int64_t* o_strides,
                             int causal, int q_offset, int nthreads);

/*
 * MLA prefill (separate head dims: Q/K rows of dqk, V/O rows of dv), restating
 * the reference's torch reference examples/python/Triton/test_flash_mla_kernel.py:27-95
 * with the same steps as fgqa_oracle_prefill_bf16 (scores over dqk, P.V over dv).
 * o has dv-element rows at strides o_strides; everything else as fgqa_oracle_prefill_bf16.
 */
int fgqa_oracle_prefill_mla_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                 float scale, uint16_t* o, float* lse,
                                 int batch, int sq, int skv, int hq, int hkv, int dqk, int dv,
                                 const int64_t* q_strides, const int64_t* k_strides,
                                 const int64_t* v_strides, const int64_t* o_strides,
                                 int causal, int q_offset, int nthreads);

/*
 * Prefill backward, restating the reference's Triton backward
 * src/python/Triton/flash_gqa_backward_kernel.py for one query row i and key j
 * of query head h (kv head h / G):
 *   :16-50   delta_i = sum_x O_i[x] dO_i[x]                         (fp32)
 *   :253-262 p = exp(q_i.k_j * scale - lse_i); 0 where j > i (causal,
 *            top-left) or j >= Skv                                   (fp32)
 *   :263     p_bf16 = bf16(p)
 *   :271-272 dV_j += p_bf16 * dO_i
 *   :274-275 dP = dO_i . v_j                                         (fp32)
 *   :283-285 dS = bf16(p * (dP - delta_i) * scale)
 *   :287     dK_j += dS * q_i          :292-293  dQ_i += dS * k_j
 * summed over the G query heads of the kv head for dK/dV.  Outputs are the
 * fp32 accumulators (the reference casts them to bf16 at :470-472):
 *   dq: float [B, Sq, Hq, D]; dk, dv: float [B, Skv, Hkv, D], contiguous.
 * Strides as fgqa_oracle_prefill_bf16 (o: os, grad_o: dos); lse fp32
 * contiguous [B, Hq, Sq] (natural log, as the forward writes it).
 * rows (nullable) = {first, end}: dq is computed only for query rows in
 * [first, end) (other rows left untouched); keys (nullable) likewise limits
 * the dk/dv rows computed.  dq/dk/dv may each be NULL to skip that output.
 */
int fgqa_oracle_prefill_backward_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                      const uint16_t* o, const float* lse, const uint16_t* grad_o,
                                      float scale, float* dq, float* dk, float* dv,
                                      int batch, int sq, int skv, int hq, int hkv, int d,
                                      const int64_t* q_strides, const int64_t* k_strides,
                                      const int64_t* v_strides, const int64_t* o_strides,
                                      const int64_t* grad_o_strides, int causal,
                                      const int* rows, const int* keys, int nthreads);

/*
 * Gradient of textbook softmax attention in double precision: P recomputed
 * from scratch (no LSE input), dV = P^T dO, dP = dO V^T,
 * dS = P (dP - delta), dQ = scale dS K, dK = scale dS^T Q.  delta_i is
 * sum_j P_ij dP_ij (the exact gradient) when o == NULL, else
 * sum_x O_i[x] dO_i[x] from the given bf16 O, which restates the reference's
 * torch backward reference examples/python/Triton/test_flash_gqa_kernel.py:97-173.
 * Outputs double, contiguous: dq [B, Sq, Hq, D]; dk, dv [B, Skv, Hkv, D].
 */
int fgqa_oracle_attention_backward_f64(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                       const uint16_t* o, const uint16_t* grad_o, double scale,
                                       double* dq, double* dk, double* dv,
                                       int batch, int sq, int skv, int hq, int hkv, int d,
                                       const int64_t* q_strides, const int64_t* k_strides,
                                       const int64_t* v_strides, const int64_t* o_strides,
                                       const int64_t* grad_o_strides, int causal, int nthreads);

/*
 * MLA backward, following
 * src/python/Triton/flash_mla_backward_kernel.py: the steps of
 * fgqa_oracle_prefill_backward_bf16 with Q/K rows of dqk and V/O/dO rows of
 * dvd (scores over dqk, dP and delta over dvd).  dq, dk: fp32, dqk-element
 * rows; dv: fp32, dvd-element rows (BSHD, as fgqa_oracle_prefill_backward_bf16).
 */
int fgqa_oracle_prefill_mla_backward_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                          const uint16_t* o, const float* lse, const uint16_t* grad_o,
                                          float scale, float* dq, float* dk, float* dv,
                                          int batch, int sq, int skv, int hq, int hkv, int dqk, int dvd,
                                          const int64_t* qs, const int64_t* ks,
                                          const int64_t* vs, const int64_t* os,
                                          const int64_t* dos, int causal,
                                          const int* rows, const int* keys, int nthreads);

/* The float64 gradient of fgqa_oracle_attention_backward_f64 with separate
 * Q/K (dqk) and V/O (dvd) row lengths. */
int fgqa_oracle_attention_mla_backward_f64(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                           const uint16_t* o, const uint16_t* grad_o, double scale,
                                           double* dq, double* dk, double* dv,
                                           int batch, int sq, int skv, int hq, int hkv, int dqk, int dvd,
                                           const int64_t* qs, const int64_t* ks,
                                           const int64_t* vs, const int64_t* os,
                                           const int64_t* dos, int causal, int nthreads);

/*
 * Sliding-window backward, restating the reference's Triton SWA backward
 * src/python/Triton/SWA/flash_swa_backward_kernel.py:157-321: the steps of
 * fgqa_oracle_prefill_backward_bf16 with its causal + window mask (:278-282,
 * row i uses keys (i - window, i]).  The LSE is the forward's, sink included;
 * the reference computes no sink gradient.  window > 0.
 */
int fgqa_oracle_prefill_swa_backward_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                          const uint16_t* o, const float* lse, const uint16_t* grad_o,
                                          float scale, float* dq, float* dk, float* dv,
                                          int batch, int sq, int skv, int hq, int hkv, int d,
                                          const int64_t* q_strides, const int64_t* k_strides,
                                          const int64_t* v_strides, const int64_t* o_strides,
                                          const int64_t* grad_o_strides, int window,
                                          const int* rows, const int* keys, int nthreads);

/*
 * Exact gradient (double) of causal sliding-window attention with a per-head
 * sink in the denominator: p_j = e^{s_j} / (sum_k e^{s_k} + sink[h]) over the
 * window's keys; the sink acts as a key with zero value, so the gradient keeps
 * the form of fgqa_oracle_attention_backward_f64.  sink nullable.  window > 0.
 */
int fgqa_oracle_attention_swa_backward_f64(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                           const uint16_t* o, const uint16_t* grad_o, double scale,
                                           double* dq, double* dk, double* dv,
                                           int batch, int sq, int skv, int hq, int hkv, int d,
                                           const int64_t* q_strides, const int64_t* k_strides,
                                           const int64_t* v_strides, const int64_t* o_strides,
                                           const int64_t* grad_o_strides, int window, const float* sink,
                                           int nthreads);

/*
 * Causal sliding-window prefill with a per-head sink, restating the reference's
 * torch reference examples/python/Triton/test_flash_swa_kernel.py:97-116:
 *   scores = (q . k) * scale (fp32), masked to keys [i - window + 1, i];
 *   row_max; e = exp(scores - row_max);
 *   denom = sum(e) + sink[h] * exp(-row_max); probs = e / denom;
 *   lse = log(denom) + row_max;  out = probs . v (fp32) -> bf16.
 * sink: host fp32 [Hq] or NULL (no sink).  Layouts and strides as
 * fgqa_oracle_prefill_bf16; query row i sits at position i + q_offset.  A row with no visible key gives O = 0 and
 * lse = log(max(sink, 1e-9)) (the reference kernel's convention,
 * src/python/Triton/SWA/flash_swa_kernel.py:150-155), or -inf without a sink.
 */
int fgqa_oracle_prefill_swa_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                 float scale, uint16_t* o, float* lse,
                                 int batch, int sq, int skv, int hq, int hkv, int d,
                                 const int64_t* q_strides, const int64_t* k_strides,
                                 const int64_t* v_strides, const int64_t* o_strides,
                                 int window, const float* sink, int q_offset, int nthreads);

/*
 * Sparse-index prefill, restating the reference's torch reference
 * examples/python/Triton/test_flash_sgqa_kernel.py:97-222: query row i of head
 * h attends the keys listed in idx[b][h / G][i][0 .. nsparse), skipping
 * entries < 0, >= skv or (causal) > i + q_offset; a key listed twice counts
 * twice.  fp32 scores, full softmax, fp32 P.V, bf16 O; a row with no valid
 * entry gives O = 0 and lse = -inf.
 *   idx: int32, idx_strides = {batch, kv head, query row} in elements, the
 *        entry dim contiguous.  Other layouts as fgqa_oracle_prefill_bf16.
 */
int fgqa_oracle_sparse_prefill_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                    float scale, uint16_t* o, float* lse,
                                    int batch, int sq, int skv, int hq, int hkv, int d,
                                    const int64_t* q_strides, const int64_t* k_strides,
                                    const int64_t* v_strides, const int64_t* o_strides,
                                    const int32_t* idx, const int64_t* idx_strides, int nsparse,
                                    int causal, int q_offset, int nthreads);

/*
 * Textbook softmax attention in double precision (the mathematical answer the
 * two fp32 restatements approximate).  Query row i of sequence b sees keys
 * j < kv_len(b) and, if causal, j <= i + causal_offset.  kv_len(b) = seqlens[b]
 * when seqlens != NULL, else skv.  Strides as in fgqa_oracle_prefill_bf16.
 * o: double [B, Sq, Hq, D] contiguous; lse: double [B, Hq, Sq] (nullable).
 */
int fgqa_oracle_attention_f64(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                              double scale, double* o, double* lse,
                              int batch, int sq, int skv, int hq, int hkv, int d,
                              const int64_t* q_strides, const int64_t* k_strides,
                              const int64_t* v_strides, const int32_t* seqlens,
                              int causal, int causal_offset, int nthreads);

#ifdef __cplusplus
}
#endif

#endif /* FGQA_ORACLE_H */
