// FlashGQA prefill forward: C++ operator entry points (MI355X / gfx950).
//
// The reference implements prefill only in Triton
// (src/python/Triton/flash_gqa_kernel.py:185-338, kernel :15-138); these are
// its C++ counterparts.  Same maths and LSE layout; the default layout is
// BSHD, matching the reference's C++ decode K/V layout.
#pragma once

#include <cstdint>

#include "Utils/utils.h"

/**
 * @brief Launches the FlashGQA bf16 prefill forward (BSHD layout).
 * @param q Device query tensor [batchSize, seqLengthQ, numQueryHeads, headDim].
 * @param k Device key tensor [batchSize, seqLengthKv, numKvHeads, headDim].
 * @param v Device value tensor [batchSize, seqLengthKv, numKvHeads, headDim].
 * @param scale Scaling factor applied to QK scores.
 * @param o Device output tensor [batchSize, seqLengthQ, numQueryHeads, headDim].
 * @param lse Device fp32 log-sum-exp [batchSize, numQueryHeads, seqLengthQ] (natural log), or nullptr.
 * @param batchSize Batch size.
 * @param seqLengthQ Query sequence length.
 * @param seqLengthKv Key/value sequence length.
 * @param numQueryHeads Number of query heads.
 * @param numKvHeads Number of KV heads (must divide numQueryHeads).
 * @param headDim Per-head embedding dimension in [1, 256]: 128 runs the kernels
 *        directly, other values run on copies zero-padded to 128 or 256, as the
 *        reference's Triton launcher pads its head-dim blocks
 *        (src/python/Triton/flash_gqa_kernel.py:266-269).
 * @param causal Apply the top-left aligned causal mask (query i sees keys j <= i).
 */
void LaunchFlashGqaForwardBf16Kernel(const bf16_t* q,
                                     const bf16_t* k,
                                     const bf16_t* v,
                                     float scale,
                                     bf16_t* o,
                                     float* lse,
                                     int batchSize,
                                     int seqLengthQ,
                                     int seqLengthKv,
                                     int numQueryHeads,
                                     int numKvHeads,
                                     int headDim,
                                     bool causal);

/**
 * @brief Strided variant: element strides {batch, sequence, head} per tensor
 *        (head dim contiguous).  BHSD, the Triton layout, is
 *        qStride = {Hq*Sq*D, D, Sq*D}, kStride = vStride = {Hkv*Skv*D, D, Skv*D}.
 */
void LaunchFlashGqaForwardBf16KernelStrided(const bf16_t* q,
                                            const bf16_t* k,
                                            const bf16_t* v,
                                            float scale,
                                            bf16_t* o,
                                            float* lse,
                                            int batchSize,
                                            int seqLengthQ,
                                            int seqLengthKv,
                                            int numQueryHeads,
                                            int numKvHeads,
                                            int headDim,
                                            bool causal,
                                            const int64_t qStride[3],
                                            const int64_t kStride[3],
                                            const int64_t vStride[3],
                                            const int64_t oStride[3]);

/**
 * @brief Sliding-window prefill with a per-head sink (BSHD), the C++
 *        counterpart of the reference's Triton-only SWA launcher
 *        (src/python/Triton/SWA/flash_swa_kernel.py:188-370): causal, row i
 *        sees keys [i - windowSize + 1, i]; sink (nullable device fp32
 *        [numQueryHeads]) joins the softmax denominator as sink * exp(-max).
 */
void LaunchFlashSwaForwardBf16Kernel(const bf16_t* q,
                                     const bf16_t* k,
                                     const bf16_t* v,
                                     float scale,
                                     bf16_t* o,
                                     float* lse,
                                     int batchSize,
                                     int seqLengthQ,
                                     int seqLengthKv,
                                     int numQueryHeads,
                                     int numKvHeads,
                                     int headDim,
                                     int windowSize,
                                     const float* sink);

/**
 * @brief MLA prefill forward (BSHD): Q/K head dim headDimQk, V/O head dim
 *        headDimV, the C++ counterpart of the reference's Triton-only MLA
 *        launcher (src/python/Triton/flash_mla_kernel.py:315-508, kernel
 *        :16-270).  Supported: (headDimQk, headDimV) = (192, 128), or any pair
 *        with both dims in [1, 256] (on zero-padded copies unless built).
 * @param q Device query tensor [batchSize, seqLengthQ, numQueryHeads, headDimQk].
 * @param k Device key tensor [batchSize, seqLengthKv, numKvHeads, headDimQk].
 * @param v Device value tensor [batchSize, seqLengthKv, numKvHeads, headDimV].
 * @param o Device output tensor [batchSize, seqLengthQ, numQueryHeads, headDimV].
 * @param lse Device fp32 log-sum-exp [batchSize, numQueryHeads, seqLengthQ] (natural log), or nullptr.
 */
void LaunchFlashMlaForwardBf16Kernel(const bf16_t* q,
                                     const bf16_t* k,
                                     const bf16_t* v,
                                     float scale,
                                     bf16_t* o,
                                     float* lse,
                                     int batchSize,
                                     int seqLengthQ,
                                     int seqLengthKv,
                                     int numQueryHeads,
                                     int numKvHeads,
                                     int headDimQk,
                                     int headDimV,
                                     bool causal);

/**
 * @brief Sparse-index GQA prefill forward (BSHD), the C++ counterpart of the
 *        reference's Triton-only sparse-GQA launcher
 *        (src/python/Triton/SparseGQA/flash_sgqa_kernel.py:202-396, kernel
 *        :15-137).  Query row i of every query head of KV head h attends the
 *        keys listed in kvIndices[b][h][i][0 .. numSparseKv); entries < 0,
 *        >= seqLengthKv or (causal) > i are skipped, duplicates count twice.
 * @param kvIndices Device int32 [batchSize, numKvHeads, seqLengthQ, numSparseKv], contiguous.
 * @param lse Device fp32 [batchSize, numQueryHeads, seqLengthQ] (natural log), or nullptr.
 */
void LaunchFlashSgqaForwardBf16Kernel(const bf16_t* q,
                                      const bf16_t* k,
                                      const bf16_t* v,
                                      const int32_t* kvIndices,
                                      int numSparseKv,
                                      float scale,
                                      bf16_t* o,
                                      float* lse,
                                      int batchSize,
                                      int seqLengthQ,
                                      int seqLengthKv,
                                      int numQueryHeads,
                                      int numKvHeads,
                                      int headDim,
                                      bool causal);
