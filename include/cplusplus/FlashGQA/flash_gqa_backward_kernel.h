// FlashGQA prefill backward: C++ operator entry point (MI355X / gfx950).
//
// The reference implements the backward only in Triton
// (src/python/Triton/flash_gqa_backward_kernel.py:312-478, kernels :16-50 and
// :159-310); this is its C++ counterpart, in the BSHD layout of
// LaunchFlashGqaForwardBf16Kernel and consuming that call's O and LSE.
#pragma once

#include <cstdint>

#include "Utils/utils.h"

/**
 * @brief Launches the FlashGQA bf16 prefill backward (BSHD layout).
 * @param q Device query tensor [batchSize, seqLengthQ, numQueryHeads, headDim].
 * @param k Device key tensor [batchSize, seqLengthKv, numKvHeads, headDim].
 * @param v Device value tensor [batchSize, seqLengthKv, numKvHeads, headDim].
 * @param o Forward output [batchSize, seqLengthQ, numQueryHeads, headDim].
 * @param lse Forward fp32 log-sum-exp [batchSize, numQueryHeads, seqLengthQ] (natural log).
 * @param gradO Gradient of the output, layout of o.
 * @param scale Scaling factor the forward applied to QK scores.
 * @param gradQ Output: gradient of q, layout of q.
 * @param gradK Output: gradient of k, layout of k.
 * @param gradV Output: gradient of v, layout of v.
 * @param batchSize Batch size.
 * @param seqLengthQ Query sequence length.
 * @param seqLengthKv Key/value sequence length.
 * @param numQueryHeads Number of query heads.
 * @param numKvHeads Number of KV heads (must divide numQueryHeads).
 * @param headDim Per-head embedding dimension: 128, or any value in [1, 128) on zero-padded copies.
 * @param causal The forward's top-left aligned causal mask (query i sees keys j <= i).
 *
 * Uses the library's per-device cached workspace on the default stream; the
 * status of the call is returned by FlashGqaGetLastStatus().
 */
void LaunchFlashGqaBackwardBf16Kernel(const bf16_t* q,
                                      const bf16_t* k,
                                      const bf16_t* v,
                                      const bf16_t* o,
                                      const float* lse,
                                      const bf16_t* gradO,
                                      float scale,
                                      bf16_t* gradQ,
                                      bf16_t* gradK,
                                      bf16_t* gradV,
                                      int batchSize,
                                      int seqLengthQ,
                                      int seqLengthKv,
                                      int numQueryHeads,
                                      int numKvHeads,
                                      int headDim,
                                      bool causal);

/**
 * @brief Launches the sliding-window (SWA) bf16 prefill backward (BSHD layout).
 *
 * Counterpart of the reference's Triton SWA backward launcher
 * (src/python/Triton/SWA/flash_swa_backward_kernel.py:323-489, kernel
 * :157-321): query i's gradients cover keys [i - windowSize + 1, i].  lse is
 * LaunchFlashSwaForwardBf16Kernel's, computed with the sink term; the sink
 * has no value row, so no sink gradient is produced (as in the reference).
 * Parameters as LaunchFlashGqaBackwardBf16Kernel, with
 * @param windowSize Sliding-window size (> 0).
 */
void LaunchFlashSwaBackwardBf16Kernel(const bf16_t* q,
                                      const bf16_t* k,
                                      const bf16_t* v,
                                      const bf16_t* o,
                                      const float* lse,
                                      const bf16_t* gradO,
                                      float scale,
                                      bf16_t* gradQ,
                                      bf16_t* gradK,
                                      bf16_t* gradV,
                                      int batchSize,
                                      int seqLengthQ,
                                      int seqLengthKv,
                                      int numQueryHeads,
                                      int numKvHeads,
                                      int headDim,
                                      int windowSize);

/**
 * @brief Launches the MLA bf16 prefill backward (BSHD layout): Q/K head dim
 *        headDimQk, V/O head dim headDimV.
 *
 * Counterpart of the reference's Triton MLA backward launcher
 * (src/python/Triton/flash_mla_backward_kernel.py:788-969, kernel :202-786).
 * q, gradQ [B, Sq, Hq, headDimQk]; k, gradK [B, Skv, Hkv, headDimQk];
 * v, gradV [B, Skv, Hkv, headDimV]; o, gradO [B, Sq, Hq, headDimV]; lse from
 * LaunchFlashMlaForwardBf16Kernel.  (headDimQk, headDimV): built for (192, 128)
 * and (128, 128); headDimQk up to 128 (or 192) with headDimV up to 128 runs on
 * zero-padded copies.  Other parameters as LaunchFlashGqaBackwardBf16Kernel.
 */
void LaunchFlashMlaBackwardBf16Kernel(const bf16_t* q,
                                      const bf16_t* k,
                                      const bf16_t* v,
                                      const bf16_t* o,
                                      const float* lse,
                                      const bf16_t* gradO,
                                      float scale,
                                      bf16_t* gradQ,
                                      bf16_t* gradK,
                                      bf16_t* gradV,
                                      int batchSize,
                                      int seqLengthQ,
                                      int seqLengthKv,
                                      int numQueryHeads,
                                      int numKvHeads,
                                      int headDimQk,
                                      int headDimV,
                                      bool causal);
