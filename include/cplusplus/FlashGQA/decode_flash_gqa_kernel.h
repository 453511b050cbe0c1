// FlashGQA decode: C++ operator entry point (MI355X / gfx950).
//
// Drop-in for the reference's include/cplusplus/FlashGQA/decode_flash_gqa_kernel.cuh:28-38
// (definition src/cplusplus/FlashGQA/decode_flash_gqa_kernel.cu:405-470): same
// name, same 11 parameters in the same order, same tensor layouts, bf16 in/out,
// fp32 accumulation, asynchronous launch on the default stream, void return.
#pragma once

#include "Utils/utils.h"

// Hardware wavefront width on gfx950 (the reference's header exports its CUDA
// warp width, 32, under this name).
constexpr int WARP_SIZE = 64;

/**
 * @brief Launches the FlashGQA bf16 decoding path (split-KV pass + log-sum-exp combine).
 * @param q Device query tensor [batchSize, numQueryHeads, headDim].
 * @param k Device key tensor [batchSize, seqLength, numKvHeads, headDim].
 * @param v Device value tensor [batchSize, seqLength, numKvHeads, headDim].
 * @param scale Scaling factor applied to QK scores (the reference uses 1/sqrt(headDim)).
 * @param o Device output tensor [batchSize, numQueryHeads, headDim].
 * @param oIntermediate Device fp32 buffer of batchSize*numQueryHeads*headDim floats.
 *        Accepted for signature compatibility and left untouched: the split
 *        partials (two or more fp32 rows per query head, with their max and
 *        sum) do not fit in it and go to the library's fixed device scratch
 *        (fgqa_decode_bf16_noalloc), so the call allocates nothing; calls
 *        that share that scratch must not overlap on the GPU.  Only a plan
 *        beyond it (over 32 MiB of partials) uses the library's cached buffer.
 * @param batchSize Batch size.
 * @param seqLength Sequence length (any value >= 1; the reference required a multiple of 128).
 * @param numQueryHeads Number of query heads.
 * @param numKvHeads Number of KV heads (numQueryHeads / numKvHeads <= 16; the reference required 16).
 * @param headDim Per-head embedding dimension (128).
 *
 * Like the reference, unsupported arguments launch nothing and report nothing
 * through the return value; FlashGqaGetLastStatus() gives the reason.
 */
void LaunchFlashGqaBf16Kernel(const bf16_t* q,
                              const bf16_t* k,
                              const bf16_t* v,
                              float scale,
                              bf16_t* o,
                              float* oIntermediate,
                              int batchSize,
                              int seqLength,
                              int numQueryHeads,
                              int numKvHeads,
                              int headDim);

/**
 * @brief Ragged variant: per-sequence valid lengths (device int32 [batchSize],
 *        each <= maxSeqLength) over K/V padded to maxSeqLength; positions at or
 *        past a sequence's length are never read.  Split partials go to the
 *        library's fixed device scratch, as for LaunchFlashGqaBf16Kernel.  No
 *        reference counterpart.
 */
void LaunchFlashGqaBf16KernelVarlen(const bf16_t* q,
                                    const bf16_t* k,
                                    const bf16_t* v,
                                    float scale,
                                    bf16_t* o,
                                    const int32_t* seqLengths,
                                    int batchSize,
                                    int maxSeqLength,
                                    int numQueryHeads,
                                    int numKvHeads,
                                    int headDim);

/**
 * @brief Paged variant: K/V live in a page cache [numPages, pageSize, numKvHeads, headDim]
 *        (bf16, or OCP fp8 e4m3 bytes when kvFp8 is true, holding K/kScale and
 *        V/vScale); token t of sequence b is slot t % pageSize of page
 *        blockTable[b * maxPagesPerSeq + t / pageSize].  pageSize is a power of
 *        two; seqLengths (device int32 [batchSize]) are each <= maxPagesPerSeq * pageSize.
 *        No reference counterpart: the serving-engine layout of the decode above.
 */
void LaunchFlashGqaBf16KernelPaged(const bf16_t* q,
                                   const void* kCache,
                                   const void* vCache,
                                   bool kvFp8,
                                   float scale,
                                   float kScale,
                                   float vScale,
                                   bf16_t* o,
                                   const int32_t* blockTable,
                                   const int32_t* seqLengths,
                                   int batchSize,
                                   int maxPagesPerSeq,
                                   int pageSize,
                                   int numPages,
                                   int numQueryHeads,
                                   int numKvHeads,
                                   int headDim);

/**
 * @brief Status (an fgqa_status value from fgqa.h) of the calling thread's last
 *        Launch* call in this API: 0 when it launched.
 */
int FlashGqaGetLastStatus();
