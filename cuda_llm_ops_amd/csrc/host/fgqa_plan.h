// Host-only argument validation and launch planning of the flash-GQA C ABI.
//
// Plain C++17 with no HIP types or calls (the device's CU count comes in as an
// argument), so that the library builds it with g++ and the CPU test suite
// builds it again with AddressSanitizer and UndefinedBehaviorSanitizer and
// drives it with invalid and extreme shapes (tests/host/test_plan.cpp).  The
// HIP translation units call these before any launch: a call they reject
// touches no device memory.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "fgqa.h"

namespace fgqa {

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

namespace plan {

constexpr int kHeadDim = 128;   // D (and Dv) of every kernel; MLA's Q/K head dim is 192
// Longest sequence (and sparse index list) of any entry: token positions and
// their tile-rounded ends stay far inside the kernels' 32-bit integers.
constexpr int kMaxTokens = 1 << 30;

// ---------------------------------------------------------------- decode
constexpr int kDecodeStepRound = 128;     // tokens of one pass of a decode workgroup's 4 waves
constexpr int kDecodeMaxAutoChunk = 4096; // longest split the planner picks by itself
constexpr int kDecodeRaggedChunk = 4096;  // split length for ragged batches (work-list mode)

// Split plan inputs: the sizes alone (shared by the contiguous and paged entries).
struct DecodeShape {
    int batch, max_seqlen, num_q_heads, num_kv_heads, split_tokens;
    bool ragged;   // per-sequence lengths are given
};

struct DecodePlan {
    int chunk;            // tokens per split (a multiple of kDecodeStepRound)
    int nsplit;           // splits per sequence
    bool list;            // ragged batch: a device-built work list of non-empty splits
    size_t part_o_bytes;  // fp32 partial O of every split (nsplit > 1)
    size_t part_ml_bytes; // their (max, sum)
    size_t ws_bytes;      // the workspace: partials, then the list (1 + batch * nsplit int32)
};

int validate_decode(const fgqa_decode_args* a);
int validate_decode_pointers(const fgqa_decode_args* a);
DecodeShape decode_shape(const fgqa_decode_args* a);
// Whether plan_decode reads `cus` for this shape: uniform lengths (or a batch
// too large for a work list) without a forced split size.
bool decode_needs_cus(const DecodeShape& s);
// cus: compute units of the device.  Returns FGQA_OK, FGQA_ERR_HIP when it
// needs cus and cus <= 0, or FGQA_ERR_UNSUPPORTED for a workspace beyond 2^46
// bytes.
int plan_decode(const DecodeShape& s, int cus, DecodePlan* plan);

int validate_paged(const fgqa_decode_paged_args* a);
int validate_paged_pointers(const fgqa_decode_paged_args* a);
// The paged decode always runs the work-list kernel (it needs no CU count): a
// shape the list cannot index (batch >= 2^15 or >= 2^16 splits) is
// FGQA_ERR_UNSUPPORTED.
int plan_paged(const fgqa_decode_paged_args* a, DecodePlan* plan);

// ---------------------------------------------------------------- prefill
constexpr int kPrefillMaxSplit = 128;     // most unit pairs whose units a launch may split
constexpr int kPrefillPartFloats = 2 * 4 * 66 * 64;   // floats of one partial-result slot
constexpr size_t kPrefillZeroBytes = FGQA_PREFILL_WORKSPACE_ZERO_BYTES;

int validate_prefill(const fgqa_prefill_args* a);
// Head-dim pairs up to 256 other than the built ones (Q/K 128, 192 or 256
// with V/O 128): the call copies Q and K into zero-padded rows of
// padded_dk() = 128, 192 or 256 elements and V into rows of padded_dv() =
// 128 or 256, runs the built kernels on the copies (once per 128 columns of
// V) and copies the first head_dim_v columns of O back.  (Zero columns add
// nothing to Q.K^T, and the padded columns of O are dropped; the reference's
// Triton kernels pad their head-dim blocks to a power of two the same way,
// src/python/Triton/flash_gqa_kernel.py:266-269, 80-94.)
bool prefill_padded(const fgqa_prefill_args* a);
int padded_dk(const fgqa_prefill_args* a);
int padded_dv(const fgqa_prefill_args* a);
// The call on the copies (head dims padded_dk() and 128, V and O rows of
// padded_dv() elements): same shape and options, contiguous strides, null
// tensor pointers and no workspace (the caller fills them in, and offsets V
// and O by 128 columns for the second launch when padded_dv() is 256).
fgqa_prefill_args padded_args(const fgqa_prefill_args* a);
// Byte offsets in the padded call's workspace: the merge scratch of the
// (128, 128) call at 0 (its zeroed prefix first; at least the prefix when
// that call merges nothing), then the copies of Q, K, V and O, each 256-byte
// aligned.
struct PadLayout {
    size_t q, k, v, o, total;
};
PadLayout pad_layout(const fgqa_prefill_args* a, size_t merge_bytes);
// fgqa_prefill_workspace_bytes of a validated call.
size_t prefill_workspace_bytes(const fgqa_prefill_args* a, int cus);
// Unit pairs of the 256-row kernels (units of up to 8 heads of a KV group).
int64_t wide_pairs(const fgqa_prefill_args* a);
// Whether the 256-row kernels run unit pairs on two workgroups each (at most
// kPrefillMaxSplit pairs and one pair per two CUs; the tall kernel only under
// a causal mask) rather than whole units on a persistent grid.
bool wide_on_pairs(const fgqa_prefill_args* a, int cus);
bool tall_on_pairs(const fgqa_prefill_args* a, int cus);
// The kernel shape (an fgqa_kernel_choice other than AUTO) of a validated call.
int prefill_choice(const fgqa_prefill_args* a, int cus);
// Merge scratch bytes of a validated call with kernel `choice`.
size_t merge_scratch_bytes(const fgqa_prefill_args* a, int choice, int cus);
constexpr size_t merge_scratch_bytes_for(int64_t pairs) {
    return kPrefillZeroBytes + (size_t)pairs * 2 * kPrefillPartFloats * sizeof(float);
}
// The kernel function a validated call launches (static storage).
const char* prefill_kernel_name(const fgqa_prefill_args* a, int cus);

// ---------------------------------------------------------------- backward
constexpr int kBackwardKvKeys = 128;      // keys per dK/dV workgroup

struct BwdPlan {
    int n_hsplit;   // query-head subsets per KV head in the dK/dV pass (1: dK/dV written directly)
    size_t stat_bytes, part_k_bytes, part_v_bytes, ws_bytes;
};

int validate_backward(const fgqa_prefill_backward_args* a);
// Q/K head dims up to 128 (or 192) with V/O head dims up to 128, other than
// the built (128, 128) and (192, 128): the call copies Q, K, V, O and dO
// into zero-padded rows (Q/K of backward_padded_dk() = 128 or 192 elements,
// the others of 128), runs the built kernels on the copies and copies the
// first head_dim / head_dim_v columns of dQ, dK and dV back.  Zero columns
// of Q and K add nothing to the scores, zero columns of O and dO nothing to
// the row statistic sum(O * dO), and the padded gradient columns are dropped.
bool backward_padded(const fgqa_prefill_backward_args* a);
int backward_padded_dk(const fgqa_prefill_backward_args* a);
// The call on the copies: same shape and options, contiguous strides, null
// tensor pointers and no workspace (the caller fills them in).
fgqa_prefill_backward_args backward_padded_args(const fgqa_prefill_backward_args* a);
// Byte offsets in the padded call's workspace: the built call's workspace
// (ws_bytes) at 0, then the copies of Q, K, V, O, dO, dQ, dK, dV, each
// 256-byte aligned.
struct BwdPadLayout {
    size_t q, k, v, o, dout, dq, dk, dv, total;
};
BwdPadLayout backward_pad_layout(const fgqa_prefill_backward_args* a, size_t ws_bytes);
// fgqa_prefill_backward_workspace_bytes of a validated call.
size_t backward_workspace_bytes(const fgqa_prefill_backward_args* a, int cus);
int validate_backward_pointers(const fgqa_prefill_backward_args* a);
BwdPlan plan_backward(const fgqa_prefill_backward_args* a, int cus);
// FGQA_ERR_UNSUPPORTED when a grid or a row count of the launches planned by
// `pl` reaches 2^31 (the kernels index units and rows with 32-bit integers).
int check_backward_grid(const fgqa_prefill_backward_args* a, const BwdPlan& pl);

// ---------------------------------------------------------------- sparse
constexpr int kSparseWaves = 4;           // waves (one work item each) per sparse workgroup

int validate_sparse(const fgqa_sparse_prefill_args* a);

}  // namespace plan
}  // namespace fgqa
