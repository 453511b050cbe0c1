// Host-side internals shared by the flash-GQA translation units.
#pragma once

#include <mutex>

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "fgqa.h"
#include "../host/fgqa_plan.h"   // aligned16, ceil_div and the host-only validation / planning

namespace fgqa {

// Compute units of the current device (queried once per device, then cached).
// Returns 0 when the device cannot be queried.
int device_cu_count();

// Library-owned, per-device, grow-only scratch buffer used when a caller
// passes no workspace.  The caller holds workspace_lock() from this call until
// its kernels are launched: growth frees the old buffer (after draining the
// device), so another thread must not grow it in between.  Returns nullptr
// and sets *status on failure.
std::unique_lock<std::mutex> workspace_lock();
void* internal_workspace(size_t bytes, int* status);

// Sets a kernel's dynamic-LDS limit once per device (the attribute is per
// kernel and per device).  slot: a distinct small index per kernel.
int set_kernel_smem_once(int slot, const void* fn, int bytes);

// Copies for head dims the kernels are not built for (flash_gqa_forward.hip):
// B x S x H rows of D bf16 elements at element strides st = {b, s, h} ->
// contiguous rows of `width` (a multiple of 8) zero-padded elements, and
// back (the first D columns of each row).  2-byte accesses: no alignment
// needed.  Launch errors are left for hipGetLastError.
void launch_pad_rows(const void* src, const int64_t* st, int B, int S, int H, int D, int width, void* dst,
                     hipStream_t s);
void launch_unpad_rows(const void* src, int width, void* dst, const int64_t* st, int B, int S, int H, int D,
                       hipStream_t s);

}  // namespace fgqa
