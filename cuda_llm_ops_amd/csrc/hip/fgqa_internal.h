// Host-side internals shared by the flash-GQA translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "fgqa.h"

namespace fgqa {

// Compute units of the current device (queried once per device, then cached).
// Returns 0 when the device cannot be queried.
int device_cu_count();

// Library-owned, per-device, grow-only scratch buffer used when a caller
// passes no workspace.  Allocation happens on first use (or growth) under a
// mutex; the returned pointer stays valid until the next growth.  Returns
// nullptr and sets *status on failure.
void* internal_workspace(size_t bytes, int* status);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace fgqa
