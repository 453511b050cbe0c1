// Host entry of the 64-rows-per-wave prefill kernels (flash_gqa_forward_tall.hip).
#pragma once

#include <hip/hip_runtime.h>

#include "prefill_common.h"

namespace fgqa {

// Dynamic LDS bytes of a tall workgroup.
extern const int kTallSmemBytes;

// Launches the tall prefill on `s` for the 256-row unit geometry in `p` (head
// dim 128, no window or sink).  pairs: unit pairs on two workgroups of one XCD
// with split units merged through p.wide_part / p.wide_ctr (at most
// kPwMaxSplit pairs); else whole units on min(units, cus) persistent
// workgroups.  Returns FGQA_OK or FGQA_ERR_HIP.
int launch_prefill_tall(const PrefillParams& p, bool pairs, int cus, hipStream_t s);

}  // namespace fgqa
