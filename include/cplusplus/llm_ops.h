// Umbrella header for the MI355X flash-GQA C++ operator API.
// Counterpart of the reference's include/cplusplus/cuda_llm_ops.h:8-27,
// restricted to the FlashGQA path.
#pragma once

#include "FlashGQA/decode_flash_gqa_kernel.h"
#include "FlashGQA/flash_gqa_backward_kernel.h"
#include "FlashGQA/flash_gqa_forward_kernel.h"
#include "Utils/utils.h"
