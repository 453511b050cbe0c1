"""MI355X-native flash grouped-query attention (decode incl. paged/fp8 KV caches, causal, sliding-window, MLA and sparse-index prefill, and the causal, sliding-window and MLA prefill backward).

The kernels live in libfgqa.so (HIP, gfx950); ``flash_gqa`` is the Python host
interface over its C ABI (include/fgqa.h).
"""
from ._lib import FgqaError, LIB_PATH, lib, status_string  # noqa: F401
from .flash_gqa import (  # noqa: F401
    backward_workspace_bytes,
    decode_flash_gqa_bshd,
    decode_flash_gqa_paged,
    decode_workspace_bytes,
    flash_gqa_backward_bshd,
    flash_gqa_forward_bshd,
    launch_decode_flash_gqa_bf16_kernel,
    launch_flash_gqa_backward_bf16_kernel,
    launch_flash_gqa_forward_bf16_kernel,
    launch_flash_swa_backward_bf16_kernel,
    launch_flash_swa_forward_bf16_kernel,
    launch_flash_mla_backward_bf16_kernel,
    launch_flash_mla_forward_bf16_kernel,
    launch_flash_sgqa_forward_bf16_kernel,
    flash_sgqa_forward_bshd,
    prepare_sparse_prefill,
    PREFILL_HEAD_DIMS,
    BACKWARD_HEAD_DIMS,
    paged_decode_workspace_bytes,
    prepare_backward,
    prepare_decode,
    prepare_decode_paged,
    prefill_kernel_choice,
    prefill_kernel_name,
    prepare_prefill,
    PreparedLaunch,
)

__version__ = "0.1.0"
