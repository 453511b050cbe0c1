"""ctypes binding of libfgqa.so, the C ABI declared in include/fgqa.h.

The library is built in-tree (``make -C cuda_llm_ops_amd/csrc`` or
``__graft_entry__.build()``).  Loading fails loudly when it is missing: there
is no fallback implementation of any entry point.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libfgqa.so")

FGQA_OK = 0
FGQA_ERR_INVALID_ARGUMENT = -1
FGQA_ERR_UNSUPPORTED = -2
FGQA_ERR_WORKSPACE = -3
FGQA_ERR_HIP = -4

# fgqa_kernel_choice: the `kernel` / `dq_kernel` fields (0 = automatic)
FGQA_KERNEL_AUTO = 0
FGQA_KERNEL_WHOLE = 1
FGQA_KERNEL_SPLIT = 2
FGQA_KERNEL_WIDE = 3
FGQA_KERNEL_TALL = 4

_I64x2 = ctypes.c_int64 * 2
_I64x3 = ctypes.c_int64 * 3


class DecodeArgs(ctypes.Structure):
    """Mirror of ``fgqa_decode_args`` (include/fgqa.h)."""
    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("lse", ctypes.c_void_p),
        ("seqlens", ctypes.c_void_p),
        ("batch", ctypes.c_int32),
        ("max_seqlen", ctypes.c_int32),
        ("num_q_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("q_stride", _I64x2),
        ("k_stride", _I64x3),
        ("v_stride", _I64x3),
        ("o_stride", _I64x2),
        ("split_tokens", ctypes.c_int32),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
    ]


class PrefillArgs(ctypes.Structure):
    """Mirror of ``fgqa_prefill_args`` (include/fgqa.h)."""
    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("lse", ctypes.c_void_p),
        ("batch", ctypes.c_int32),
        ("seqlen_q", ctypes.c_int32),
        ("seqlen_kv", ctypes.c_int32),
        ("num_q_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("causal", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("q_stride", _I64x3),
        ("k_stride", _I64x3),
        ("v_stride", _I64x3),
        ("o_stride", _I64x3),
        ("window_size", ctypes.c_int32),
        ("sink", ctypes.c_void_p),
        ("head_dim_v", ctypes.c_int32),
        ("kernel", ctypes.c_int32),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
    ]


# leading bytes of a prefill workspace that must be zero before its first use
FGQA_PREFILL_WORKSPACE_ZERO_BYTES = 4096

FGQA_KV_BF16 = 0
FGQA_KV_FP8_E4M3 = 1


class PagedDecodeArgs(ctypes.Structure):
    """Mirror of ``fgqa_decode_paged_args`` (include/fgqa.h)."""
    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k_cache", ctypes.c_void_p),
        ("v_cache", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("lse", ctypes.c_void_p),
        ("block_table", ctypes.c_void_p),
        ("seqlens", ctypes.c_void_p),
        ("batch", ctypes.c_int32),
        ("max_seqlen", ctypes.c_int32),
        ("num_q_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("page_size", ctypes.c_int32),
        ("num_pages", ctypes.c_int32),
        ("kv_dtype", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("k_scale", ctypes.c_float),
        ("v_scale", ctypes.c_float),
        ("q_stride", _I64x2),
        ("o_stride", _I64x2),
        ("k_stride", _I64x3),
        ("v_stride", _I64x3),
        ("block_table_stride", ctypes.c_int64),
        ("split_tokens", ctypes.c_int32),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
    ]


class BackwardArgs(ctypes.Structure):
    """Mirror of ``fgqa_prefill_backward_args`` (include/fgqa.h)."""
    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("lse", ctypes.c_void_p),
        ("grad_o", ctypes.c_void_p),
        ("grad_q", ctypes.c_void_p),
        ("grad_k", ctypes.c_void_p),
        ("grad_v", ctypes.c_void_p),
        ("batch", ctypes.c_int32),
        ("seqlen_q", ctypes.c_int32),
        ("seqlen_kv", ctypes.c_int32),
        ("num_q_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("causal", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("q_stride", _I64x3),
        ("k_stride", _I64x3),
        ("v_stride", _I64x3),
        ("o_stride", _I64x3),
        ("grad_o_stride", _I64x3),
        ("grad_q_stride", _I64x3),
        ("grad_k_stride", _I64x3),
        ("grad_v_stride", _I64x3),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("window_size", ctypes.c_int32),
        ("head_dim_v", ctypes.c_int32),
        ("kv_head_split", ctypes.c_int32),
        ("dq_kernel", ctypes.c_int32),
    ]


class SparsePrefillArgs(ctypes.Structure):
    """Mirror of ``fgqa_sparse_prefill_args`` (include/fgqa.h)."""
    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("lse", ctypes.c_void_p),
        ("kv_indices", ctypes.c_void_p),
        ("batch", ctypes.c_int32),
        ("seqlen_q", ctypes.c_int32),
        ("seqlen_kv", ctypes.c_int32),
        ("num_q_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("num_sparse_kv", ctypes.c_int32),
        ("causal", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("q_stride", _I64x3),
        ("k_stride", _I64x3),
        ("v_stride", _I64x3),
        ("o_stride", _I64x3),
        ("idx_stride", _I64x3),
    ]


class FgqaError(RuntimeError):
    def __init__(self, status: int, where: str):
        self.status = status
        super().__init__(f"{where}: {status_string(status)} (status {status})")


_lib = None


def lib() -> ctypes.CDLL:
    """Load libfgqa.so (once).  Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `make -C cuda_llm_ops_amd/csrc` "
                "or __graft_entry__.build(); there is no fallback path")
        L = ctypes.CDLL(LIB_PATH)
        L.fgqa_decode_workspace_bytes.restype = ctypes.c_int
        L.fgqa_decode_workspace_bytes.argtypes = [ctypes.POINTER(DecodeArgs), ctypes.POINTER(ctypes.c_size_t)]
        L.fgqa_decode_bf16.restype = ctypes.c_int
        L.fgqa_decode_bf16.argtypes = [ctypes.POINTER(DecodeArgs), ctypes.c_void_p]
        L.fgqa_decode_bf16_noalloc.restype = ctypes.c_int
        L.fgqa_decode_bf16_noalloc.argtypes = [ctypes.POINTER(DecodeArgs), ctypes.c_void_p]
        L.fgqa_prefill_bf16.restype = ctypes.c_int
        L.fgqa_prefill_bf16.argtypes = [ctypes.POINTER(PrefillArgs), ctypes.c_void_p]
        L.fgqa_prefill_kernel_choice.restype = ctypes.c_int
        L.fgqa_prefill_kernel_choice.argtypes = [ctypes.POINTER(PrefillArgs), ctypes.POINTER(ctypes.c_int32)]
        L.fgqa_prefill_kernel_name.restype = ctypes.c_int
        L.fgqa_prefill_kernel_name.argtypes = [ctypes.POINTER(PrefillArgs), ctypes.POINTER(ctypes.c_char_p)]
        L.fgqa_prefill_workspace_bytes.restype = ctypes.c_int
        L.fgqa_prefill_workspace_bytes.argtypes = [ctypes.POINTER(PrefillArgs), ctypes.POINTER(ctypes.c_size_t)]
        L.fgqa_decode_paged_workspace_bytes.restype = ctypes.c_int
        L.fgqa_decode_paged_workspace_bytes.argtypes = [ctypes.POINTER(PagedDecodeArgs),
                                                        ctypes.POINTER(ctypes.c_size_t)]
        L.fgqa_decode_paged.restype = ctypes.c_int
        L.fgqa_decode_paged.argtypes = [ctypes.POINTER(PagedDecodeArgs), ctypes.c_void_p]
        L.fgqa_prefill_backward_workspace_bytes.restype = ctypes.c_int
        L.fgqa_prefill_backward_workspace_bytes.argtypes = [ctypes.POINTER(BackwardArgs),
                                                            ctypes.POINTER(ctypes.c_size_t)]
        L.fgqa_prefill_backward_bf16.restype = ctypes.c_int
        L.fgqa_prefill_backward_bf16.argtypes = [ctypes.POINTER(BackwardArgs), ctypes.c_void_p]
        L.fgqa_sparse_prefill_bf16.restype = ctypes.c_int
        L.fgqa_sparse_prefill_bf16.argtypes = [ctypes.POINTER(SparsePrefillArgs), ctypes.c_void_p]
        L.fgqa_status_string.restype = ctypes.c_char_p
        L.fgqa_status_string.argtypes = [ctypes.c_int]
        L.fgqa_version.restype = ctypes.c_int
        L.fgqa_version.argtypes = []
        L.fgqa_clock_sample.restype = ctypes.c_int
        L.fgqa_clock_sample.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
        _lib = L
    return _lib


def status_string(status: int) -> str:
    return lib().fgqa_status_string(int(status)).decode()


def check(status: int, where: str) -> None:
    if status != FGQA_OK:
        raise FgqaError(status, where)
