"""Python host interface of the flash-GQA path, over the C ABI (libfgqa.so).

Two families of entry points:

* Mirrors of the reference's Python launchers, same names, argument meaning and
  ``ValueError`` behaviour, BHSD layout:
    - ``launch_flash_gqa_forward_bf16_kernel`` <- src/python/Triton/flash_gqa_kernel.py:185-338
    - ``launch_decode_flash_gqa_bf16_kernel``  <- src/python/Triton/decode_flash_gqa_kernel.py:137-196
    - ``launch_flash_gqa_backward_bf16_kernel`` <- src/python/Triton/flash_gqa_backward_kernel.py:312-478
    - ``launch_flash_swa_forward_bf16_kernel``  <- src/python/Triton/SWA/flash_swa_kernel.py:188-370
    - ``launch_flash_mla_forward_bf16_kernel``  <- src/python/Triton/flash_mla_kernel.py:315-508
    - ``launch_flash_sgqa_forward_bf16_kernel`` <- src/python/Triton/SparseGQA/flash_sgqa_kernel.py:202-396
* The C++ layouts of the reference's C++ decode entry point (Q/O ``[B,Hq,D]``,
  K/V ``[B,S,Hkv,D]``, decode_flash_gqa_kernel.cuh:28-38) and of the new C++
  prefill entry point (BSHD):
    - ``decode_flash_gqa_bshd``  (adds per-sequence lengths and an LSE output)
    - ``decode_flash_gqa_paged`` (paged KV cache with a block table, bf16 or fp8 e4m3)
    - ``flash_gqa_forward_bshd``
    - ``flash_gqa_backward_bshd``

PyTorch only provides device memory and the current stream; every launch goes
through ``fgqa_decode_bf16`` / ``fgqa_prefill_bf16`` / ``fgqa_prefill_backward_bf16``.
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _lib

__all__ = [
    "launch_flash_gqa_forward_bf16_kernel",
    "launch_decode_flash_gqa_bf16_kernel",
    "launch_flash_gqa_backward_bf16_kernel",
    "launch_flash_swa_forward_bf16_kernel",
    "launch_flash_mla_forward_bf16_kernel",
    "launch_flash_sgqa_forward_bf16_kernel",
    "flash_sgqa_forward_bshd",
    "prepare_sparse_prefill",
    "PREFILL_HEAD_DIMS",
    "BACKWARD_HEAD_DIMS",
    "decode_flash_gqa_bshd",
    "decode_flash_gqa_paged",
    "paged_decode_workspace_bytes",
    "prepare_decode_paged",
    "flash_gqa_forward_bshd",
    "flash_gqa_backward_bshd",
    "decode_workspace_bytes",
    "backward_workspace_bytes",
    "prepare_decode",
    "prepare_prefill",
    "prefill_kernel_choice",
    "prefill_kernel_name",
    "prepare_backward",
    "PreparedLaunch",
]


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _require_cuda(*ts: torch.Tensor) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("Flash GQA tensors must live on the GPU")


def _kernel_ready(t: torch.Tensor) -> bool:
    """Head dim contiguous, 16-byte aligned base, strides multiple of 8 elements."""
    if t.stride(-1) != 1 or t.data_ptr() % 16 != 0:
        return False
    return all(s % 8 == 0 for s in t.stride()[:-1])


def _prep(t: torch.Tensor) -> torch.Tensor:
    return t if _kernel_ready(t) else t.contiguous()


# --------------------------------------------------------------------------- decode
def _decode_args(q, k, v, o, scale, seqlens, lse, split_tokens, workspace) -> _lib.DecodeArgs:
    B, Hq, D = q.shape
    _, S, Hkv, _ = k.shape
    a = _lib.DecodeArgs()
    a.q, a.k, a.v, a.o = _ptr(q), _ptr(k), _ptr(v), _ptr(o)
    a.lse = _ptr(lse)
    a.seqlens = _ptr(seqlens)
    a.batch, a.max_seqlen, a.num_q_heads, a.num_kv_heads, a.head_dim = B, S, Hq, Hkv, D
    a.scale = float(scale)
    a.q_stride[:] = [q.stride(0), q.stride(1)]
    a.k_stride[:] = [k.stride(0), k.stride(1), k.stride(2)]
    a.v_stride[:] = [v.stride(0), v.stride(1), v.stride(2)]
    a.o_stride[:] = [o.stride(0), o.stride(1)]
    a.split_tokens = int(split_tokens)
    if workspace is not None:
        a.workspace = workspace.data_ptr()
        a.workspace_bytes = workspace.numel() * workspace.element_size()
    return a


def decode_workspace_bytes(batch, max_seqlen, num_q_heads, num_kv_heads, head_dim=128, split_tokens=0,
                           ragged=False) -> int:
    """Bytes of scratch ``decode_flash_gqa_bshd`` needs for a caller workspace.
    ``ragged``: the call will pass per-sequence lengths (``seqlens``)."""
    a = _lib.DecodeArgs()
    if ragged:
        a.seqlens = 16   # only tested for NULL by the size query, never read
    a.batch, a.max_seqlen, a.num_q_heads, a.num_kv_heads, a.head_dim = (
        batch, max_seqlen, num_q_heads, num_kv_heads, head_dim)
    a.scale = 1.0
    a.q_stride[:] = [num_q_heads * head_dim, head_dim]
    a.o_stride[:] = [num_q_heads * head_dim, head_dim]
    a.k_stride[:] = [max_seqlen * num_kv_heads * head_dim, num_kv_heads * head_dim, head_dim]
    a.v_stride[:] = list(a.k_stride)
    a.split_tokens = int(split_tokens)
    n = ctypes.c_size_t(0)
    _lib.check(_lib.lib().fgqa_decode_workspace_bytes(ctypes.byref(a), ctypes.byref(n)),
               "fgqa_decode_workspace_bytes")
    return int(n.value)


def _decode_prepare(q, k, v, scale, out, seqlens, lse, split_tokens, workspace):
    """Validate decode arguments and build the C ABI argument block (no launch)."""
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        raise ValueError("Flash GQA decoding expects bf16 inputs")
    if q.dim() != 3 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("expected q [B,Hq,D] and k/v [B,S,Hkv,D]")
    _require_cuda(q, k, v)
    B, Hq, D = q.shape
    if k.shape != v.shape or k.shape[0] != B or k.shape[3] != D:
        raise ValueError("K and V must be [B, S, Hkv, D] matching Q")
    if Hq % k.shape[2] != 0:
        raise ValueError("Query heads must be divisible by KV heads")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    q, k, v = _prep(q), _prep(k), _prep(v)
    if out is None:
        out = torch.empty((B, Hq, D), device=q.device, dtype=torch.bfloat16)
    elif out.shape != (B, Hq, D) or out.dtype != torch.bfloat16 or not _kernel_ready(out):
        raise ValueError("out must be a bf16 [B, Hq, D] tensor with contiguous rows")
    if seqlens is not None:
        if seqlens.dtype != torch.int32 or seqlens.shape != (B,) or not seqlens.is_contiguous():
            raise ValueError("seqlens must be a contiguous int32 [B] tensor")
        _require_cuda(seqlens)
    if lse is not None and (lse.dtype != torch.float32 or lse.shape != (B, Hq) or not lse.is_contiguous()):
        raise ValueError("lse must be a contiguous fp32 [B, Hq] tensor")
    a = _decode_args(q, k, v, out, scale, seqlens, lse, split_tokens, workspace)
    # keep every tensor the argument block points at alive with it
    return a, out, (q, k, v, out, seqlens, lse, workspace)


def decode_flash_gqa_bshd(q, k, v, scale=None, out=None, seqlens=None, lse=None,
                          split_tokens=0, workspace=None):
    """Single-token GQA decode in the reference C++ layout.

    q: bf16 [B, Hq, D]; k, v: bf16 [B, S_max, Hkv, D]; seqlens: optional int32
    [B] device tensor of valid lengths; lse: optional fp32 [B, Hq] output.
    Returns ``out`` (bf16 [B, Hq, D]).
    """
    a, out, _keep = _decode_prepare(q, k, v, scale, out, seqlens, lse, split_tokens, workspace)
    _lib.check(_lib.lib().fgqa_decode_bf16(ctypes.byref(a), ctypes.c_void_p(_stream())), "fgqa_decode_bf16")
    return out


class PreparedLaunch:
    """A launch validated once whose C ABI argument block is kept: calling it
    re-launches the same work on torch's current stream with only the cost of
    one C call (for serving loops and benchmarks that repeat a step on the same
    buffers).  The tensors it was built from stay referenced by it."""

    def __init__(self, fn, args, keep, out, where):
        self._fn = fn
        self._args = args
        self._ref = ctypes.byref(args)
        self._keep = keep
        self.out = out
        self._where = where

    def __call__(self):
        st = self._fn(self._ref, ctypes.c_void_p(_stream()))
        if st != _lib.FGQA_OK:
            raise _lib.FgqaError(st, self._where)
        return self.out


def prepare_decode(q, k, v, scale=None, out=None, seqlens=None, lse=None, split_tokens=0, workspace=None):
    """``decode_flash_gqa_bshd`` validated once; returns a ``PreparedLaunch``."""
    a, out, keep = _decode_prepare(q, k, v, scale, out, seqlens, lse, split_tokens, workspace)
    return PreparedLaunch(_lib.lib().fgqa_decode_bf16, a, keep, out, "fgqa_decode_bf16")


# --------------------------------------------------------------------------- paged decode
_PAGED_DTYPES = {torch.bfloat16: _lib.FGQA_KV_BF16}
if hasattr(torch, "float8_e4m3fn"):
    _PAGED_DTYPES[torch.float8_e4m3fn] = _lib.FGQA_KV_FP8_E4M3


def _paged_args(q, kc, vc, block_table, seqlens, o, lse, scale, k_scale, v_scale, max_seqlen,
                split_tokens, workspace):
    B, Hq, D = q.shape
    num_pages, page_size, Hkv, _ = kc.shape
    a = _lib.PagedDecodeArgs()
    a.q, a.k_cache, a.v_cache, a.o, a.lse = _ptr(q), _ptr(kc), _ptr(vc), _ptr(o), _ptr(lse)
    a.block_table, a.seqlens = _ptr(block_table), _ptr(seqlens)
    a.batch, a.max_seqlen, a.num_q_heads, a.num_kv_heads, a.head_dim = B, max_seqlen, Hq, Hkv, D
    a.page_size, a.num_pages = page_size, num_pages
    a.kv_dtype = _PAGED_DTYPES[kc.dtype]
    a.scale, a.k_scale, a.v_scale = float(scale), float(k_scale), float(v_scale)
    a.q_stride[:] = [q.stride(0), q.stride(1)]
    a.o_stride[:] = [o.stride(0), o.stride(1)]
    a.k_stride[:] = [kc.stride(0), kc.stride(1), kc.stride(2)]
    a.v_stride[:] = [vc.stride(0), vc.stride(1), vc.stride(2)]
    a.block_table_stride = block_table.stride(0) if block_table.dim() == 2 else 0
    a.split_tokens = int(split_tokens)
    if workspace is not None:
        a.workspace = workspace.data_ptr()
        a.workspace_bytes = workspace.numel() * workspace.element_size()
    return a


def paged_decode_workspace_bytes(batch, max_seqlen, num_q_heads, num_kv_heads, page_size, head_dim=128,
                                 split_tokens=0) -> int:
    """Bytes of scratch ``decode_flash_gqa_paged`` needs for a caller workspace."""
    a = _lib.PagedDecodeArgs()
    a.batch, a.max_seqlen, a.num_q_heads, a.num_kv_heads, a.head_dim = (
        batch, max_seqlen, num_q_heads, num_kv_heads, head_dim)
    a.page_size, a.num_pages, a.kv_dtype = page_size, 1, _lib.FGQA_KV_BF16
    a.scale = a.k_scale = a.v_scale = 1.0
    a.block_table_stride = -(-max_seqlen // page_size) if max_seqlen > 0 else 0
    a.split_tokens = int(split_tokens)
    n = ctypes.c_size_t(0)
    _lib.check(_lib.lib().fgqa_decode_paged_workspace_bytes(ctypes.byref(a), ctypes.byref(n)),
               "fgqa_decode_paged_workspace_bytes")
    return int(n.value)


def _paged_prepare(q, k_cache, v_cache, block_table, seqlens, scale, k_scale, v_scale, out, lse, max_seqlen,
                   split_tokens, workspace):
    if q.dtype != torch.bfloat16:
        raise ValueError("paged decode expects a bf16 query")
    if k_cache.dtype != v_cache.dtype or k_cache.dtype not in _PAGED_DTYPES:
        raise ValueError("k_cache and v_cache must both be bf16 or float8_e4m3fn")
    if q.dim() != 3 or k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        raise ValueError("expected q [B,Hq,D] and k_cache/v_cache [num_pages, page_size, Hkv, D]")
    _require_cuda(q, k_cache, v_cache, block_table, seqlens)
    B, Hq, D = q.shape
    if k_cache.shape[3] != D:
        raise ValueError("the caches' head_dim must match Q")
    if Hq % k_cache.shape[2] != 0:
        raise ValueError("Query heads must be divisible by KV heads")
    if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.shape[0] != B \
            or block_table.stride(1) != 1:
        raise ValueError("block_table must be an int32 [B, max_pages] tensor with contiguous rows")
    if seqlens.dtype != torch.int32 or seqlens.shape != (B,) or not seqlens.is_contiguous():
        raise ValueError("seqlens must be a contiguous int32 [B] tensor")
    if k_cache.stride(3) != 1 or v_cache.stride(3) != 1:
        raise ValueError("the caches' head_dim must be contiguous")
    page_size = k_cache.shape[1]
    if max_seqlen is None:
        max_seqlen = block_table.shape[1] * page_size
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    q = _prep(q)
    if out is None:
        out = torch.empty((B, Hq, D), device=q.device, dtype=torch.bfloat16)
    elif out.shape != (B, Hq, D) or out.dtype != torch.bfloat16 or not _kernel_ready(out):
        raise ValueError("out must be a bf16 [B, Hq, D] tensor with contiguous rows")
    if lse is not None and (lse.dtype != torch.float32 or lse.shape != (B, Hq) or not lse.is_contiguous()):
        raise ValueError("lse must be a contiguous fp32 [B, Hq] tensor")
    a = _paged_args(q, k_cache, v_cache, block_table, seqlens, out, lse, scale, k_scale, v_scale,
                    int(max_seqlen), split_tokens, workspace)
    return a, out, (q, k_cache, v_cache, block_table, seqlens, out, lse, workspace)


def decode_flash_gqa_paged(q, k_cache, v_cache, block_table, seqlens, scale=None, k_scale=1.0, v_scale=1.0,
                           out=None, lse=None, max_seqlen=None, split_tokens=0, workspace=None):
    """Single-token GQA decode over a paged KV cache.

    q: bf16 [B, Hq, D]; k_cache, v_cache: [num_pages, page_size, Hkv, D] in
    bf16 or torch.float8_e4m3fn (holding K / k_scale and V / v_scale);
    block_table: int32 [B, max_pages] (token t of sequence b is slot
    t % page_size of page block_table[b, t // page_size]); seqlens: int32 [B].
    page_size must be a power of two.  Returns ``out`` (bf16 [B, Hq, D]).
    """
    a, out, _keep = _paged_prepare(q, k_cache, v_cache, block_table, seqlens, scale, k_scale, v_scale, out,
                                   lse, max_seqlen, split_tokens, workspace)
    _lib.check(_lib.lib().fgqa_decode_paged(ctypes.byref(a), ctypes.c_void_p(_stream())), "fgqa_decode_paged")
    return out


def prepare_decode_paged(q, k_cache, v_cache, block_table, seqlens, scale=None, k_scale=1.0, v_scale=1.0,
                         out=None, lse=None, max_seqlen=None, split_tokens=0, workspace=None):
    """``decode_flash_gqa_paged`` validated once; returns a ``PreparedLaunch``."""
    a, out, keep = _paged_prepare(q, k_cache, v_cache, block_table, seqlens, scale, k_scale, v_scale, out, lse,
                                  max_seqlen, split_tokens, workspace)
    return PreparedLaunch(_lib.lib().fgqa_decode_paged, a, keep, out, "fgqa_decode_paged")


def launch_decode_flash_gqa_bf16_kernel(q, k, v, out=None):
    """Mirror of the reference's Triton decode launcher
    (src/python/Triton/decode_flash_gqa_kernel.py:137-196): BHSD tensors
    q [B, Hq, Sq, D] (query row 0 of each head is decoded, as in the reference
    kernel :76-78,111-113), k/v [B, Hkv, S, D]; contiguous inputs; scale 1/sqrt(D)."""
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        raise ValueError("Flash GQA decoding expects bf16 inputs")
    if not (q.is_contiguous() and k.is_contiguous() and v.is_contiguous()):
        raise ValueError("Flash GQA decoding kernel expects contiguous Q/K/V tensors")
    batch, q_heads, seqlen_q, head_dim = q.shape
    k_batch, num_kv_heads, seqlen_kv, k_head_dim = k.shape
    v_batch, v_heads, v_seqlen, v_head_dim = v.shape
    if batch != k_batch or batch != v_batch:
        raise ValueError("Q, K, and V must share batch dimension")
    if seqlen_kv != v_seqlen:
        raise ValueError("K and V must share sequence length")
    if k_head_dim != v_head_dim or head_dim != k_head_dim:
        raise ValueError("Q, K, and V must share head_dim")
    if v_heads != num_kv_heads:
        raise ValueError("K and V must share number of KV heads")
    if q_heads % num_kv_heads != 0:
        raise ValueError("Query heads must be divisible by KV heads")
    if out is None:
        out = torch.empty_like(q)
    if not out.is_contiguous():
        raise ValueError("Output tensor must be contiguous")
    _require_cuda(q, k, v, out)
    # BHSD views in the C++ decode's index order: q/o [B, Hq, D] at row 0,
    # k/v [B, S, Hkv, D] by permuting strides (no copy).
    q3 = q[:, :, 0, :]
    o3 = out[:, :, 0, :]
    k4 = k.permute(0, 2, 1, 3)
    v4 = v.permute(0, 2, 1, 3)
    decode_flash_gqa_bshd(q3, k4, v4, scale=1.0 / math.sqrt(head_dim), out=o3)
    return out


# --------------------------------------------------------------------------- prefill
def _kernel_choice(kernel) -> int:
    """'auto' / 'whole' / 'split' (or the FGQA_KERNEL_* value) -> the C ABI value."""
    names = {"auto": _lib.FGQA_KERNEL_AUTO, "whole": _lib.FGQA_KERNEL_WHOLE, "split": _lib.FGQA_KERNEL_SPLIT,
             "wide": _lib.FGQA_KERNEL_WIDE, "tall": _lib.FGQA_KERNEL_TALL}
    if isinstance(kernel, str):
        if kernel not in names:
            raise ValueError(f"kernel must be one of {sorted(names)}")
        return names[kernel]
    return int(kernel)


def _prefill_args(q, k, v, o, lse, scale, causal, layout, window_size=0, sink=None,
                  kernel="auto") -> _lib.PrefillArgs:
    """C ABI argument block for q/k/v/o 4-D in `layout` ('bshd' or 'bhsd')."""
    def sbh(t):
        if layout == "bshd":
            return [t.stride(0), t.stride(1), t.stride(2)]
        return [t.stride(0), t.stride(2), t.stride(1)]

    if layout == "bshd":
        B, Sq, Hq, D = q.shape
        _, Skv, Hkv, _ = k.shape
    else:
        B, Hq, Sq, D = q.shape
        _, Hkv, Skv, _ = k.shape
    a = _lib.PrefillArgs()
    a.q, a.k, a.v, a.o, a.lse = _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(lse)
    a.batch, a.seqlen_q, a.seqlen_kv = B, Sq, Skv
    a.num_q_heads, a.num_kv_heads, a.head_dim = Hq, Hkv, D
    a.head_dim_v = v.shape[3]
    a.causal = 1 if causal else 0
    a.scale = float(scale)
    a.q_stride[:] = sbh(q)
    a.k_stride[:] = sbh(k)
    a.v_stride[:] = sbh(v)
    a.o_stride[:] = sbh(o)
    a.window_size = int(window_size)
    a.sink = _ptr(sink)
    a.kernel = _kernel_choice(kernel)
    return a


# (Q/K head dim, V/O head dim) pairs the prefill kernels are built for:
# GQA, MLA (src/python/Triton/flash_mla_kernel.py's 192 / 128) and Q/K 256.
# The forward also takes any other pair with both dims at most 256: the
# library runs it on copies zero-padded to a built pair (V in 128-column
# halves), as the reference's Triton launcher pads its head-dim blocks to a
# power of two (src/python/Triton/flash_gqa_kernel.py:266-269).  The
# backward is built for (128, 128) and (192, 128), and takes Q/K head dims
# up to 128 (or 192) with V/O head dims up to 128 on padded copies.
PREFILL_HEAD_DIMS = ((128, 128), (192, 128), (256, 128))
BACKWARD_HEAD_DIMS = ((128, 128), (192, 128))


def _padded_head_dims(dqk, dv):
    return 0 < dqk <= 256 and 0 < dv <= 256 and (dqk, dv) not in PREFILL_HEAD_DIMS


def _padded_backward_head_dims(dqk, dv):
    return (0 < dqk <= 128 or dqk == 192) and 0 < dv <= 128 and (dqk, dv) not in BACKWARD_HEAD_DIMS


def _check_head_dims(dqk, dv, window_size=0, sink=None, padded_ok=False):
    """padded_ok: the forward's rule (any pair up to 256); else the backward's."""
    built = PREFILL_HEAD_DIMS if padded_ok else BACKWARD_HEAD_DIMS
    padded = _padded_head_dims(dqk, dv) if padded_ok else _padded_backward_head_dims(dqk, dv)
    if (dqk, dv) not in built and not padded:
        more = ", or both at most 256" if padded_ok else ", or Q/K up to 128 (or 192) with V/O up to 128"
        raise ValueError(f"(head_dim_qk, head_dim_v) = ({dqk}, {dv}) is not supported; "
                         f"supported: {built}{more}")
    # the 192 kernels (MLA, and Q/K 192 with any V dim) have no window / sink form
    if dqk == 192 and (int(window_size) != 0 or sink is not None):
        raise ValueError("a sliding window or sink is not supported with head_dim_qk 192")


def _out_ready(t, dqk, dv) -> bool:
    """A prefill output the library can write: kernel-ready rows, or (head
    dims run on padded copies, whose O is copied out element by element) rows
    whose head dim is contiguous."""
    return _kernel_ready(t) or (_padded_head_dims(dqk, dv) and t.stride(-1) == 1)


# Merge scratch of the prefill kernels that split a unit over two workgroups
# (include/fgqa.h, fgqa_prefill_args.workspace): one per (device, stream), so
# calls on different streams never share one, and calls on one stream run in
# order.
_PREFILL_WORKSPACES = {}


def _new_prefill_workspace(nbytes, device):
    """Uninitialised device bytes (torch's blocks are 512-byte aligned) whose
    arrival-counter prefix is zeroed on the current stream, before any launch
    that uses it."""
    ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
    ws[:_lib.FGQA_PREFILL_WORKSPACE_ZERO_BYTES].zero_()
    return ws


def _attach_prefill_workspace(a, device, own=False):
    """Sets `a`'s workspace for the kernel its call runs on this device: the
    current stream's cached one, or (own) a new one; None when the kernel
    needs none.  Returns the tensor, which the caller keeps alive."""
    n = ctypes.c_size_t(0)
    _lib.check(_lib.lib().fgqa_prefill_workspace_bytes(ctypes.byref(a), ctypes.byref(n)),
               "fgqa_prefill_workspace_bytes")
    if n.value == 0:
        return None
    if own:
        ws = _new_prefill_workspace(n.value, device)
    else:
        key = (device.index, _stream())
        ws = _PREFILL_WORKSPACES.get(key)
        if ws is None or ws.numel() < n.value:
            ws = _new_prefill_workspace(n.value, device)
            _PREFILL_WORKSPACES[key] = ws
    a.workspace = ws.data_ptr()
    a.workspace_bytes = ws.numel()
    return ws


def _prefill(q, k, v, o, lse, scale, causal, layout, window_size=0, sink=None):
    a = _prefill_args(q, k, v, o, lse, scale, causal, layout, window_size, sink)
    _attach_prefill_workspace(a, q.device)
    _lib.check(_lib.lib().fgqa_prefill_bf16(ctypes.byref(a), ctypes.c_void_p(_stream())), "fgqa_prefill_bf16")


def _check_sink(sink, hq, dev):
    if sink is None:
        return None
    if not isinstance(sink, torch.Tensor) or sink.dim() != 1 or sink.numel() != hq:
        raise ValueError(f"sink must be a 1D tensor with {hq} elements")
    if sink.device != dev:
        raise ValueError("sink must be on the same device as Q")
    return sink.to(torch.float32).contiguous()


def _prefill_bshd_prepare(q, k, v, scale, out, lse, causal, window_size=0, sink=None, kernel="auto"):
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        raise ValueError("Flash GQA forward expects bf16 inputs")
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("expected 4-D BSHD tensors")
    _require_cuda(q, k, v)
    B, Sq, Hq, D = q.shape
    Dv = v.shape[3]
    if k.shape[:3] != v.shape[:3] or k.shape[0] != B or k.shape[3] != D:
        raise ValueError("K must be [B, Skv, Hkv, D] matching Q and V [B, Skv, Hkv, Dv]")
    if Hq % k.shape[2] != 0:
        raise ValueError("Query heads must be divisible by KV heads")
    _check_head_dims(D, Dv, window_size, sink, padded_ok=True)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    q, k, v = _prep(q), _prep(k), _prep(v)
    if out is None:
        out = torch.empty((B, Sq, Hq, Dv), device=q.device, dtype=torch.bfloat16)
    elif out.shape != (B, Sq, Hq, Dv) or out.dtype != torch.bfloat16 or not _out_ready(out, D, Dv):
        raise ValueError("Output must be a bf16 [batch, seqlen_q, q_heads, head_dim_v] tensor with contiguous rows")
    if lse is None:
        lse = torch.empty((B, Hq, Sq), device=q.device, dtype=torch.float32)
    elif lse.shape != (B, Hq, Sq) or lse.dtype != torch.float32 or not lse.is_contiguous():
        raise ValueError("LSE must be a contiguous fp32 [batch, q_heads, seqlen_q] tensor")
    sink = _check_sink(sink, Hq, q.device)
    a = _prefill_args(q, k, v, out, lse, scale, causal, "bshd", window_size, sink, kernel)
    return a, out, lse, (q, k, v, out, lse, sink)


def flash_gqa_forward_bshd(q, k, v, scale=None, out=None, lse=None, causal=True, window_size=0, sink=None,
                           kernel="auto"):
    """Prefill forward in BSHD: q [B,Sq,Hq,D], k [B,Skv,Hkv,D], v [B,Skv,Hkv,Dv]
    -> (out [B,Sq,Hq,Dv], lse [B,Hq,Sq]).  (D, Dv) is (128, 128), or (192, 128)
    for MLA.  window_size > 0 (causal only): row i sees keys [i - window_size + 1, i];
    sink: optional fp32 [Hq] added to the softmax denominator as sink * exp(-max)
    (the reference's SWA kernel); both need D == Dv == 128.
    kernel: 'auto', or 'whole' / 'split' / 'wide' / 'tall' to force one kernel
    shape (the window / sink variant has no split or tall form).  The kernels
    that merge a unit's two halves through device memory get a workspace held
    per (device, stream), so calls on different streams may overlap."""
    a, out, lse, _keep = _prefill_bshd_prepare(q, k, v, scale, out, lse, causal, window_size, sink, kernel)
    _attach_prefill_workspace(a, q.device)
    _lib.check(_lib.lib().fgqa_prefill_bf16(ctypes.byref(a), ctypes.c_void_p(_stream())), "fgqa_prefill_bf16")
    return out, lse


def prepare_prefill(q, k, v, scale=None, out=None, lse=None, causal=True, window_size=0, sink=None,
                    kernel="auto"):
    """``flash_gqa_forward_bshd`` validated once; returns a ``PreparedLaunch``
    whose ``out`` is the output tensor (the LSE tensor is ``.lse``).  It owns
    its merge workspace (when its kernel needs one), so its calls must not
    overlap on the GPU, as they would share ``out`` anyway."""
    a, out, lse, keep = _prefill_bshd_prepare(q, k, v, scale, out, lse, causal, window_size, sink, kernel)
    keep = keep + (_attach_prefill_workspace(a, q.device, own=True),)
    pl = PreparedLaunch(_lib.lib().fgqa_prefill_bf16, a, keep, out, "fgqa_prefill_bf16")
    pl.lse = lse
    return pl


def _prefill_query_args(q, k, v, causal, window_size, sink, kernel):
    """The argument block of a BSHD prefill call for queries that launch
    nothing: no output tensors are allocated (O's pointer is Q's, its
    strides the contiguous ones, LSE none)."""
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("expected 4-D BSHD tensors")
    B, Sq, Hq, _ = q.shape
    Dv = v.shape[3]
    a = _prefill_args(q, k, v, q, None, 1.0, causal, "bshd", window_size, sink, kernel)
    a.o_stride[:] = [Sq * Hq * Dv, Hq * Dv, Dv]
    return a


def prefill_kernel_choice(q, k, v, causal=True, window_size=0, sink=None, kernel="auto") -> str:
    """The kernel shape ('whole', 'split', 'wide' or 'tall')
    ``flash_gqa_forward_bshd`` runs for these tensors on the current device
    (what ``kernel='auto'`` resolves to); launches and allocates nothing."""
    a = _prefill_query_args(q, k, v, causal, window_size, sink, kernel)
    c = ctypes.c_int32(0)
    st = _lib.lib().fgqa_prefill_kernel_choice(ctypes.byref(a), ctypes.byref(c))
    if st != _lib.FGQA_OK:
        raise _lib.FgqaError(st, "fgqa_prefill_kernel_choice")
    return {_lib.FGQA_KERNEL_WHOLE: "whole", _lib.FGQA_KERNEL_SPLIT: "split", _lib.FGQA_KERNEL_WIDE: "wide",
            _lib.FGQA_KERNEL_TALL: "tall"}[c.value]


def prefill_kernel_name(q, k, v, causal=True, window_size=0, sink=None, kernel="auto") -> str:
    """The name of the kernel function ``flash_gqa_forward_bshd`` launches for
    these tensors on the current device (it tells apart the grid forms of one
    kernel shape, e.g. ``prefill_wide_kernel`` on unit pairs and
    ``prefill_wide_persistent_kernel``); launches and allocates nothing."""
    a = _prefill_query_args(q, k, v, causal, window_size, sink, kernel)
    name = ctypes.c_char_p()
    _lib.check(_lib.lib().fgqa_prefill_kernel_name(ctypes.byref(a), ctypes.byref(name)), "fgqa_prefill_kernel_name")
    return name.value.decode()


def launch_flash_gqa_forward_bf16_kernel(q, k, v, scale=None, out=None, lse=None, causal=True,
                                         block_kv_sub=32, num_warps=8, num_stages=3):
    """Mirror of the reference's Triton prefill launcher
    (src/python/Triton/flash_gqa_kernel.py:185-338): BHSD q [B,Hq,Sq,D] (or 3-D
    [Hq,Sq,D]), k/v [B,Hkv,Skv,D]; returns (out, lse [B,Hq,Sq]).

    ``block_kv_sub``, ``num_warps`` and ``num_stages`` are Triton tuning knobs
    and are accepted for signature compatibility only.  Unlike the reference,
    which writes a non-contiguous ``out``/``lse`` into a silent copy (:280-297),
    a provided buffer is always written in place or rejected with ValueError.
    """
    del block_kv_sub, num_warps, num_stages
    return _launch_bhsd_prefill("GQA", q, k, v, scale, out, lse, causal)


def launch_flash_mla_forward_bf16_kernel(q, k, v, scale=None, out=None, lse=None, causal=True,
                                         block_kv_sub=64, num_warps=8, num_stages=3):
    """Mirror of the reference's Triton MLA prefill launcher
    (src/python/Triton/flash_mla_kernel.py:315-508): BHSD q [B,Hq,Sq,Dqk] (or
    3-D [Hq,Sq,Dqk]), k [B,Hkv,Skv,Dqk], v [B,Hkv,Skv,Dv]; returns
    (out [B,Hq,Sq,Dv], lse [B,Hq,Sq]).  The default scale is 1/sqrt(Dqk).

    Same checks and ValueError messages as the reference (:356-436).  The
    kernels are built for (Dqk, Dv) = (192, 128), the reference's MLA shape,
    and (128, 128); other pairs raise ValueError.  ``block_kv_sub``,
    ``num_warps`` and ``num_stages`` are Triton tuning knobs, accepted for
    signature compatibility only.  A provided ``out``/``lse`` is written in
    place or rejected (the reference writes a non-contiguous one into a copy).
    """
    del block_kv_sub, num_warps, num_stages
    return _launch_bhsd_prefill("MLA", q, k, v, scale, out, lse, causal)


def _launch_bhsd_prefill(kind, q, k, v, scale, out, lse, causal):
    """Shared body of the GQA and MLA Triton-launcher mirrors (BHSD, 3-D or 4-D)."""
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        raise ValueError(f"Flash {kind} forward expects bf16 inputs")
    if q.dim() not in (3, 4):
        raise ValueError("Q must be 3D or 4D")
    if k.dim() != q.dim() or v.dim() != q.dim():
        raise ValueError("Q, K, and V must have matching ranks")
    _require_cuda(q, k, v)
    squeeze_output = q.dim() == 3
    qb = q.unsqueeze(0) if squeeze_output else q
    kb = k.unsqueeze(0) if squeeze_output else k
    vb = v.unsqueeze(0) if squeeze_output else v
    batch, q_heads, seqlen_q, head_dim_qk = qb.shape
    _, num_kv_heads, seqlen_kv, k_head_dim = kb.shape
    _, v_heads, v_seqlen, head_dim_v = vb.shape
    if seqlen_kv != v_seqlen:
        raise ValueError("K and V must share sequence length")
    if k_head_dim != head_dim_qk:
        raise ValueError("Q and K must share head_dim_qk")
    if v_heads != num_kv_heads:
        raise ValueError("K and V must share number of KV heads")
    if q_heads % num_kv_heads != 0:
        raise ValueError("Query heads must be divisible by KV heads")
    if kind == "GQA" and head_dim_v != head_dim_qk:
        raise ValueError("head_dim_v must equal head_dim_qk on this path")
    _check_head_dims(head_dim_qk, head_dim_v, padded_ok=True)
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim_qk)
    qb, kb, vb = _prep(qb), _prep(kb), _prep(vb)
    if out is None:
        out_b = torch.empty((batch, q_heads, seqlen_q, head_dim_v), device=qb.device, dtype=torch.bfloat16)
    else:
        if squeeze_output:
            if out.dim() != 3:
                raise ValueError("Output must be 3D when Q is 3D")
            out_b = out.unsqueeze(0)
        else:
            if out.dim() != 4:
                raise ValueError("Output must be 4D when Q is 4D")
            out_b = out
        if out_b.dtype != torch.bfloat16 or not _out_ready(out_b, head_dim_qk, head_dim_v):
            raise ValueError("Output must be bf16 with contiguous, 16-byte aligned rows")
    if out_b.shape != (batch, q_heads, seqlen_q, head_dim_v):
        raise ValueError("Output must have shape [batch, q_heads, seqlen_q, head_dim_v]")
    if lse is None:
        lse_b = torch.empty((batch, q_heads, seqlen_q), device=qb.device, dtype=torch.float32)
    else:
        if squeeze_output:
            if lse.dim() != 2:
                raise ValueError("LSE must be 2D when Q is 3D")
            lse_b = lse.unsqueeze(0)
        else:
            if lse.dim() != 3:
                raise ValueError("LSE must be 3D when Q is 4D")
            lse_b = lse
        if lse_b.shape != (batch, q_heads, seqlen_q) or lse_b.dtype != torch.float32 or not lse_b.is_contiguous():
            raise ValueError("LSE must be a contiguous fp32 [batch, q_heads, seqlen_q] tensor")
    _prefill(qb, kb, vb, out_b, lse_b, scale, causal, "bhsd")
    if squeeze_output:
        return out_b.squeeze(0), lse_b.squeeze(0)
    return out_b, lse_b




# --------------------------------------------------------------------------- backward
def _backward_args(q, k, v, o, lse, grad_o, dq, dk, dv, scale, causal, layout, workspace,
                   window_size=0, kv_head_split=0, dq_kernel="auto") -> _lib.BackwardArgs:
    """C ABI argument block; 4-D tensors in `layout` ('bshd' or 'bhsd')."""
    def sbh(t):
        if layout == "bshd":
            return [t.stride(0), t.stride(1), t.stride(2)]
        return [t.stride(0), t.stride(2), t.stride(1)]

    if layout == "bshd":
        B, Sq, Hq, D = q.shape
        _, Skv, Hkv, _ = k.shape
    else:
        B, Hq, Sq, D = q.shape
        _, Hkv, Skv, _ = k.shape
    a = _lib.BackwardArgs()
    a.q, a.k, a.v, a.o, a.lse, a.grad_o = (_ptr(x) for x in (q, k, v, o, lse, grad_o))
    a.grad_q, a.grad_k, a.grad_v = _ptr(dq), _ptr(dk), _ptr(dv)
    a.batch, a.seqlen_q, a.seqlen_kv = B, Sq, Skv
    a.num_q_heads, a.num_kv_heads, a.head_dim = Hq, Hkv, D
    a.causal = 1 if causal else 0
    a.scale = float(scale)
    a.window_size = int(window_size)
    a.head_dim_v = int(v.shape[-1])
    a.kv_head_split = int(kv_head_split)
    a.dq_kernel = _kernel_choice(dq_kernel)
    a.q_stride[:] = sbh(q)
    a.k_stride[:] = sbh(k)
    a.v_stride[:] = sbh(v)
    a.o_stride[:] = sbh(o)
    a.grad_o_stride[:] = sbh(grad_o)
    a.grad_q_stride[:] = sbh(dq)
    a.grad_k_stride[:] = sbh(dk)
    a.grad_v_stride[:] = sbh(dv)
    if workspace is not None:
        a.workspace = workspace.data_ptr()
        a.workspace_bytes = workspace.numel() * workspace.element_size()
    return a


def backward_workspace_bytes(batch, seqlen_q, seqlen_kv, num_q_heads, num_kv_heads, head_dim=128,
                             window_size=0, head_dim_v=0, kv_head_split=0) -> int:
    """Bytes of scratch ``flash_gqa_backward_bshd`` needs for a caller workspace
    (256-byte aligned; depends on the current device's CU count and on the
    window: a sliding-window backward needs at most the causal one's).
    head_dim 192 with head_dim_v 128: the MLA backward.  kv_head_split as in
    ``flash_gqa_backward_bshd``."""
    dv = int(head_dim_v) or head_dim
    a = _lib.BackwardArgs()
    a.batch, a.seqlen_q, a.seqlen_kv = batch, seqlen_q, seqlen_kv
    a.num_q_heads, a.num_kv_heads, a.head_dim = num_q_heads, num_kv_heads, head_dim
    a.head_dim_v = dv
    a.causal = 1
    a.window_size = int(window_size)
    a.kv_head_split = int(kv_head_split)
    a.scale = 1.0
    for name, d in (("q_stride", head_dim), ("grad_q_stride", head_dim), ("o_stride", dv), ("grad_o_stride", dv)):
        getattr(a, name)[:] = [seqlen_q * num_q_heads * d, num_q_heads * d, d]
    for name, d in (("k_stride", head_dim), ("grad_k_stride", head_dim), ("v_stride", dv), ("grad_v_stride", dv)):
        getattr(a, name)[:] = [seqlen_kv * num_kv_heads * d, num_kv_heads * d, d]
    n = ctypes.c_size_t(0)
    _lib.check(_lib.lib().fgqa_prefill_backward_workspace_bytes(ctypes.byref(a), ctypes.byref(n)),
               "fgqa_prefill_backward_workspace_bytes")
    return int(n.value)


def _grad_out(t, shape, ref, name, padded=False):
    """A gradient output: kernel-ready rows, or with padded head dims (whose
    gradients are copied out element by element) rows with a contiguous head dim."""
    if t is None:
        return torch.empty(shape, device=ref.device, dtype=torch.bfloat16)
    ready = _kernel_ready(t) or (padded and t.stride(-1) == 1)
    if tuple(t.shape) != tuple(shape) or t.dtype != torch.bfloat16 or not ready:
        raise ValueError(f"{name} must be a bf16 tensor of shape {list(shape)} with contiguous, aligned rows")
    return t


def _backward_bshd_prepare(q, k, v, o, lse, grad_o, scale, causal, grad_q, grad_k, grad_v, workspace,
                           window_size=0, kv_head_split=0, dq_kernel="auto"):
    for t in (q, k, v, o, grad_o):
        if t.dtype != torch.bfloat16:
            raise ValueError("Flash GQA backward expects bf16 inputs and grad_o")
    if lse.dtype != torch.float32:
        raise ValueError("Flash GQA backward expects lse to be float32")
    if any(t.dim() != 4 for t in (q, k, v, o, grad_o)):
        raise ValueError("expected 4-D BSHD tensors")
    _require_cuda(q, k, v, o, lse, grad_o)
    B, Sq, Hq, D = q.shape
    Dv = v.shape[3]
    if k.shape[:3] != v.shape[:3] or k.shape[0] != B or k.shape[3] != D:
        raise ValueError("K must be [B, Skv, Hkv, D] matching Q and V [B, Skv, Hkv, Dv]")
    if o.shape != (B, Sq, Hq, Dv) or grad_o.shape != o.shape:
        raise ValueError("O and grad_o must be [B, Sq, Hq, Dv] with V's head dim")
    _check_head_dims(D, Dv, window_size)
    if Hq % k.shape[2] != 0:
        raise ValueError("Query heads must be divisible by KV heads")
    if lse.shape != (B, Hq, Sq) or not lse.is_contiguous():
        raise ValueError("LSE must be a contiguous fp32 [batch, q_heads, seqlen_q] tensor")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    q, k, v, o, grad_o = (_prep(t) for t in (q, k, v, o, grad_o))
    padded = _padded_backward_head_dims(D, Dv)
    grad_q = _grad_out(grad_q, q.shape, q, "grad_q", padded)
    grad_k = _grad_out(grad_k, k.shape, q, "grad_k", padded)
    grad_v = _grad_out(grad_v, v.shape, q, "grad_v", padded)
    a = _backward_args(q, k, v, o, lse, grad_o, grad_q, grad_k, grad_v, scale, causal, "bshd", workspace,
                       window_size, kv_head_split, dq_kernel)
    return a, (grad_q, grad_k, grad_v), (q, k, v, o, lse, grad_o, grad_q, grad_k, grad_v, workspace)


def flash_gqa_backward_bshd(q, k, v, o, lse, grad_o, scale=None, causal=True,
                            grad_q=None, grad_k=None, grad_v=None, workspace=None, window_size=0,
                            kv_head_split=0, dq_kernel="auto"):
    """Prefill backward in BSHD: q/o/grad_o [B,Sq,Hq,D], k/v [B,Skv,Hkv,D], lse
    [B,Hq,Sq] from the forward -> (grad_q, grad_k, grad_v) bf16 in q/k/v's shapes.

    ``window_size`` > 0 (causal only) restricts row i to keys
    [i - window_size + 1, i], the sliding-window backward; pass the forward's
    LSE (with the sink term when the forward had one) and the gradients follow
    the sink-adjusted softmax.

    kv_head_split (0 = automatic, else a divisor of Hq / Hkv) and dq_kernel
    ('auto' / 'whole' / 'split') force the work split of the dK/dV and dQ passes."""
    a, grads, _keep = _backward_bshd_prepare(q, k, v, o, lse, grad_o, scale, causal,
                                             grad_q, grad_k, grad_v, workspace, window_size,
                                             kv_head_split, dq_kernel)
    _lib.check(_lib.lib().fgqa_prefill_backward_bf16(ctypes.byref(a), ctypes.c_void_p(_stream())),
               "fgqa_prefill_backward_bf16")
    return grads


def prepare_backward(q, k, v, o, lse, grad_o, scale=None, causal=True,
                     grad_q=None, grad_k=None, grad_v=None, workspace=None, window_size=0,
                     kv_head_split=0, dq_kernel="auto"):
    """``flash_gqa_backward_bshd`` validated once; returns a ``PreparedLaunch``
    whose ``out`` is the (grad_q, grad_k, grad_v) tuple."""
    a, grads, keep = _backward_bshd_prepare(q, k, v, o, lse, grad_o, scale, causal,
                                            grad_q, grad_k, grad_v, workspace, window_size,
                                            kv_head_split, dq_kernel)
    return PreparedLaunch(_lib.lib().fgqa_prefill_backward_bf16, a, keep, grads, "fgqa_prefill_backward_bf16")


def _launch_bhsd_backward(kind, q, k, v, o, lse, grad_o, scale, causal, window_size):
    """Shared body of the GQA, SWA and MLA backward mirrors: the reference's
    checks and messages (``kind`` is "GQA", "SWA" or "MLA"), then one C ABI call."""
    if (q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16
            or o.dtype != torch.bfloat16 or grad_o.dtype != torch.bfloat16):
        raise ValueError(f"Flash {kind} backward expects bf16 inputs and grad_o")
    if lse.dtype != torch.float32:
        raise ValueError(f"Flash {kind} backward expects lse to be float32")
    if q.dim() not in (3, 4):
        raise ValueError("Q must be 3D or 4D")
    if k.dim() != q.dim() or v.dim() != q.dim() or o.dim() != q.dim() or grad_o.dim() != q.dim():
        raise ValueError("Q, K, V, O, and grad_o must have matching ranks")
    squeeze_output = q.dim() == 3
    qb, kb, vb, ob, gb = (t.unsqueeze(0) if squeeze_output else t for t in (q, k, v, o, grad_o))
    batch, q_heads, seqlen_q, head_dim_qk = qb.shape
    _, num_kv_heads, seqlen_kv, k_head_dim = kb.shape
    _, v_heads, v_seqlen, head_dim_v = vb.shape
    _, o_heads, o_seqlen, o_head_dim = ob.shape
    _, grad_o_heads, grad_o_seqlen, grad_o_head_dim = gb.shape
    if seqlen_kv != v_seqlen:
        raise ValueError("K and V must share sequence length")
    if seqlen_q != o_seqlen or seqlen_q != grad_o_seqlen:
        raise ValueError("Q, O, and grad_o must share sequence length")
    if k_head_dim != head_dim_qk:
        raise ValueError("Q and K must share head_dim_qk")
    if o_head_dim != head_dim_v or grad_o_head_dim != head_dim_v:
        raise ValueError("O and grad_o must share head_dim_v with V")
    if v_heads != num_kv_heads:
        raise ValueError("K and V must share number of KV heads")
    if o_heads != q_heads or grad_o_heads != q_heads:
        raise ValueError("Q, O, and grad_o must share number of query heads")
    if q_heads % num_kv_heads != 0:
        raise ValueError("Query heads must be divisible by KV heads")
    if squeeze_output:
        if lse.dim() != 2:
            raise ValueError("LSE must be 2D when Q is 3D")
        lse_b = lse.unsqueeze(0)
    else:
        if lse.dim() != 3:
            raise ValueError("LSE must be 3D when Q is 4D")
        lse_b = lse
    if tuple(lse_b.shape) != (batch, q_heads, seqlen_q):
        raise ValueError("LSE must have shape [batch, q_heads, seqlen_q]")
    if kind == "SWA":
        if window_size is None:
            raise ValueError("window_size must be provided")
        if int(window_size) <= 0:
            raise ValueError("window_size must be positive")
    if any(t.shape[0] != batch for t in (kb, vb, ob, gb)):
        raise ValueError("Q, K, V, O, and grad_o must share batch dimension")
    if kind == "MLA":
        _check_head_dims(head_dim_qk, head_dim_v)
    elif head_dim_v != head_dim_qk:
        raise ValueError("head_dim_v must equal head_dim_qk on this path")
    _require_cuda(qb, kb, vb, ob, lse_b, gb)
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim_qk)
    qb, kb, vb, ob, gb = (_prep(t) for t in (qb, kb, vb, ob, gb))
    lse_b = lse_b.contiguous()
    dq = torch.empty((batch, q_heads, seqlen_q, head_dim_qk), device=qb.device, dtype=torch.bfloat16)
    dk = torch.empty((batch, num_kv_heads, seqlen_kv, head_dim_qk), device=qb.device, dtype=torch.bfloat16)
    dv = torch.empty((batch, num_kv_heads, seqlen_kv, head_dim_v), device=qb.device, dtype=torch.bfloat16)
    a = _backward_args(qb, kb, vb, ob, lse_b, gb, dq, dk, dv, scale, causal, "bhsd", None,
                       int(window_size or 0))
    _lib.check(_lib.lib().fgqa_prefill_backward_bf16(ctypes.byref(a), ctypes.c_void_p(_stream())),
               "fgqa_prefill_backward_bf16")
    if squeeze_output:
        return dq.squeeze(0), dk.squeeze(0), dv.squeeze(0)
    return dq, dk, dv


def launch_flash_gqa_backward_bf16_kernel(q, k, v, o, lse, grad_o, scale=None, causal=True,
                                          block_kv=64, num_warps=4, num_stages=3):
    """Mirror of the reference's Triton backward launcher
    (src/python/Triton/flash_gqa_backward_kernel.py:312-478): BHSD q/o/grad_o
    [B,Hq,Sq,D] (or 3-D [Hq,Sq,D]), k/v [B,Hkv,Skv,D], lse [B,Hq,Sq] (or
    [Hq,Sq]); returns bf16 (grad_q, grad_k, grad_v) shaped like q, k, v.

    Same checks and ValueError messages as the reference (:356-405).
    ``block_kv``, ``num_warps`` and ``num_stages`` are Triton tuning knobs,
    accepted for signature compatibility only.  Beyond the reference, inputs
    must share the batch dimension and head_dim_v must equal head_dim_qk (128).
    """
    del block_kv, num_warps, num_stages
    return _launch_bhsd_backward("GQA", q, k, v, o, lse, grad_o, scale, causal, 0)


def launch_flash_mla_backward_bf16_kernel(q, k, v, o, lse, grad_o, scale=None, causal=True,
                                          block_kv=64, num_warps=8, num_stages=3):
    """Mirror of the reference's Triton MLA backward launcher
    (src/python/Triton/flash_mla_backward_kernel.py:788-969): BHSD q
    [B,Hq,Sq,192], k [B,Hkv,Skv,192], v [B,Hkv,Skv,128], o/grad_o
    [B,Hq,Sq,128] (or 3-D), lse [B,Hq,Sq] from the MLA forward; returns bf16
    (grad_q, grad_k, grad_v) shaped like q, k, v.  The default scale is
    1/sqrt(head_dim_qk), as in the reference.

    Same checks and ValueError messages as the reference (:836-890).
    ``block_kv``, ``num_warps`` and ``num_stages`` are Triton tuning knobs,
    accepted for signature compatibility only.  Beyond the reference, inputs
    must share the batch dimension and (head_dim_qk, head_dim_v) must be
    (192, 128) or (128, 128).
    """
    del block_kv, num_warps, num_stages
    return _launch_bhsd_backward("MLA", q, k, v, o, lse, grad_o, scale, causal, 0)


def launch_flash_swa_backward_bf16_kernel(q, k, v, o, lse, grad_o, scale=None, window_size=None,
                                          block_kv=64, num_warps=8, num_stages=3):
    """Mirror of the reference's Triton SWA backward launcher
    (src/python/Triton/SWA/flash_swa_backward_kernel.py:323-489): gradients of
    causal sliding-window attention (row i sees keys [i - window_size + 1, i]).
    ``lse`` is the forward's, computed with the sink term; the sink has no
    value row, so the gradients are the windowed softmax's with that LSE.
    BHSD q/o/grad_o [B,Hq,Sq,D] (or 3-D), k/v [B,Hkv,Skv,D], lse [B,Hq,Sq];
    returns bf16 (grad_q, grad_k, grad_v) shaped like q, k, v.

    Same checks and ValueError messages as the reference (:370-420).
    ``block_kv``, ``num_warps`` and ``num_stages`` are Triton tuning knobs,
    accepted for signature compatibility only.  Beyond the reference,
    window_size must be positive, inputs must share the batch dimension and
    head_dim_v must equal head_dim_qk (128).
    """
    del block_kv, num_warps, num_stages
    return _launch_bhsd_backward("SWA", q, k, v, o, lse, grad_o, scale, True, window_size)


# --------------------------------------------------------------------------- sliding window + sink
def launch_flash_swa_forward_bf16_kernel(q, k, v, scale=None, out=None, lse=None, window_size=None,
                                         sink_value=None, block_kv_sub=16, num_warps=4, num_stages=3):
    """Mirror of the reference's Triton SWA launcher
    (src/python/Triton/SWA/flash_swa_kernel.py:188-370): causal sliding-window
    attention (row i sees keys [i - window_size + 1, i]) with a per-head sink
    in the softmax denominator; BHSD q [B,Hq,Sq,D] (or 3-D), k/v [B,Hkv,Skv,D];
    returns (out, lse [B,Hq,Sq]).

    Same checks and ValueError messages as the reference.  ``block_kv_sub``,
    ``num_warps`` and ``num_stages`` are Triton tuning knobs, accepted for
    signature compatibility only.  Beyond the reference, window_size must be
    positive (the reference masks every key for 0) and head_dim_v must equal
    head_dim_qk (128).
    """
    del block_kv_sub, num_warps, num_stages
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        raise ValueError("Flash SWA forward expects bf16 inputs")
    if q.dim() not in (3, 4):
        raise ValueError("Q must be 3D or 4D")
    if k.dim() != q.dim() or v.dim() != q.dim():
        raise ValueError("Q, K, and V must have matching ranks")
    squeeze_output = q.dim() == 3
    qb = q.unsqueeze(0) if squeeze_output else q
    kb = k.unsqueeze(0) if squeeze_output else k
    vb = v.unsqueeze(0) if squeeze_output else v
    batch, q_heads, seqlen_q, head_dim_qk = qb.shape
    _, num_kv_heads, seqlen_kv, k_head_dim = kb.shape
    _, v_heads, v_seqlen, head_dim_v = vb.shape
    if seqlen_kv != v_seqlen:
        raise ValueError("K and V must share sequence length")
    if k_head_dim != head_dim_qk:
        raise ValueError("Q and K must share head_dim_qk")
    if v_heads != num_kv_heads:
        raise ValueError("K and V must share number of KV heads")
    if q_heads % num_kv_heads != 0:
        raise ValueError("Query heads must be divisible by KV heads")
    if window_size is None:
        raise ValueError("window_size must be provided")
    if sink_value is None:
        raise ValueError("sink_value must be provided")
    if int(window_size) <= 0:
        raise ValueError("window_size must be positive")
    if head_dim_v != head_dim_qk:
        raise ValueError("head_dim_v must equal head_dim_qk on this path")
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim_qk)
    if out is None:
        out_b = torch.empty((batch, q_heads, seqlen_q, head_dim_v), device=qb.device, dtype=torch.bfloat16)
    else:
        if squeeze_output:
            if out.dim() != 3:
                raise ValueError("Output must be 3D when Q is 3D")
            out_b = out.unsqueeze(0)
        else:
            if out.dim() != 4:
                raise ValueError("Output must be 4D when Q is 4D")
            out_b = out
        if out_b.dtype != torch.bfloat16 or not _out_ready(out_b, head_dim_qk, head_dim_v):
            raise ValueError("Output must be bf16 with contiguous, 16-byte aligned rows")
    if out_b.shape != (batch, q_heads, seqlen_q, head_dim_v):
        raise ValueError("Output must have shape [batch, q_heads, seqlen_q, head_dim_v]")
    if lse is None:
        lse_b = torch.empty((batch, q_heads, seqlen_q), device=qb.device, dtype=torch.float32)
    else:
        if squeeze_output:
            if lse.dim() != 2:
                raise ValueError("LSE must be 2D when Q is 3D")
            lse_b = lse.unsqueeze(0)
        else:
            if lse.dim() != 3:
                raise ValueError("LSE must be 3D when Q is 4D")
            lse_b = lse
        if lse_b.dtype != torch.float32 or not lse_b.is_contiguous():
            raise ValueError("LSE must be a contiguous fp32 tensor")
    if lse_b.shape != (batch, q_heads, seqlen_q):
        raise ValueError("LSE must have shape [batch, q_heads, seqlen_q]")
    if not isinstance(sink_value, torch.Tensor):
        raise ValueError("sink_value must be a torch.Tensor")
    if sink_value.dim() != 1:
        raise ValueError("sink_value must be a 1D tensor with shape [q_heads]")
    if sink_value.numel() != q_heads:
        raise ValueError(f"sink_value must have {q_heads} elements")
    if sink_value.device != qb.device:
        raise ValueError("sink_value must be on the same device as Q")
    _require_cuda(qb, kb, vb)
    sink = sink_value.to(torch.float32).contiguous()
    qb, kb, vb = _prep(qb), _prep(kb), _prep(vb)
    _prefill(qb, kb, vb, out_b, lse_b, scale, True, "bhsd", int(window_size), sink)
    if squeeze_output:
        return out_b.squeeze(0), lse_b.squeeze(0)
    return out_b, lse_b


# --------------------------------------------------------------------------- sparse-index prefill
def _sparse_args(q, k, v, o, lse, idx, scale, causal, layout) -> _lib.SparsePrefillArgs:
    """C ABI argument block; q/k/v/o 4-D in `layout` ('bshd' or 'bhsd'), idx [B, Hkv, Sq, n]."""
    def sbh(t):
        if layout == "bshd":
            return [t.stride(0), t.stride(1), t.stride(2)]
        return [t.stride(0), t.stride(2), t.stride(1)]

    if layout == "bshd":
        B, Sq, Hq, D = q.shape
        _, Skv, Hkv, _ = k.shape
    else:
        B, Hq, Sq, D = q.shape
        _, Hkv, Skv, _ = k.shape
    a = _lib.SparsePrefillArgs()
    a.q, a.k, a.v, a.o, a.lse, a.kv_indices = (_ptr(x) for x in (q, k, v, o, lse, idx))
    a.batch, a.seqlen_q, a.seqlen_kv = B, Sq, Skv
    a.num_q_heads, a.num_kv_heads, a.head_dim = Hq, Hkv, D
    a.num_sparse_kv = idx.shape[3]
    a.causal = 1 if causal else 0
    a.scale = float(scale)
    a.q_stride[:] = sbh(q)
    a.k_stride[:] = sbh(k)
    a.v_stride[:] = sbh(v)
    a.o_stride[:] = sbh(o)
    a.idx_stride[:] = [idx.stride(0), idx.stride(1), idx.stride(2)]
    return a


def _check_indices(idx, B, Hkv, Sq):
    if not isinstance(idx, torch.Tensor) or idx.dtype != torch.int32:
        raise ValueError("kv_indices must be an int32 tensor")
    if idx.dim() != 4 or idx.shape[:3] != (B, Hkv, Sq) or idx.shape[3] < 1:
        raise ValueError("kv_indices must be [batch, num_kv_heads, seqlen_q, num_sparse_kv]")
    if idx.stride(3) != 1:
        idx = idx.contiguous()
    return idx


def _sparse_bshd_prepare(q, k, v, kv_indices, scale, out, lse, causal):
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        raise ValueError("Flash SGQA forward expects bf16 inputs")
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("expected 4-D BSHD tensors")
    _require_cuda(q, k, v, kv_indices)
    B, Sq, Hq, D = q.shape
    if k.shape != v.shape or k.shape[0] != B or k.shape[3] != D:
        raise ValueError("K and V must be [B, Skv, Hkv, D] matching Q")
    if Hq % k.shape[2] != 0:
        raise ValueError("Query heads must be divisible by KV heads")
    if D != 128:
        raise ValueError("head_dim must be 128 on this path")
    idx = _check_indices(kv_indices, B, k.shape[2], Sq)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    q, k, v = _prep(q), _prep(k), _prep(v)
    if out is None:
        out = torch.empty((B, Sq, Hq, D), device=q.device, dtype=torch.bfloat16)
    elif out.shape != (B, Sq, Hq, D) or out.dtype != torch.bfloat16 or not _kernel_ready(out):
        raise ValueError("Output must be a bf16 [batch, seqlen_q, q_heads, head_dim] tensor with contiguous rows")
    if lse is None:
        lse = torch.empty((B, Hq, Sq), device=q.device, dtype=torch.float32)
    elif lse.shape != (B, Hq, Sq) or lse.dtype != torch.float32 or not lse.is_contiguous():
        raise ValueError("LSE must be a contiguous fp32 [batch, q_heads, seqlen_q] tensor")
    a = _sparse_args(q, k, v, out, lse, idx, scale, causal, "bshd")
    return a, out, lse, (q, k, v, out, lse, idx)


def flash_sgqa_forward_bshd(q, k, v, kv_indices, scale=None, out=None, lse=None, causal=True):
    """Sparse-index prefill in BSHD: q [B,Sq,Hq,D], k/v [B,Skv,Hkv,D], kv_indices
    int32 [B,Hkv,Sq,n] (key lists shared by a KV head's query heads; entries
    < 0, >= Skv or, if causal, > the row are skipped) -> (out [B,Sq,Hq,D], lse [B,Hq,Sq])."""
    a, out, lse, _keep = _sparse_bshd_prepare(q, k, v, kv_indices, scale, out, lse, causal)
    _lib.check(_lib.lib().fgqa_sparse_prefill_bf16(ctypes.byref(a), ctypes.c_void_p(_stream())),
               "fgqa_sparse_prefill_bf16")
    return out, lse


def prepare_sparse_prefill(q, k, v, kv_indices, scale=None, out=None, lse=None, causal=True):
    """``flash_sgqa_forward_bshd`` validated once; returns a ``PreparedLaunch``
    (the LSE tensor is ``.lse``)."""
    a, out, lse, keep = _sparse_bshd_prepare(q, k, v, kv_indices, scale, out, lse, causal)
    pl = PreparedLaunch(_lib.lib().fgqa_sparse_prefill_bf16, a, keep, out, "fgqa_sparse_prefill_bf16")
    pl.lse = lse
    return pl


def launch_flash_sgqa_forward_bf16_kernel(q, k, v, sparse_kv_indices, num_sparse_kv, scale=None, out=None,
                                          lse=None, causal=True, block_sparse_sub=None, num_warps=None,
                                          num_stages=None):
    """Mirror of the reference's Triton sparse-GQA launcher
    (src/python/Triton/SparseGQA/flash_sgqa_kernel.py:202-396): BHSD q [B,Hq,Sq,D] (or
    3-D [Hq,Sq,D]), k/v [B,Hkv,Skv,D], sparse_kv_indices int32
    [B,Hkv,Sq,num_sparse_kv]; returns (out, lse [B,Hq,Sq]).

    Same checks and ValueError messages as the reference (:247-361), including
    its rule that a provided out/lse must be contiguous.  ``block_sparse_sub``,
    ``num_warps`` and ``num_stages`` are validated as the reference does and
    otherwise unused (Triton tuning knobs).  Beyond the reference, head_dim and
    head_dim_v must be 128.
    """
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        raise ValueError("Flash SGQA forward expects bf16 inputs")
    if sparse_kv_indices.dtype != torch.int32:
        raise ValueError("sparse_kv_indices must be int32")
    if sparse_kv_indices.dim() != 4:
        raise ValueError("sparse_kv_indices must be 4D [batch, num_kv_heads, seqlen_q, num_sparse_kv]")
    if not isinstance(num_sparse_kv, int):
        raise ValueError("num_sparse_kv must be an int")
    if num_sparse_kv < 1:
        raise ValueError("num_sparse_kv must be >= 1")
    if block_sparse_sub is not None and (not isinstance(block_sparse_sub, int) or block_sparse_sub < 1):
        raise ValueError("block_sparse_sub must be None or an int >= 1")
    if num_warps is not None and (not isinstance(num_warps, int) or num_warps < 1):
        raise ValueError("num_warps must be None or an int >= 1")
    if num_stages is not None and (not isinstance(num_stages, int) or num_stages < 1):
        raise ValueError("num_stages must be None or an int >= 1")
    if q.dim() not in (3, 4):
        raise ValueError("Q must be 3D or 4D")
    if k.dim() != q.dim() or v.dim() != q.dim():
        raise ValueError("Q, K, and V must have matching ranks")
    _require_cuda(q, k, v, sparse_kv_indices)
    squeeze_output = q.dim() == 3
    qb = q.unsqueeze(0) if squeeze_output else q
    kb = k.unsqueeze(0) if squeeze_output else k
    vb = v.unsqueeze(0) if squeeze_output else v
    batch, q_heads, seqlen_q, head_dim_qk = qb.shape
    _, num_kv_heads, seqlen_kv, k_head_dim = kb.shape
    _, v_heads, v_seqlen, head_dim_v = vb.shape
    if seqlen_kv != v_seqlen:
        raise ValueError("K and V must share sequence length")
    if k_head_dim != head_dim_qk:
        raise ValueError("Q and K must share head_dim_qk")
    if v_heads != num_kv_heads:
        raise ValueError("K and V must share number of KV heads")
    if q_heads % num_kv_heads != 0:
        raise ValueError("Query heads must be divisible by KV heads")
    if sparse_kv_indices.shape != (batch, num_kv_heads, seqlen_q, num_sparse_kv):
        raise ValueError("sparse_kv_indices must have shape "
                         f"[batch, num_kv_heads, seqlen_q, {num_sparse_kv}]")
    if head_dim_qk != 128 or head_dim_v != 128:
        raise ValueError("head_dim_qk and head_dim_v must be 128 on this path")
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim_qk)
    if out is None:
        out_b = torch.empty((batch, q_heads, seqlen_q, head_dim_v), device=qb.device, dtype=torch.bfloat16)
    else:
        if squeeze_output:
            if out.dim() != 3:
                raise ValueError("Output must be 3D when Q is 3D")
            if not out.is_contiguous():
                raise ValueError("Output must be contiguous when provided")
            out_b = out.unsqueeze(0)
        else:
            if out.dim() != 4:
                raise ValueError("Output must be 4D when Q is 4D")
            if not out.is_contiguous():
                raise ValueError("Output must be contiguous when provided")
            out_b = out
        if out_b.dtype != torch.bfloat16:
            raise ValueError("Output must be bf16")
    if out_b.shape != (batch, q_heads, seqlen_q, head_dim_v):
        raise ValueError("Output must have shape [batch, q_heads, seqlen_q, head_dim_v]")
    if lse is None:
        lse_b = torch.empty((batch, q_heads, seqlen_q), device=qb.device, dtype=torch.float32)
    else:
        if squeeze_output:
            if lse.dim() != 2:
                raise ValueError("LSE must be 2D when Q is 3D")
            if not lse.is_contiguous():
                raise ValueError("LSE must be contiguous when provided")
            lse_b = lse.unsqueeze(0)
        else:
            if lse.dim() != 3:
                raise ValueError("LSE must be 3D when Q is 4D")
            if not lse.is_contiguous():
                raise ValueError("LSE must be contiguous when provided")
            lse_b = lse
        if lse_b.dtype != torch.float32:
            raise ValueError("LSE must be fp32")
    if lse_b.shape != (batch, q_heads, seqlen_q):
        raise ValueError("LSE must have shape [batch, q_heads, seqlen_q]")
    if seqlen_q > 0:
        qb, kb, vb = _prep(qb), _prep(kb), _prep(vb)
        idx = sparse_kv_indices if sparse_kv_indices.stride(3) == 1 else sparse_kv_indices.contiguous()
        a = _sparse_args(qb, kb, vb, out_b, lse_b, idx, scale, causal, "bhsd")
        _lib.check(_lib.lib().fgqa_sparse_prefill_bf16(ctypes.byref(a), ctypes.c_void_p(_stream())),
                   "fgqa_sparse_prefill_bf16")
    if squeeze_output:
        return out_b.squeeze(0), lse_b.squeeze(0)
    return out_b, lse_b
