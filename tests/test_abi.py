"""CPU tests of the drop-in boundary: libfgqa.so loads, exports every entry
point the headers declare, and rejects bad arguments before touching a GPU."""
import ctypes
import os
import re
import subprocess

import pytest

import cuda_llm_ops_amd as fg
from cuda_llm_ops_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _exported():
    out = subprocess.run(["nm", "-D", "--defined-only", "-C", _lib.LIB_PATH], check=True,
                         capture_output=True, text=True).stdout
    return out


def test_c_abi_symbols_exported():
    hdr = open(os.path.join(ROOT, "include", "fgqa.h")).read()
    names = set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(fgqa_\w+)\s*\(", hdr, flags=re.M))
    assert names == {"fgqa_decode_workspace_bytes", "fgqa_decode_bf16", "fgqa_decode_bf16_noalloc", "fgqa_prefill_bf16",
                     "fgqa_prefill_kernel_choice", "fgqa_prefill_kernel_name", "fgqa_prefill_workspace_bytes",
                     "fgqa_prefill_backward_workspace_bytes", "fgqa_prefill_backward_bf16",
                     "fgqa_decode_paged_workspace_bytes", "fgqa_decode_paged", "fgqa_sparse_prefill_bf16",
                     "fgqa_status_string", "fgqa_version", "fgqa_clock_sample"}
    L = _lib.lib()
    syms = _exported()
    for n in names:
        assert hasattr(L, n), n
        assert re.search(rf"\bT {n}$", syms, flags=re.M), f"{n} not exported with C linkage"


def test_cplusplus_entry_points_exported():
    syms = _exported()
    decls = []
    for sub in ("FlashGQA/decode_flash_gqa_kernel.h", "FlashGQA/flash_gqa_forward_kernel.h",
                "FlashGQA/flash_gqa_backward_kernel.h"):
        hdr = open(os.path.join(ROOT, "include", "cplusplus", sub)).read()
        decls += re.findall(r"^(?:void|int)\s+(\w+)\(", hdr, flags=re.M)
    assert set(decls) == {"LaunchFlashGqaBf16Kernel", "LaunchFlashGqaBf16KernelVarlen", "FlashGqaGetLastStatus",
                          "LaunchFlashGqaBf16KernelPaged",
                          "LaunchFlashGqaForwardBf16Kernel", "LaunchFlashGqaForwardBf16KernelStrided",
                          "LaunchFlashGqaBackwardBf16Kernel", "LaunchFlashSwaForwardBf16Kernel",
                          "LaunchFlashSwaBackwardBf16Kernel", "LaunchFlashMlaBackwardBf16Kernel",
                          "LaunchFlashMlaForwardBf16Kernel", "LaunchFlashSgqaForwardBf16Kernel"}
    for d in decls:
        assert re.search(rf"\bT {d}\(", syms), d
    # the drop-in keeps the reference's exact parameter list
    # (decode_flash_gqa_kernel.cuh:28-38: 3 const bf16*, float, bf16*, float*, 5 ints)
    assert "LaunchFlashGqaBf16Kernel(bf16_t const*, bf16_t const*, bf16_t const*, float, bf16_t*, float*, " \
           "int, int, int, int, int)" in syms


def test_status_strings_and_version():
    assert fg.status_string(0) == "ok"
    for code in (-1, -2, -3, -4):
        assert fg.status_string(code) not in ("ok", "unknown status")
    assert fg.status_string(12345) == "unknown status"
    assert _lib.lib().fgqa_version() >= 100


def _decode_args(**kw):
    a = _lib.DecodeArgs()
    B, S, Hq, Hkv, D = kw.get("B", 2), kw.get("S", 512), kw.get("Hq", 16), kw.get("Hkv", 2), kw.get("D", 128)
    a.batch, a.max_seqlen, a.num_q_heads, a.num_kv_heads, a.head_dim = B, S, Hq, Hkv, D
    a.scale = kw.get("scale", D ** -0.5)
    a.q_stride[:] = [Hq * D, D]
    a.o_stride[:] = [Hq * D, D]
    a.k_stride[:] = [S * Hkv * D, Hkv * D, D]
    a.v_stride[:] = [S * Hkv * D, Hkv * D, D]
    a.split_tokens = kw.get("split_tokens", 256)
    for name in ("q", "k", "v", "o"):
        setattr(a, name, kw.get(name, 4096))  # fake, aligned, never dereferenced on the host
    return a


def _ws(a):
    n = ctypes.c_size_t(0)
    st = _lib.lib().fgqa_decode_workspace_bytes(ctypes.byref(a), ctypes.byref(n))
    return st, n.value


def test_decode_workspace_formula():
    # B*Hq*nsplit partials of 128 fp32 O and of (max, sum), each array rounded to 256 bytes
    for S, split in ((512, 256), (4096, 1024), (1000, 128), (100, 128)):
        st, n = _ws(_decode_args(S=S, split_tokens=split))
        nsplit = -(-S // split)
        slots = 2 * 16 * nsplit
        expect = 0 if nsplit == 1 else -(-slots * 512 // 256) * 256 + -(-slots * 8 // 256) * 256
        assert st == 0 and n == expect, (S, split, n, expect)
    # ragged batches (seqlens given) add the work list: 1 + B*nsplit int32
    for S, split in ((2048, 256), (4096, 1024), (1000, 128)):
        a = _decode_args(S=S, split_tokens=split)
        a.seqlens = 64
        st, n = _ws(a)
        nsplit = -(-S // split)
        slots = 2 * 16 * nsplit
        expect = -(-slots * 512 // 256) * 256 + -(-slots * 8 // 256) * 256 + (1 + 2 * nsplit) * 4
        assert st == 0 and n == expect, (S, split, n, expect)
    # split_tokens rounds up to the 128-token step of a workgroup
    assert _ws(_decode_args(S=4096, split_tokens=1000)) == _ws(_decode_args(S=4096, split_tokens=1024))


@pytest.mark.parametrize("kw,code", [
    (dict(Hq=15), _lib.FGQA_ERR_INVALID_ARGUMENT),      # Hq % Hkv != 0
    (dict(B=-1), _lib.FGQA_ERR_INVALID_ARGUMENT),
    (dict(S=-5), _lib.FGQA_ERR_INVALID_ARGUMENT),
    (dict(scale=float("nan")), _lib.FGQA_ERR_INVALID_ARGUMENT),
    (dict(split_tokens=-1), _lib.FGQA_ERR_INVALID_ARGUMENT),
    (dict(D=64), _lib.FGQA_ERR_UNSUPPORTED),
    (dict(Hq=64, Hkv=2), _lib.FGQA_ERR_UNSUPPORTED),     # group of 32 heads
])
def test_decode_rejects_before_launch(kw, code):
    a = _decode_args(**kw)
    assert _ws(a)[0] == code
    assert _lib.lib().fgqa_decode_bf16(ctypes.byref(a), None) == code


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="fake device pointers: run only where no GPU could launch")
def test_noalloc_decode_refuses_oversize_plan_before_launch():
    """fgqa_decode_bf16_noalloc with a ragged B=1024, Hq=64, 32 K-token plan
    (256 MiB of partials, past the 32 MiB built-in scratch): FGQA_ERR_WORKSPACE
    from the host planner, before any HIP call.  A caller workspace is refused
    outright.  (The GPU suite repeats the refusal over real tensors.)"""
    L = _lib.lib()
    a = _decode_args(B=1024, S=32768, Hq=64, Hkv=8, split_tokens=0)
    a.seqlens = 4096
    st, need = _ws(a)
    assert st == 0 and need > 32 << 20
    assert L.fgqa_decode_bf16_noalloc(ctypes.byref(a), None) == _lib.FGQA_ERR_WORKSPACE
    b = _decode_args()
    b.workspace, b.workspace_bytes = 4096, 1 << 20
    assert L.fgqa_decode_bf16_noalloc(ctypes.byref(b), None) == _lib.FGQA_ERR_INVALID_ARGUMENT


def test_extreme_sizes_are_refused_before_launch():
    """Sizes the kernels' integer widths cannot hold come back as
    FGQA_ERR_UNSUPPORTED from every entry, with no device call."""
    L = _lib.lib()
    a = _decode_args(S=(1 << 30) + 1)
    a.k_stride[1] = a.v_stride[1] = 0
    assert _ws(a)[0] == _lib.FGQA_ERR_UNSUPPORTED
    assert L.fgqa_decode_bf16(ctypes.byref(a), None) == _lib.FGQA_ERR_UNSUPPORTED
    a = _decode_args(B=3)
    a.k_stride[0] = (1 << 62)   # batch 2's rows at 2^63 elements
    assert L.fgqa_decode_bf16(ctypes.byref(a), None) == _lib.FGQA_ERR_UNSUPPORTED
    p = _prefill_args()
    p.batch, p.seqlen_q, p.seqlen_kv = 2**31 - 1, 32, 32
    assert L.fgqa_prefill_bf16(ctypes.byref(p), None) == _lib.FGQA_ERR_UNSUPPORTED


def test_decode_rejects_pointers_and_alignment():
    L = _lib.lib()
    a = _decode_args(q=None)
    assert L.fgqa_decode_bf16(ctypes.byref(a), None) == _lib.FGQA_ERR_INVALID_ARGUMENT
    a = _decode_args(k=4096 + 2)
    assert L.fgqa_decode_bf16(ctypes.byref(a), None) == _lib.FGQA_ERR_UNSUPPORTED
    a = _decode_args()
    a.k_stride[1] = 2 * 128 + 4
    assert L.fgqa_decode_bf16(ctypes.byref(a), None) == _lib.FGQA_ERR_UNSUPPORTED
    # an explicit workspace that is too small
    a = _decode_args(split_tokens=128)
    a.workspace, a.workspace_bytes = 4096, 16
    assert L.fgqa_decode_bf16(ctypes.byref(a), None) == _lib.FGQA_ERR_WORKSPACE
    assert L.fgqa_decode_bf16(None, None) == _lib.FGQA_ERR_INVALID_ARGUMENT
    assert L.fgqa_decode_workspace_bytes(None, None) == _lib.FGQA_ERR_INVALID_ARGUMENT
    # batch == 0 is a valid no-op that launches nothing
    assert L.fgqa_decode_bf16(ctypes.byref(_decode_args(B=0, q=None)), None) == 0


def _prefill_args(**kw):
    a = _lib.PrefillArgs()
    B, Sq, Skv, Hq, Hkv, D = (kw.get(n, d) for n, d in
                              (("B", 1), ("Sq", 256), ("Skv", 256), ("Hq", 16), ("Hkv", 1), ("D", 128)))
    a.batch, a.seqlen_q, a.seqlen_kv, a.num_q_heads, a.num_kv_heads, a.head_dim = B, Sq, Skv, Hq, Hkv, D
    a.causal = 1
    a.scale = kw.get("scale", D ** -0.5)
    a.q_stride[:] = [Sq * Hq * D, Hq * D, D]
    a.o_stride[:] = kw.get("ostride", [Sq * Hq * D, Hq * D, D])
    a.k_stride[:] = [Skv * Hkv * D, Hkv * D, D]
    a.v_stride[:] = [Skv * Hkv * D, Hkv * D, D]
    for name in ("q", "k", "v", "o"):
        setattr(a, name, kw.get(name, 4096))
    a.window_size = kw.get("window", 0)
    a.sink = kw.get("sink", None)
    a.causal = kw.get("causal", 1)
    a.head_dim_v = kw.get("Dv", 0)
    a.kernel = kw.get("kernel", 0)
    return a


@pytest.mark.parametrize("kw,code", [
    (dict(Hq=15, Hkv=2), _lib.FGQA_ERR_INVALID_ARGUMENT),
    (dict(Sq=-1), _lib.FGQA_ERR_INVALID_ARGUMENT),
    (dict(scale=float("inf")), _lib.FGQA_ERR_INVALID_ARGUMENT),
    (dict(kernel=5), _lib.FGQA_ERR_INVALID_ARGUMENT),
    (dict(kernel=-1), _lib.FGQA_ERR_INVALID_ARGUMENT),
    (dict(kernel=_lib.FGQA_KERNEL_TALL, window=64), _lib.FGQA_ERR_UNSUPPORTED),    # tall: no window / sink
    (dict(kernel=_lib.FGQA_KERNEL_TALL, sink=4096), _lib.FGQA_ERR_UNSUPPORTED),
    (dict(kernel=_lib.FGQA_KERNEL_TALL, D=192, Dv=128), _lib.FGQA_ERR_UNSUPPORTED),   # tall: head dim 128
    (dict(kernel=_lib.FGQA_KERNEL_TALL, D=200), _lib.FGQA_ERR_UNSUPPORTED),           # (padded to 256)
    (dict(kernel=_lib.FGQA_KERNEL_SPLIT, D=256, Dv=128), _lib.FGQA_ERR_UNSUPPORTED),  # 256: whole-range only
    (dict(kernel=_lib.FGQA_KERNEL_WIDE, D=160, Dv=96), _lib.FGQA_ERR_UNSUPPORTED),
    (dict(kernel=_lib.FGQA_KERNEL_SPLIT, window=64), _lib.FGQA_ERR_UNSUPPORTED),   # no split SWA kernel
    (dict(kernel=_lib.FGQA_KERNEL_SPLIT, sink=4096), _lib.FGQA_ERR_UNSUPPORTED),
    (dict(ostride=[256 * 16 * 128, 16 * 128 + 4, 128]), _lib.FGQA_ERR_UNSUPPORTED),  # O rows: 16-byte stores
    (dict(D=257), _lib.FGQA_ERR_UNSUPPORTED),             # head dims above 256 are not built
    (dict(D=512), _lib.FGQA_ERR_UNSUPPORTED),
    (dict(v=None), _lib.FGQA_ERR_INVALID_ARGUMENT),
    (dict(o=4096 + 8), _lib.FGQA_ERR_UNSUPPORTED),
    (dict(window=-1), _lib.FGQA_ERR_INVALID_ARGUMENT),
    (dict(window=64, causal=0), _lib.FGQA_ERR_INVALID_ARGUMENT),   # a window is causal
    (dict(Dv=-1), _lib.FGQA_ERR_INVALID_ARGUMENT),
    (dict(D=192, window=64), _lib.FGQA_ERR_UNSUPPORTED),  # (192, 192) runs the 192 kernels: no window
    (dict(D=192, Dv=64, sink=4096), _lib.FGQA_ERR_UNSUPPORTED),
    (dict(D=128, Dv=300), _lib.FGQA_ERR_UNSUPPORTED),
    (dict(D=192, Dv=128, window=64), _lib.FGQA_ERR_UNSUPPORTED),   # MLA has no window form
    (dict(D=192, Dv=128, sink=4096), _lib.FGQA_ERR_UNSUPPORTED),
])
def test_prefill_rejects_before_launch(kw, code):
    assert _lib.lib().fgqa_prefill_bf16(ctypes.byref(_prefill_args(**kw)), None) == code
    if code != _lib.FGQA_OK:   # the kernel-choice query validates the same way
        c = ctypes.c_int32(-7)
        assert _lib.lib().fgqa_prefill_kernel_choice(ctypes.byref(_prefill_args(**kw)), ctypes.byref(c)) == code
        assert c.value == -7


def test_ctypes_structs_match_the_header(tmp_path):
    """Every ctypes mirror in _lib has the C struct's size and field offsets
    (a small C program compiled against include/fgqa.h prints them)."""
    mirrors = {"fgqa_decode_args": _lib.DecodeArgs, "fgqa_decode_paged_args": _lib.PagedDecodeArgs,
               "fgqa_prefill_args": _lib.PrefillArgs, "fgqa_prefill_backward_args": _lib.BackwardArgs,
               "fgqa_sparse_prefill_args": _lib.SparsePrefillArgs}
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "fgqa.h"', "int main(void) {"]
    for cname, py in mirrors.items():
        lines.append(f'    printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in py._fields_:
            lines.append(f'    printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines += ["    return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    got = {tuple(ln.split()[:2]): int(ln.split()[2]) for ln in out if ln.strip()}
    for cname, py in mirrors.items():
        assert got[(cname, "size")] == ctypes.sizeof(py), cname
        for fname, _ in py._fields_:
            assert got[(cname, fname)] == getattr(py, fname).offset, f"{cname}.{fname}"


def _sparse_args(**kw):
    a = _lib.SparsePrefillArgs()
    B, Sq, Skv, Hq, Hkv, D, n = (kw.get(nm, d) for nm, d in (("B", 1), ("Sq", 256), ("Skv", 256), ("Hq", 16),
                                                               ("Hkv", 1), ("D", 128), ("n", 64)))
    a.batch, a.seqlen_q, a.seqlen_kv, a.num_q_heads, a.num_kv_heads, a.head_dim = B, Sq, Skv, Hq, Hkv, D
    a.num_sparse_kv = n
    a.causal = 1
    a.scale = kw.get("scale", D ** -0.5)
    a.q_stride[:] = [Sq * Hq * D, Hq * D, D]
    a.o_stride[:] = kw.get("ostride", [Sq * Hq * D, Hq * D, D])
    a.k_stride[:] = [Skv * Hkv * D, Hkv * D, D]
    a.v_stride[:] = [Skv * Hkv * D, Hkv * D, D]
    a.idx_stride[:] = [Hkv * Sq * n, Sq * n, n]
    for name in ("q", "k", "v", "o", "kv_indices"):
        setattr(a, name, kw.get(name, 4096))
    return a


@pytest.mark.parametrize("kw,code", [
    (dict(Hq=15, Hkv=2), _lib.FGQA_ERR_INVALID_ARGUMENT),
    (dict(n=0), _lib.FGQA_ERR_INVALID_ARGUMENT),
    (dict(Skv=-1), _lib.FGQA_ERR_INVALID_ARGUMENT),
    (dict(scale=float("nan")), _lib.FGQA_ERR_INVALID_ARGUMENT),
    (dict(D=64), _lib.FGQA_ERR_UNSUPPORTED),
    (dict(kv_indices=None), _lib.FGQA_ERR_INVALID_ARGUMENT),
    (dict(kv_indices=4098), _lib.FGQA_ERR_UNSUPPORTED),   # int32 entries need 4-byte alignment
    (dict(q=4096 + 8), _lib.FGQA_ERR_UNSUPPORTED),
    (dict(ostride=[256 * 16 * 128, 16 * 128 + 4, 128]), _lib.FGQA_ERR_UNSUPPORTED),   # strides: multiples of 8
])
def test_sparse_prefill_rejects_before_launch(kw, code):
    assert _lib.lib().fgqa_sparse_prefill_bf16(ctypes.byref(_sparse_args(**kw)), None) == code


def test_sparse_prefill_empty_is_noop():
    L = _lib.lib()
    assert L.fgqa_sparse_prefill_bf16(ctypes.byref(_sparse_args(Sq=0, q=None)), None) == 0
    assert L.fgqa_sparse_prefill_bf16(ctypes.byref(_sparse_args(B=0, kv_indices=None)), None) == 0


def test_sparse_mirror_validation_without_gpu():
    """The mirror raises the reference's ValueErrors
    (SparseGQA/flash_sgqa_kernel.py:247-266) before touching a GPU."""
    import torch
    bf = torch.bfloat16
    q = torch.zeros(1, 4, 8, 128, dtype=bf)
    k = torch.zeros(1, 1, 8, 128, dtype=bf)
    idx = torch.zeros(1, 1, 8, 4, dtype=torch.int32)
    f = fg.launch_flash_sgqa_forward_bf16_kernel
    with pytest.raises(ValueError, match="Flash SGQA forward expects bf16 inputs"):
        f(q.half(), k, k, idx, 4)
    with pytest.raises(ValueError, match="sparse_kv_indices must be int32"):
        f(q, k, k, idx.long(), 4)
    with pytest.raises(ValueError, match="sparse_kv_indices must be 4D"):
        f(q, k, k, idx[0], 4)
    with pytest.raises(ValueError, match="num_sparse_kv must be an int"):
        f(q, k, k, idx, 4.0)
    with pytest.raises(ValueError, match="num_sparse_kv must be >= 1"):
        f(q, k, k, idx, 0)
    with pytest.raises(ValueError, match="block_sparse_sub must be None or an int >= 1"):
        f(q, k, k, idx, 4, block_sparse_sub=0)
    with pytest.raises(ValueError, match="num_warps must be None"):
        f(q, k, k, idx, 4, num_warps="8")
    with pytest.raises(ValueError, match="num_stages must be None"):
        f(q, k, k, idx, 4, num_stages=-1)
    with pytest.raises(ValueError, match="Q must be 3D or 4D"):
        f(q[0, 0], k[0, 0], k[0, 0], idx, 4)
    with pytest.raises(ValueError, match="matching ranks"):
        f(q, k[0], k, idx, 4)
    with pytest.raises(ValueError, match="GPU"):
        f(q, k, k, idx, 4)


def test_prefill_empty_is_noop():
    L = _lib.lib()
    assert L.fgqa_prefill_bf16(ctypes.byref(_prefill_args(Sq=0, q=None)), None) == 0
    assert L.fgqa_prefill_bf16(ctypes.byref(_prefill_args(B=0, q=None)), None) == 0


def test_python_mirror_validation_without_gpu():
    import torch
    q = torch.zeros(2, 16, 1, 128, dtype=torch.float16)
    k = torch.zeros(2, 2, 64, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="bf16"):
        fg.launch_decode_flash_gqa_bf16_kernel(q, k, k)
    with pytest.raises(ValueError, match="bf16"):
        fg.launch_flash_gqa_forward_bf16_kernel(q, k, k)
    qb = torch.zeros(2, 16, 1, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="ranks"):
        fg.launch_flash_gqa_forward_bf16_kernel(qb, k[0], k[0])
    with pytest.raises(ValueError, match="contiguous"):
        fg.launch_decode_flash_gqa_bf16_kernel(qb, k.transpose(2, 3), k)
    with pytest.raises(ValueError, match="divisible"):
        fg.launch_decode_flash_gqa_bf16_kernel(torch.zeros(2, 15, 1, 128, dtype=torch.bfloat16), k, k)
    with pytest.raises(ValueError, match="GPU"):
        fg.launch_flash_gqa_forward_bf16_kernel(qb, k, k)
    # the MLA mirror (flash_mla_kernel.py:356-361) and the BSHD head-dim check
    q192 = torch.zeros(2, 16, 64, 192, dtype=torch.bfloat16)
    k192 = torch.zeros(2, 2, 64, 192, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="Flash MLA forward expects bf16 inputs"):
        fg.launch_flash_mla_forward_bf16_kernel(q192.half(), k192, k)
    with pytest.raises(ValueError, match="Q must be 3D or 4D"):
        fg.launch_flash_mla_forward_bf16_kernel(q192[0, 0], k192[0, 0], k[0, 0])
    with pytest.raises(ValueError, match="ranks"):
        fg.launch_flash_mla_forward_bf16_kernel(q192, k192[0], k)
    with pytest.raises(ValueError, match="GPU"):
        fg.launch_flash_mla_forward_bf16_kernel(q192, k192, k)
    assert (192, 128) in fg.PREFILL_HEAD_DIMS and (128, 128) in fg.PREFILL_HEAD_DIMS


def _backward_args(**kw):
    a = _lib.BackwardArgs()
    B, Sq, Skv, Hq, Hkv, D = (kw.get(n, d) for n, d in
                              (("B", 1), ("Sq", 256), ("Skv", 256), ("Hq", 16), ("Hkv", 1), ("D", 128)))
    a.batch, a.seqlen_q, a.seqlen_kv, a.num_q_heads, a.num_kv_heads, a.head_dim = B, Sq, Skv, Hq, Hkv, D
    a.causal = kw.get("causal", 1)
    a.window_size = kw.get("window", 0)
    a.head_dim_v = kw.get("Dv", 0)
    Dv = a.head_dim_v or D
    a.scale = kw.get("scale", D ** -0.5)
    for name, d in (("q_stride", D), ("grad_q_stride", D), ("o_stride", Dv), ("grad_o_stride", Dv)):
        getattr(a, name)[:] = [Sq * Hq * d, Hq * d, d]
    for name, d in (("k_stride", D), ("grad_k_stride", D), ("v_stride", Dv), ("grad_v_stride", Dv)):
        getattr(a, name)[:] = [Skv * Hkv * d, Hkv * d, d]
    for name in ("q", "k", "v", "o", "lse", "grad_o", "grad_q", "grad_k", "grad_v"):
        setattr(a, name, kw.get(name, 4096))
    a.kv_head_split = kw.get("hsplit", 0)
    a.dq_kernel = kw.get("dq_kernel", 0)
    return a


@pytest.mark.parametrize("kw,code", [
    (dict(Hq=15, Hkv=2), _lib.FGQA_ERR_INVALID_ARGUMENT),
    (dict(Sq=-1), _lib.FGQA_ERR_INVALID_ARGUMENT),
    (dict(scale=float("nan")), _lib.FGQA_ERR_INVALID_ARGUMENT),
    (dict(D=200), _lib.FGQA_ERR_UNSUPPORTED),             # Q/K 200: neither built nor padded
    (dict(D=64, Dv=200), _lib.FGQA_ERR_UNSUPPORTED),      # V/O above 128
    (dict(lse=None), _lib.FGQA_ERR_INVALID_ARGUMENT),
    (dict(grad_k=None), _lib.FGQA_ERR_INVALID_ARGUMENT),
    (dict(grad_v=4096 + 4), _lib.FGQA_ERR_UNSUPPORTED),
    (dict(window=-1), _lib.FGQA_ERR_INVALID_ARGUMENT),
    (dict(window=64, causal=0), _lib.FGQA_ERR_INVALID_ARGUMENT),   # the window is causal only
    (dict(D=192, Dv=160), _lib.FGQA_ERR_UNSUPPORTED),              # V/O above 128
    (dict(D=192, Dv=64, window=64), _lib.FGQA_ERR_UNSUPPORTED),    # padded to 192: no window form
    (dict(D=192, Dv=128, window=64), _lib.FGQA_ERR_UNSUPPORTED),   # no MLA window form
    (dict(D=128, Dv=192), _lib.FGQA_ERR_UNSUPPORTED),
    (dict(Dv=-1), _lib.FGQA_ERR_INVALID_ARGUMENT),
    (dict(hsplit=-1), _lib.FGQA_ERR_INVALID_ARGUMENT),
    (dict(hsplit=3), _lib.FGQA_ERR_INVALID_ARGUMENT),      # not a divisor of G = 16
    (dict(hsplit=32), _lib.FGQA_ERR_INVALID_ARGUMENT),     # more than G
    (dict(dq_kernel=3), _lib.FGQA_ERR_INVALID_ARGUMENT),
    (dict(D=192, Dv=128, dq_kernel=_lib.FGQA_KERNEL_SPLIT), _lib.FGQA_ERR_UNSUPPORTED),   # no split MLA dQ
])
def test_backward_rejects_before_launch(kw, code):
    assert _lib.lib().fgqa_prefill_backward_bf16(ctypes.byref(_backward_args(**kw)), None) == code


def test_backward_empty_is_noop():
    L = _lib.lib()
    assert L.fgqa_prefill_backward_bf16(ctypes.byref(_backward_args(B=0, q=None)), None) == 0
    assert L.fgqa_prefill_backward_bf16(ctypes.byref(_backward_args(Sq=0, Skv=0, q=None)), None) == 0
    assert L.fgqa_prefill_backward_bf16(None, None) == _lib.FGQA_ERR_INVALID_ARGUMENT
    n = ctypes.c_size_t(0)
    assert L.fgqa_prefill_backward_workspace_bytes(None, ctypes.byref(n)) == _lib.FGQA_ERR_INVALID_ARGUMENT
    assert L.fgqa_prefill_backward_workspace_bytes(ctypes.byref(_backward_args()), None) == \
        _lib.FGQA_ERR_INVALID_ARGUMENT


def test_backward_mirror_validation_without_gpu():
    """The mirror of the reference launcher raises the reference's ValueErrors
    (flash_gqa_backward_kernel.py:356-405) before touching a GPU."""
    import torch
    bf = torch.bfloat16
    q = torch.zeros(2, 4, 64, 128, dtype=bf)
    k = torch.zeros(2, 2, 64, 128, dtype=bf)
    lse = torch.zeros(2, 4, 64, dtype=torch.float32)
    f = fg.launch_flash_gqa_backward_bf16_kernel
    with pytest.raises(ValueError, match="expects bf16 inputs and grad_o"):
        f(q, k, k, q, lse, q.half())
    with pytest.raises(ValueError, match="lse to be float32"):
        f(q, k, k, q, lse.double(), q)
    with pytest.raises(ValueError, match="3D or 4D"):
        f(q[0, 0], k[0, 0], k[0, 0], q[0, 0], lse[0], q[0, 0])
    with pytest.raises(ValueError, match="matching ranks"):
        f(q, k[0], k, q, lse, q)
    with pytest.raises(ValueError, match="K and V must share sequence length"):
        f(q, k, k[:, :, :32], q, lse, q)
    with pytest.raises(ValueError, match="Q, O, and grad_o must share sequence length"):
        f(q, k, k, q[:, :, :32], lse, q)
    with pytest.raises(ValueError, match="share number of KV heads"):
        f(q, k, k[:, :1], q, lse, q)
    with pytest.raises(ValueError, match="share number of query heads"):
        f(q, k, k, q[:, :2], lse, q)
    with pytest.raises(ValueError, match="divisible"):
        f(q[:, :3], k, k, q[:, :3], lse[:, :3], q[:, :3])
    with pytest.raises(ValueError, match="LSE must be 3D"):
        f(q, k, k, q, lse[0], q)
    with pytest.raises(ValueError, match="LSE must be 2D"):
        f(q[0], k[0], k[0], q[0], lse, q[0])
    with pytest.raises(ValueError, match="LSE must have shape"):
        f(q, k, k, q, lse[:, :, :32], q)
    with pytest.raises(ValueError, match="GPU"):
        f(q, k, k, q, lse, q)


def test_swa_backward_mirror_validation_without_gpu():
    """The SWA backward mirror raises the reference's ValueErrors
    (SWA/flash_swa_backward_kernel.py:370-420) before touching a GPU."""
    import torch
    bf = torch.bfloat16
    q = torch.zeros(2, 4, 64, 128, dtype=bf)
    k = torch.zeros(2, 2, 64, 128, dtype=bf)
    lse = torch.zeros(2, 4, 64, dtype=torch.float32)
    f = fg.launch_flash_swa_backward_bf16_kernel
    with pytest.raises(ValueError, match="Flash SWA backward expects bf16 inputs and grad_o"):
        f(q, k, k, q, lse, q.half(), window_size=16)
    with pytest.raises(ValueError, match="Flash SWA backward expects lse to be float32"):
        f(q, k, k, q, lse.double(), q, window_size=16)
    with pytest.raises(ValueError, match="matching ranks"):
        f(q, k[0], k, q, lse, q, window_size=16)
    with pytest.raises(ValueError, match="LSE must have shape"):
        f(q, k, k, q, lse[:, :, :32], q, window_size=16)
    with pytest.raises(ValueError, match="window_size must be provided"):
        f(q, k, k, q, lse, q)
    with pytest.raises(ValueError, match="window_size must be positive"):
        f(q, k, k, q, lse, q, window_size=0)
    with pytest.raises(ValueError, match="GPU"):
        f(q, k, k, q, lse, q, window_size=16)


def _paged_args(**kw):
    a = _lib.PagedDecodeArgs()
    B, Hq, Hkv, D, ps = kw.get("B", 2), kw.get("Hq", 16), kw.get("Hkv", 2), kw.get("D", 128), kw.get("ps", 16)
    a.batch, a.num_q_heads, a.num_kv_heads, a.head_dim, a.page_size = B, Hq, Hkv, D, ps
    a.max_seqlen = kw.get("S", 256)
    a.num_pages = kw.get("pages", 64)
    a.kv_dtype = kw.get("dtype", _lib.FGQA_KV_BF16)
    a.scale, a.k_scale, a.v_scale = D ** -0.5, kw.get("ks", 1.0), 1.0
    a.q_stride[:] = [Hq * D, D]
    a.o_stride[:] = [Hq * D, D]
    st = kw.get("kstride", [ps * Hkv * D, Hkv * D, D])
    a.k_stride[:] = st
    a.v_stride[:] = st
    a.block_table_stride = kw.get("bts", 16)
    for name in ("q", "k_cache", "v_cache", "o", "block_table", "seqlens"):
        setattr(a, name, kw.get(name, 4096))
    return a


@pytest.mark.parametrize("kw,code", [
    (dict(ps=24), _lib.FGQA_ERR_UNSUPPORTED),
    (dict(S=257), _lib.FGQA_ERR_INVALID_ARGUMENT),          # table covers 16 pages x 16 = 256 tokens
    (dict(dtype=7), _lib.FGQA_ERR_INVALID_ARGUMENT),
    (dict(seqlens=None), _lib.FGQA_ERR_INVALID_ARGUMENT),
    (dict(block_table=None), _lib.FGQA_ERR_INVALID_ARGUMENT),
    (dict(ks=float("inf")), _lib.FGQA_ERR_INVALID_ARGUMENT),
    (dict(Hq=34, Hkv=2), _lib.FGQA_ERR_UNSUPPORTED),        # G = 17
    (dict(dtype=_lib.FGQA_KV_FP8_E4M3, kstride=[16 * 2 * 128, 2 * 128 + 8, 128]), _lib.FGQA_ERR_UNSUPPORTED),
    (dict(D=64), _lib.FGQA_ERR_UNSUPPORTED),
])
def test_paged_decode_rejects_before_launch(kw, code):
    assert _lib.lib().fgqa_decode_paged(ctypes.byref(_paged_args(**kw)), None) == code


def test_paged_decode_list_limit_rejected_by_query_and_launch():
    """A batch the work list cannot index (>= 2^15 sequences) is rejected by the
    workspace query and by the launch alike, before any workspace is taken
    (an explicit split size keeps the plan off the device)."""
    L = _lib.lib()
    a = _paged_args(B=1 << 15)
    a.split_tokens = 4096
    n = ctypes.c_size_t(0)
    assert L.fgqa_decode_paged_workspace_bytes(ctypes.byref(a), ctypes.byref(n)) == _lib.FGQA_ERR_UNSUPPORTED
    assert L.fgqa_decode_paged(ctypes.byref(a), None) == _lib.FGQA_ERR_UNSUPPORTED
    b = _paged_args(B=(1 << 15) - 1)
    b.split_tokens = 4096
    assert L.fgqa_decode_paged_workspace_bytes(ctypes.byref(b), ctypes.byref(n)) == 0 and n.value > 0


def test_paged_decode_empty_batch_is_noop():
    L = _lib.lib()
    assert L.fgqa_decode_paged(ctypes.byref(_paged_args(B=0, q=None)), None) == 0
    assert L.fgqa_decode_paged(None, None) == _lib.FGQA_ERR_INVALID_ARGUMENT


def test_cmake_build_matches_make(tmp_path):
    """The CMake build (gfx950 only) gives a library with the same exported
    entry points as the Makefile's, and refuses any other GPU target."""
    import shutil
    if shutil.which("cmake") is None or shutil.which("ninja") is None:
        pytest.skip("cmake / ninja not installed")
    bad = subprocess.run(["cmake", "-S", ROOT, "-B", str(tmp_path / "bad"), "-G", "Ninja",
                          "-DCMAKE_HIP_ARCHITECTURES=gfx942"], capture_output=True, text=True)
    assert bad.returncode != 0 and "gfx950" in (bad.stdout + bad.stderr)
    b = tmp_path / "build"
    subprocess.run(["cmake", "-S", ROOT, "-B", str(b), "-G", "Ninja"], check=True, capture_output=True)
    subprocess.run(["cmake", "--build", str(b), "-j", "8"], check=True, capture_output=True)

    def exports(path):
        out = subprocess.run(["nm", "-D", "--defined-only", path], check=True, capture_output=True,
                             text=True).stdout
        return {line.split()[-1] for line in out.splitlines()
                if " T " in line and ("fgqa_" in line or "Launch" in line or "FlashGqa" in line)}

    assert exports(str(b / "libfgqa.so")) == exports(_lib.LIB_PATH)


def test_mla_backward_mirror_validation_without_gpu():
    """The MLA backward mirror raises the reference's ValueErrors
    (flash_mla_backward_kernel.py:837-890) before touching a GPU."""
    import torch
    bf = torch.bfloat16
    q = torch.zeros(2, 4, 64, 192, dtype=bf)
    k = torch.zeros(2, 2, 64, 192, dtype=bf)
    v = torch.zeros(2, 2, 64, 128, dtype=bf)
    o = torch.zeros(2, 4, 64, 128, dtype=bf)
    lse = torch.zeros(2, 4, 64, dtype=torch.float32)
    f = fg.launch_flash_mla_backward_bf16_kernel
    with pytest.raises(ValueError, match="Flash MLA backward expects bf16 inputs and grad_o"):
        f(q, k, v, o, lse, o.half())
    with pytest.raises(ValueError, match="Flash MLA backward expects lse to be float32"):
        f(q, k, v, o, lse.double(), o)
    with pytest.raises(ValueError, match="Q and K must share head_dim_qk"):
        f(q, k[..., :128], v, o, lse, o)
    with pytest.raises(ValueError, match="O and grad_o must share head_dim_v with V"):
        f(q, k, v, q, lse, o)
    with pytest.raises(ValueError, match="not supported"):
        f(q[..., :160], k[..., :160], v, o, lse, o)
    with pytest.raises(ValueError, match="GPU"):
        f(q, k, v, o, lse, o)
