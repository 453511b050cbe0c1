"""GPU tests of the sparse-index prefill against the CPU oracle.

The oracle (oracle/fgqa_oracle.c fgqa_oracle_sparse_prefill_bf16) restates the
reference's torch reference, examples/python/Triton/test_flash_sgqa_kernel.py:97-222.
Bar: max-abs 2e-2 and mean-abs 2e-3 on bf16 outputs, LSE within 1e-3.
"""
import math

import numpy as np
import pytest

import oracle
from tests._helpers import (assert_close, build_sparse_indices, from_torch_bf16, gpu_normal_bf16,
                            gpu_sparse_indices, to_torch_bf16)

pytestmark = pytest.mark.gpu

SCALE = 1.0 / math.sqrt(128)
LSE_TOL = 1e-3


def _fg():
    import cuda_llm_ops_amd as fg
    return fg


def _check(o, lse, o_ref, l_ref, what):
    assert_close(oracle.bf16_to_f32(o), oracle.bf16_to_f32(o_ref), what)
    fin = np.isfinite(l_ref)
    assert np.array_equal(np.isfinite(lse), fin), f"{what}: lse finiteness"
    assert np.max(np.abs(lse[fin] - l_ref[fin]), initial=0.0) <= LSE_TOL, f"{what}: lse"


def _inputs(seed, B, Sq, Skv, Hq, Hkv):
    q = oracle.normal_bf16(seed, (B, Sq, Hq, 128))
    k = oracle.normal_bf16(seed, (B, Skv, Hkv, 128), stream=1)
    v = oracle.normal_bf16(seed, (B, Skv, Hkv, 128), stream=2)
    return q, k, v


def _edge_entries(idx, Sq, Skv, seed):
    """Overwrite the last slots with entries the kernel must skip or keep:
    out of range, a future key, a key listed twice, -1."""
    rng = np.random.default_rng(seed)
    idx = idx.copy()
    n = idx.shape[3]
    if n >= 4:
        idx[..., -1] = rng.integers(Skv, 2 * Skv + 1, size=idx.shape[:3])
        idx[..., -2] = np.minimum(np.arange(Sq)[None, None, :] + 3, max(Skv - 1, 0))
        idx[..., -3] = idx[..., 0]
        idx[..., -4] = -1
    return idx


def _run(cuda, q, k, v, idx, scale=SCALE, causal=True):
    import torch
    qd, kd, vd = (to_torch_bf16(x, cuda) for x in (q, k, v))
    idd = torch.from_numpy(np.ascontiguousarray(idx)).to(cuda)
    out, lse = _fg().flash_sgqa_forward_bshd(qd, kd, vd, idd, scale, causal=causal)
    torch.cuda.synchronize()
    return from_torch_bf16(out), lse.cpu().numpy()


@pytest.mark.parametrize("B,Sq,Skv,Hq,Hkv,nsparse,causal", [
    (1, 300, 300, 16, 1, 64, True),     # the reference's head layout (G = 16)
    (2, 257, 257, 8, 2, 40, True),      # list length not a multiple of 32, G = 4
    (1, 200, 200, 4, 4, 33, False),     # non-causal, G = 1
    (1, 128, 128, 32, 1, 48, True),     # G = 32: two head groups per position
    (1, 100, 100, 6, 2, 20, True),      # G = 3: a partial head group
    (1, 150, 300, 4, 1, 64, False),     # Sq < Skv
    (1, 300, 120, 4, 1, 64, True),      # Sq > Skv
    (1, 700, 700, 16, 1, 512, True),    # the longest list the kernel sorts by key
    (1, 700, 700, 16, 1, 513, True),    # one longer: taken in list order
    (1, 400, 900, 4, 2, 1000, False),   # list order, non-causal
])
def test_sparse_shapes(cuda, B, Sq, Skv, Hq, Hkv, nsparse, causal):
    what = f"sparse B{B} Sq{Sq} Skv{Skv} Hq{Hq} Hkv{Hkv} n{nsparse} causal={causal}"
    print(what, flush=True)
    q, k, v = _inputs(3000 + Sq + nsparse, B, Sq, Skv, Hq, Hkv)
    idx = build_sparse_indices(3100 + Sq, B, Hkv, Sq, Skv, nsparse)
    idx = _edge_entries(idx, Sq, Skv, Sq)
    o_ref, l_ref = oracle.sparse_prefill(q, k, v, idx, SCALE, causal=causal)
    o, lse = _run(cuda, q, k, v, idx, causal=causal)
    _check(o, lse, o_ref, l_ref, what)


def test_sparse_rows_without_entries_and_negative_scale(cuda):
    """Rows whose entries are all unusable give O = 0 and lse = -inf; a negative scale."""
    print("sparse empty rows / negative scale", flush=True)
    B, S, Hq, Hkv, n = 1, 96, 8, 2, 32
    q, k, v = _inputs(3200, B, S, S, Hq, Hkv)
    idx = build_sparse_indices(3201, B, Hkv, S, S, n)
    idx[:, :, 10] = -1                      # nothing listed
    idx[:, :, 11] = 50                      # only future keys
    idx[:, 1, 12] = S + 5                   # only out-of-range keys (kv head 1)
    for scale in (SCALE, -0.07):
        o_ref, l_ref = oracle.sparse_prefill(q, k, v, idx, scale, causal=True)
        o, lse = _run(cuda, q, k, v, idx, scale=scale)
        _check(o, lse, o_ref, l_ref, f"sparse empty rows scale={scale}")
    assert np.all(oracle.bf16_to_f32(o)[:, 10:12] == 0) and np.all(np.isneginf(lse[:, :, 10:12]))
    assert np.all(oracle.bf16_to_f32(o)[:, 12, 4:] == 0) and np.all(np.isneginf(lse[:, 4:, 12]))


def test_sparse_dense_lists_match_the_prefill_kernel(cuda):
    """Every row listing keys 0..S-1: the dense causal prefill kernel's result."""
    import torch
    fg = _fg()
    print("sparse dense lists vs prefill", flush=True)
    B, S, Hq, Hkv = 1, 256, 8, 2
    q, k, v = _inputs(3300, B, S, S, Hq, Hkv)
    idx = np.broadcast_to(np.arange(S, dtype=np.int32), (B, Hkv, S, S)).copy()
    o, lse = _run(cuda, q, k, v, idx)
    qd, kd, vd = (to_torch_bf16(x, cuda) for x in (q, k, v))
    od, ld = fg.flash_gqa_forward_bshd(qd, kd, vd, SCALE, causal=True)
    torch.cuda.synchronize()
    _check(o, lse, from_torch_bf16(od), ld.cpu().numpy(), "sparse dense vs prefill kernel")


def test_sparse_reference_shape_full_size(cuda):
    """The reference's benchmark shape (B=1, S=32768, Hq=16, Hkv=1, 512 entries per
    row, causal, recent-16 + random lists): sampled row blocks against the oracle."""
    import torch
    fg = _fg()
    print("sparse full size", flush=True)
    B, S, Hq, Hkv, n = 1, 32768, 16, 1, 512
    q = gpu_normal_bf16((B, S, Hq, 128), 81, 1.0, cuda)
    k = gpu_normal_bf16((B, S, Hkv, 128), 82, 1.0, cuda)
    v = gpu_normal_bf16((B, S, Hkv, 128), 83, 1.0, cuda)
    idx = gpu_sparse_indices(B, Hkv, S, n, 84, cuda)
    out, lse = fg.flash_sgqa_forward_bshd(q, k, v, idx, SCALE, causal=True)
    torch.cuda.synchronize()
    assert bool(out.isfinite().all())
    kh, vh = from_torch_bf16(k), from_torch_bf16(v)
    for r0, r1 in ((0, 40), (700, 740), (20000, 20040), (S - 40, S)):
        o_ref, l_ref = oracle.sparse_prefill(from_torch_bf16(q[:, r0:r1]), kh, vh,
                                             idx[:, :, r0:r1].cpu().numpy(), SCALE, causal=True, q_offset=r0)
        _check(from_torch_bf16(out[:, r0:r1]), lse[:, :, r0:r1].cpu().numpy(), o_ref, l_ref,
               f"sparse full size rows {r0}:{r1}")


def test_sparse_reference_mirror_bhsd(cuda):
    """launch_flash_sgqa_forward_bf16_kernel with BHSD tensors (4-D and 3-D), the
    reference's out/lse contract and zero-query guard
    (test_flash_sgqa_kernel.py:587-720)."""
    import torch
    fg = _fg()
    print("sparse mirror", flush=True)
    B, S, Hq, Hkv, n = 2, 200, 8, 2, 48
    q, k, v = _inputs(3400, B, S, S, Hq, Hkv)
    idx = build_sparse_indices(3401, B, Hkv, S, S, n)
    o_ref, l_ref = oracle.sparse_prefill(q, k, v, idx, SCALE, causal=True)
    t = lambda x: to_torch_bf16(np.ascontiguousarray(x.transpose(0, 2, 1, 3)), cuda)  # noqa: E731
    idd = torch.from_numpy(idx).to(cuda)
    out, lse = fg.launch_flash_sgqa_forward_bf16_kernel(t(q), t(k), t(v), idd, num_sparse_kv=n)
    torch.cuda.synchronize()
    _check(from_torch_bf16(out).transpose(0, 2, 1, 3), lse.cpu().numpy(), o_ref, l_ref, "sparse mirror 4-D")
    o3, l3 = fg.launch_flash_sgqa_forward_bf16_kernel(t(q)[1], t(k)[1], t(v)[1], idd[1:], num_sparse_kv=n)
    torch.cuda.synchronize()
    assert torch.equal(o3, out[1]) and torch.equal(l3, lse[1])
    # a provided contiguous out / lse is returned as is; non-contiguous ones are rejected
    ob, lb = torch.empty_like(out), torch.empty_like(lse)
    r = fg.launch_flash_sgqa_forward_bf16_kernel(t(q), t(k), t(v), idd, num_sparse_kv=n, out=ob, lse=lb)
    torch.cuda.synchronize()
    assert r[0] is ob and r[1] is lb and torch.equal(ob, out) and torch.equal(lb, lse)
    with pytest.raises(ValueError, match="Output must be contiguous when provided"):
        fg.launch_flash_sgqa_forward_bf16_kernel(t(q), t(k), t(v), idd, num_sparse_kv=n,
                                                 out=torch.empty_like(out).transpose(2, 3))
    with pytest.raises(ValueError, match="LSE must be contiguous when provided"):
        fg.launch_flash_sgqa_forward_bf16_kernel(t(q), t(k), t(v), idd, num_sparse_kv=n,
                                                 lse=torch.empty((B, S, Hq), device=cuda).transpose(1, 2))
    with pytest.raises(ValueError, match=r"sparse_kv_indices must have shape \[batch, num_kv_heads, seqlen_q, 47\]"):
        fg.launch_flash_sgqa_forward_bf16_kernel(t(q), t(k), t(v), idd, num_sparse_kv=47)
    # zero queries: empty outputs, nothing launched
    q0 = t(q)[:, :, :0]
    idx0 = idd[:, :, :0]
    o0, l0 = fg.launch_flash_sgqa_forward_bf16_kernel(q0, t(k), t(v), idx0, num_sparse_kv=n)
    assert o0.shape == (B, Hq, 0, 128) and l0.shape == (B, Hq, 0)


def test_sparse_cplusplus_entry(cuda):
    """LaunchFlashSgqaForwardBf16Kernel (BSHD, default stream)."""
    import ctypes

    import torch
    fg = _fg()
    L = fg.lib()
    print("sparse C++ entry", flush=True)
    B, S, Hq, Hkv, n = 1, 160, 8, 2, 36
    q, k, v = _inputs(3500, B, S, S, Hq, Hkv)
    idx = _edge_entries(build_sparse_indices(3501, B, Hkv, S, S, n), S, S, 7)
    o_ref, l_ref = oracle.sparse_prefill(q, k, v, idx, SCALE, causal=True)
    qd, kd, vd = (to_torch_bf16(x, cuda) for x in (q, k, v))
    idd = torch.from_numpy(idx).to(cuda)
    od = torch.zeros_like(qd)
    ld = torch.zeros((B, Hq, S), dtype=torch.float32, device=cuda)
    fn = getattr(L, "_Z32LaunchFlashSgqaForwardBf16KernelPK6bf16_tS1_S1_PKiifPS_Pfiiiiiib")
    fn.restype = None
    st = getattr(L, "_Z21FlashGqaGetLastStatusv")
    st.restype = ctypes.c_int
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    torch.cuda.synchronize()
    fn(p(qd), p(kd), p(vd), p(idd), n, ctypes.c_float(SCALE), p(od), p(ld), B, S, S, Hq, Hkv, 128, True)
    assert st() == 0
    torch.cuda.synchronize()
    _check(from_torch_bf16(od), ld.cpu().numpy(), o_ref, l_ref, "C++ sparse")
    fn(p(qd), p(kd), p(vd), p(idd), 0, ctypes.c_float(SCALE), p(od), p(ld), B, S, S, Hq, Hkv, 128, True)
    assert st() == -1
