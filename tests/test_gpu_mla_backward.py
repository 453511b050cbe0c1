"""GPU parity tests of the MLA prefill backward (Q/K head dim 192, V/O 128)
against the CPU oracle.

The oracle (oracle/fgqa_oracle.c fgqa_oracle_prefill_mla_backward_bf16)
restates src/python/Triton/flash_mla_backward_kernel.py: the GQA backward's
steps with the scores over 192 dims and dP / delta over 128.  Inputs come
from the MLA forward oracle (O, LSE), so the GPU and the oracle see the same
O and LSE.  Bar: the backward's relative 2e-2 / 2e-3 (tests/_helpers.py
assert_grad_close).
"""
import ctypes
import math

import numpy as np
import pytest

import oracle
from tests._helpers import assert_grad_close, from_torch_bf16, gpu_normal_bf16, to_torch_bf16

pytestmark = pytest.mark.gpu

DQK, DV = 192, 128
SCALE = 1.0 / math.sqrt(DQK)


def _fg():
    import cuda_llm_ops_amd as fg
    return fg


def _sync():
    import torch
    torch.cuda.synchronize()


def _inputs(seed, B, Sq, Skv, Hq, Hkv, causal=True, scale=SCALE):
    q = oracle.normal_bf16(seed, (B, Sq, Hq, DQK))
    k = oracle.normal_bf16(seed, (B, Skv, Hkv, DQK), stream=1)
    v = oracle.normal_bf16(seed, (B, Skv, Hkv, DV), stream=2)
    do = oracle.normal_bf16(seed, (B, Sq, Hq, DV), stream=3)
    o, lse = oracle.prefill_mla(q, k, v, scale, causal=causal)
    return q, k, v, o, lse, do


def _check(grads, refs, what):
    for name, g, r in zip(("dq", "dk", "dv"), grads, refs):
        assert g.shape == r.shape, (what, name, g.shape, r.shape)
        ref = oracle.bf16_to_f32(oracle.f32_to_bf16(r))
        assert_grad_close(oracle.bf16_to_f32(g), ref, f"{what} {name}")


def _gpu_backward(cuda, q, k, v, o, lse, do, causal=True, scale=SCALE, workspace=None, **plan):
    import torch
    t = [to_torch_bf16(x, cuda) for x in (q, k, v, o, do)]
    lsed = torch.from_numpy(np.ascontiguousarray(lse)).to(cuda)
    dq, dk, dv = _fg().flash_gqa_backward_bshd(t[0], t[1], t[2], t[3], lsed, t[4], scale, causal=causal,
                                               workspace=workspace, **plan)
    _sync()
    return from_torch_bf16(dq), from_torch_bf16(dk), from_torch_bf16(dv)


@pytest.mark.parametrize("B,Sq,Skv,Hq,Hkv,causal", [
    (1, 256, 256, 16, 16, True),   # the reference's MLA grouping (G = 1)
    (1, 300, 300, 8, 2, True),     # G = 4, ragged tails
    (2, 200, 200, 4, 4, False),    # non-causal
    (1, 161, 97, 4, 1, True),      # Sq > Skv
    (1, 64, 640, 4, 2, True),      # Sq < Skv: keys >= Sq get zero gradients
    (1, 1, 1, 2, 1, True),         # one row, one key
    (1, 130, 130, 16, 1, True),    # G = 16: heads split over workgroups
])
def test_mla_backward_shapes(cuda, B, Sq, Skv, Hq, Hkv, causal):
    what = f"mla backward B{B} Sq{Sq} Skv{Skv} Hq{Hq} Hkv{Hkv} causal{causal}"
    print(what, flush=True)
    q, k, v, o, lse, do = _inputs(2100 + Sq, B, Sq, Skv, Hq, Hkv, causal=causal)
    refs = oracle.prefill_backward(q, k, v, o, lse, do, SCALE, causal=causal)
    grads = _gpu_backward(cuda, q, k, v, o, lse, do, causal=causal)
    _check(grads, refs, what)
    if causal and Skv > Sq:
        assert np.all(oracle.bf16_to_f32(grads[1])[:, Sq:] == 0)
        assert np.all(oracle.bf16_to_f32(grads[2])[:, Sq:] == 0)


@pytest.mark.parametrize("hsplit", [1, 2, 4])
def test_mla_backward_head_split_modes(cuda, hsplit):
    """Heads of a KV group in one workgroup (dK/dV straight from registers) or
    split over workgroups (fp32 partials of 192- and 128-wide rows summed)."""
    print(f"mla backward hsplit={hsplit}", flush=True)
    q, k, v, o, lse, do = _inputs(2210, 1, 384, 384, 8, 2)
    refs = oracle.prefill_backward(q, k, v, o, lse, do, SCALE, causal=True)
    _check(_gpu_backward(cuda, q, k, v, o, lse, do, kv_head_split=hsplit), refs, f"mla hsplit={hsplit}")


# a zero scale runs the dK/dV kernel's select form of the mask
@pytest.mark.parametrize("scale", [0.2, -0.05, 0.0])
def test_mla_backward_scale_values(cuda, scale):
    print(f"mla backward scale={scale}", flush=True)
    q, k, v, o, lse, do = _inputs(2220, 1, 200, 200, 4, 2, scale=scale)
    refs = oracle.prefill_backward(q, k, v, o, lse, do, scale, causal=True)
    _check(_gpu_backward(cuda, q, k, v, o, lse, do, scale=scale), refs, f"mla scale={scale}")


def test_mla_backward_mirror_chain_bhsd(cuda):
    """The reference's call sequence: the MLA forward mirror's O and LSE into
    the MLA backward mirror (flash_mla_backward_kernel.py:788-969), BHSD, 4-D
    and 3-D; the mirror at (128, 128) equals the GQA backward mirror bit for bit."""
    import torch
    fg = _fg()
    print("mla backward mirror chain", flush=True)
    B, S, Hq, Hkv = 2, 160, 4, 2
    q = oracle.normal_bf16(2230, (B, S, Hq, DQK))
    k = oracle.normal_bf16(2230, (B, S, Hkv, DQK), stream=1)
    v = oracle.normal_bf16(2230, (B, S, Hkv, DV), stream=2)
    do = oracle.normal_bf16(2230, (B, S, Hq, DV), stream=3)
    t = lambda x: to_torch_bf16(np.ascontiguousarray(x.transpose(0, 2, 1, 3)), cuda)  # noqa: E731
    back = lambda x: from_torch_bf16(x).transpose(0, 2, 1, 3)  # noqa: E731
    qd, kd, vd, dod = t(q), t(k), t(v), t(do)
    out, lse = fg.launch_flash_mla_forward_bf16_kernel(qd, kd, vd)
    dq, dk, dv = fg.launch_flash_mla_backward_bf16_kernel(qd, kd, vd, out, lse, dod)
    _sync()
    assert dq.shape == qd.shape and dk.shape == kd.shape and dv.shape == vd.shape
    refs = oracle.prefill_backward(q, k, v, back(out), lse.cpu().numpy(), do, SCALE, causal=True)
    _check((back(dq), back(dk), back(dv)), refs, "mla mirror 4-D")
    dq3, dk3, dv3 = fg.launch_flash_mla_backward_bf16_kernel(qd[1], kd[1], vd[1], out[1], lse[1], dod[1])
    _sync()
    back3 = lambda x: from_torch_bf16(x)[None].transpose(0, 2, 1, 3)  # noqa: E731
    _check((back3(dq3), back3(dk3), back3(dv3)), tuple(r[1:] for r in refs), "mla mirror 3-D")
    # (128, 128) through the MLA mirror is the GQA backward
    q1 = t(oracle.normal_bf16(2231, (B, S, Hq, 128)))
    k1 = t(oracle.normal_bf16(2231, (B, S, Hkv, 128), stream=1))
    v1 = t(oracle.normal_bf16(2231, (B, S, Hkv, 128), stream=2))
    d1 = t(oracle.normal_bf16(2231, (B, S, Hq, 128), stream=3))
    o1, l1 = fg.launch_flash_gqa_forward_bf16_kernel(q1, k1, v1)
    g_mla = fg.launch_flash_mla_backward_bf16_kernel(q1, k1, v1, o1, l1, d1)
    g_gqa = fg.launch_flash_gqa_backward_bf16_kernel(q1, k1, v1, o1, l1, d1)
    _sync()
    for a, b in zip(g_mla, g_gqa):
        assert torch.equal(a, b)


def test_mla_backward_caller_workspace(cuda):
    """A caller workspace sized for the MLA shapes (one byte short is rejected)."""
    import torch
    fg = _fg()
    print("mla backward caller workspace", flush=True)
    B, S, Hq, Hkv = 1, 256, 16, 1
    q, k, v, o, lse, do = _inputs(2240, B, S, S, Hq, Hkv)
    refs = oracle.prefill_backward(q, k, v, o, lse, do, SCALE, causal=True)
    n = fg.backward_workspace_bytes(B, S, S, Hq, Hkv, head_dim=DQK, head_dim_v=DV)
    small = torch.empty(n - 1, dtype=torch.uint8, device=cuda)
    qd, kd, vd, od, dod = (to_torch_bf16(x, cuda) for x in (q, k, v, o, do))
    lsed = torch.from_numpy(lse).to(cuda)
    with pytest.raises(fg.FgqaError):
        fg.flash_gqa_backward_bshd(qd, kd, vd, od, lsed, dod, SCALE, workspace=small)
    ws = torch.empty(n, dtype=torch.uint8, device=cuda)
    g = fg.flash_gqa_backward_bshd(qd, kd, vd, od, lsed, dod, SCALE, workspace=ws)
    _sync()
    _check(tuple(from_torch_bf16(x) for x in g), refs, "mla caller workspace")


def test_mla_backward_reference_shape_full_size(cuda):
    """The reference's MLA benchmark shape (B=1, S=4096, Hq = Hkv = 16, causal),
    N(0,1) inputs: GPU forward then backward; sampled rows / keys against the
    oracle, plus sum_j dK_j ~ 0 and sum_j dV_j ~ sum_i dO_i per head over every key."""
    import torch
    fg = _fg()
    print("mla backward reference shape", flush=True)
    B, S, H = 1, 4096, 16
    q = gpu_normal_bf16((B, S, H, DQK), 71, 1.0, cuda)
    k = gpu_normal_bf16((B, S, H, DQK), 72, 1.0, cuda)
    v = gpu_normal_bf16((B, S, H, DV), 73, 1.0, cuda)
    do = gpu_normal_bf16((B, S, H, DV), 74, 1.0, cuda)
    out, lse = fg.flash_gqa_forward_bshd(q, k, v, SCALE)
    dq, dk, dv = fg.flash_gqa_backward_bshd(q, k, v, out, lse, do, SCALE)
    _sync()
    for g in (dq, dk, dv):
        assert bool(g.isfinite().all())
    h = [from_torch_bf16(x) for x in (q, k, v, out, do)]
    lse_np = lse.cpu().numpy()
    gq, gk, gv = (from_torch_bf16(x) for x in (dq, dk, dv))
    for rows in ((0, 32), (S - 32, S)):
        rq, _, _ = oracle.prefill_backward(*h[:4], lse_np, h[4], SCALE, causal=True, rows=rows, want=("dq",))
        assert_grad_close(oracle.bf16_to_f32(gq[:, rows[0]:rows[1]]),
                          oracle.bf16_to_f32(oracle.f32_to_bf16(rq[:, rows[0]:rows[1]])), f"mla dq rows {rows}")
    for keys in ((0, 4), (S - 32, S)):
        _, rk, rv = oracle.prefill_backward(*h[:4], lse_np, h[4], SCALE, causal=True, keys=keys,
                                            want=("dk", "dv"))
        for name, g, r in (("dk", gk, rk), ("dv", gv, rv)):
            assert_grad_close(oracle.bf16_to_f32(g[:, keys[0]:keys[1]]),
                              oracle.bf16_to_f32(oracle.f32_to_bf16(r[:, keys[0]:keys[1]])),
                              f"mla {name} keys {keys}")
    sk = dk.double().sum(1)
    assert float(sk.abs().max()) < 5e-3 * float(dk.double().abs().sum(1).mean())
    dosum = do.double().sum(1)                     # [B, H, DV]: G = 1
    err = (dv.double().sum(1) - dosum).abs().max()
    assert float(err) < 2e-3 * float(dosum.abs().max())


def test_mla_backward_cplusplus_dropin(cuda):
    """LaunchFlashMlaBackwardBf16Kernel (BSHD, default stream)."""
    import torch
    fg = _fg()
    L = fg.lib()
    print("mla backward C++ entry point", flush=True)
    B, S, Hq, Hkv = 1, 192, 4, 2
    q, k, v, o, lse, do = _inputs(2250, B, S, S, Hq, Hkv)
    refs = oracle.prefill_backward(q, k, v, o, lse, do, SCALE, causal=True)
    qd, kd, vd, od, dod = (to_torch_bf16(x, cuda) for x in (q, k, v, o, do))
    lsed = torch.from_numpy(lse).to(cuda)
    gq, gk, gv = torch.zeros_like(qd), torch.zeros_like(kd), torch.zeros_like(vd)
    fn = getattr(L, "_Z32LaunchFlashMlaBackwardBf16KernelPK6bf16_tS1_S1_S1_PKfS1_fPS_S4_S4_iiiiiiib")
    fn.restype = None
    torch.cuda.synchronize()
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    fn(p(qd), p(kd), p(vd), p(od), p(lsed), p(dod), ctypes.c_float(SCALE), p(gq), p(gk), p(gv),
       B, S, S, Hq, Hkv, DQK, DV, ctypes.c_bool(True))
    st = getattr(L, "_Z21FlashGqaGetLastStatusv")
    st.restype = ctypes.c_int
    assert st() == 0
    torch.cuda.synchronize()
    _check((from_torch_bf16(gq), from_torch_bf16(gk), from_torch_bf16(gv)), refs, "C++ mla backward")
