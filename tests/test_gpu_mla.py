"""GPU tests of the MLA prefill (Q/K head dim 192, V/O head dim 128) against the CPU oracle.

The oracle (oracle/fgqa_oracle.c fgqa_oracle_prefill_mla_bf16) restates the
reference's torch MLA reference, examples/python/Triton/test_flash_mla_kernel.py:27-95.
Bar: max-abs 2e-2 and mean-abs 2e-3 on bf16 outputs, LSE within 1e-3.
"""
import math

import numpy as np
import pytest

import oracle
from tests._helpers import assert_close, from_torch_bf16, gpu_normal_bf16, to_torch_bf16

pytestmark = pytest.mark.gpu

DQK, DV = 192, 128
SCALE = 1.0 / math.sqrt(DQK)   # the reference launcher's default
LSE_TOL = 1e-3


def _fg():
    import cuda_llm_ops_amd as fg
    return fg


def _check(o, lse, o_ref, l_ref, what):
    assert_close(oracle.bf16_to_f32(o), oracle.bf16_to_f32(o_ref), what)
    fin = np.isfinite(l_ref)
    assert np.array_equal(np.isfinite(lse), fin), f"{what}: lse finiteness"
    assert np.max(np.abs(lse[fin] - l_ref[fin]), initial=0.0) <= LSE_TOL, f"{what}: lse"


def _inputs(seed, B, Sq, Skv, Hq, Hkv, uniform=False):
    if uniform:   # the reference test's inputs: torch.rand, U[0, 1)
        rng = np.random.default_rng(seed)
        mk = lambda shape: oracle.f32_to_bf16(rng.random(shape, dtype=np.float32))  # noqa: E731
        return mk((B, Sq, Hq, DQK)), mk((B, Skv, Hkv, DQK)), mk((B, Skv, Hkv, DV))
    q = oracle.normal_bf16(seed, (B, Sq, Hq, DQK))
    k = oracle.normal_bf16(seed, (B, Skv, Hkv, DQK), stream=1)
    v = oracle.normal_bf16(seed, (B, Skv, Hkv, DV), stream=2)
    return q, k, v


@pytest.mark.parametrize("split", ["whole", "split", "wide"])
@pytest.mark.parametrize("B,Sq,Skv,Hq,Hkv,causal", [
    (1, 256, 256, 2, 2, True),     # G = 1, the reference's MLA head layout
    (1, 1500, 1500, 4, 4, True),   # G = 1, wide units of 256 positions, split pairs
    (8, 600, 600, 16, 16, True),   # more unit pairs than one per two CUs: whole wide units, persistent
    (2, 300, 300, 4, 1, True),     # ragged tail, G = 4
    (1, 257, 257, 16, 1, True),    # G = 16
    (1, 200, 330, 2, 1, False),    # non-causal, Sq != Skv
    (1, 330, 200, 6, 3, True),     # Sq > Skv (rows past the keys see all of them)
    (1, 100, 160, 4, 2, True),     # Sq < Skv, causal: top-left aligned
])
def test_mla_shapes(cuda, split, B, Sq, Skv, Hq, Hkv, causal):
    what = f"mla kernel={split} B{B} Sq{Sq} Skv{Skv} Hq{Hq} Hkv{Hkv} causal={causal}"
    print(what, flush=True)
    q, k, v = _inputs(2000 + Sq + Skv, B, Sq, Skv, Hq, Hkv)
    o_ref, l_ref = oracle.prefill_mla(q, k, v, SCALE, causal=causal)
    qd, kd, vd = (to_torch_bf16(x, cuda) for x in (q, k, v))
    out, lse = _fg().flash_gqa_forward_bshd(qd, kd, vd, SCALE, causal=causal, kernel=split)
    assert out.shape == (B, Sq, Hq, DV)
    _check(from_torch_bf16(out), lse.cpu().numpy(), o_ref, l_ref, what)


def test_mla_reference_inputs_and_negative_scale(cuda):
    """U[0,1) inputs (the reference test's distribution) and a negative scale."""
    fg = _fg()
    print("mla uniform inputs / negative scale", flush=True)
    q, k, v = _inputs(2100, 1, 384, 384, 4, 4, uniform=True)
    qd, kd, vd = (to_torch_bf16(x, cuda) for x in (q, k, v))
    for scale in (SCALE, -0.05):
        o_ref, l_ref = oracle.prefill_mla(q, k, v, scale, causal=True)
        out, lse = fg.flash_gqa_forward_bshd(qd, kd, vd, scale, causal=True)
        _check(from_torch_bf16(out), lse.cpu().numpy(), o_ref, l_ref, f"mla uniform scale={scale}")


def test_mla_reference_shape_full_size(cuda):
    """The reference's MLA benchmark shape (B=1, S=4096, Hq=Hkv=16, Dqk=192, Dv=128,
    causal), N(0,1) inputs: sampled row blocks against the oracle, every kernel."""
    import torch
    fg = _fg()
    B, S, Hq, Hkv = 1, 4096, 16, 16
    q = gpu_normal_bf16((B, S, Hq, DQK), 71, 1.0, cuda)
    k = gpu_normal_bf16((B, S, Hkv, DQK), 72, 1.0, cuda)
    v = gpu_normal_bf16((B, S, Hkv, DV), 73, 1.0, cuda)
    for split in ("whole", "split", "wide"):
        print(f"mla full size kernel={split}", flush=True)
        out, lse = fg.flash_gqa_forward_bshd(q, k, v, SCALE, causal=True, kernel=split)
        torch.cuda.synchronize()
        assert bool(out.isfinite().all())
        for r0, r1 in ((0, 64), (2000, 2064), (S - 64, S)):
            o_ref, l_ref = oracle.prefill_mla(from_torch_bf16(q[:, r0:r1]), from_torch_bf16(k[:, :r1]),
                                              from_torch_bf16(v[:, :r1]), SCALE, causal=True, q_offset=r0)
            _check(from_torch_bf16(out[:, r0:r1]), lse[:, :, r0:r1].cpu().numpy(), o_ref, l_ref,
                   f"mla full size split={split} rows {r0}:{r1}")


def test_mla_reference_mirror_bhsd(cuda):
    """launch_flash_mla_forward_bf16_kernel with the reference's BHSD tensors, 4-D and 3-D,
    its default scale 1/sqrt(Dqk), and its ValueErrors."""
    import torch
    fg = _fg()
    print("mla mirror", flush=True)
    B, S, Hq, Hkv = 2, 200, 4, 2
    q, k, v = _inputs(2200, B, S, S, Hq, Hkv)
    o_ref, l_ref = oracle.prefill_mla(q, k, v, SCALE, causal=True)
    t = lambda x: to_torch_bf16(np.ascontiguousarray(x.transpose(0, 2, 1, 3)), cuda)  # noqa: E731
    out, lse = fg.launch_flash_mla_forward_bf16_kernel(t(q), t(k), t(v))
    torch.cuda.synchronize()
    assert out.shape == (B, Hq, S, DV)
    _check(from_torch_bf16(out).transpose(0, 2, 1, 3), lse.cpu().numpy(), o_ref, l_ref, "mla mirror 4-D")
    o3, l3 = fg.launch_flash_mla_forward_bf16_kernel(t(q)[1], t(k)[1], t(v)[1])
    torch.cuda.synchronize()
    assert torch.equal(o3, out[1]) and torch.equal(l3, lse[1])
    # provided out / lse are written in place
    ob = torch.empty_like(out)
    lb = torch.empty_like(lse)
    r = fg.launch_flash_mla_forward_bf16_kernel(t(q), t(k), t(v), out=ob, lse=lb)
    torch.cuda.synchronize()
    assert r[0] is ob and r[1] is lb and torch.equal(ob, out) and torch.equal(lb, lse)
    with pytest.raises(ValueError, match="Flash MLA forward expects bf16 inputs"):
        fg.launch_flash_mla_forward_bf16_kernel(t(q).float(), t(k), t(v))
    with pytest.raises(ValueError, match="Q and K must share head_dim_qk"):
        fg.launch_flash_mla_forward_bf16_kernel(t(q)[..., :128], t(k), t(v))
    with pytest.raises(ValueError, match="Output must have shape"):
        fg.launch_flash_mla_forward_bf16_kernel(t(q), t(k), t(v), out=torch.empty_like(t(q)))
    with pytest.raises(ValueError, match="not supported"):
        v320 = torch.zeros((*t(v).shape[:-1], 320), dtype=torch.bfloat16, device=cuda)
        fg.launch_flash_mla_forward_bf16_kernel(t(q), t(k), v320)


def test_mla_mirror_equal_dims_is_the_gqa_prefill(cuda):
    """(Dqk, Dv) = (128, 128) through the MLA mirror: the GQA mirror's result, bit for bit."""
    import torch
    fg = _fg()
    print("mla mirror 128/128", flush=True)
    B, S, Hq, Hkv = 1, 190, 4, 1
    q = oracle.normal_bf16(2300, (B, Hq, S, 128))
    k = oracle.normal_bf16(2300, (B, Hkv, S, 128), stream=1)
    v = oracle.normal_bf16(2300, (B, Hkv, S, 128), stream=2)
    qd, kd, vd = (to_torch_bf16(x, cuda) for x in (q, k, v))
    o1, l1 = fg.launch_flash_mla_forward_bf16_kernel(qd, kd, vd)
    o2, l2 = fg.launch_flash_gqa_forward_bf16_kernel(qd, kd, vd)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(l1, l2)


def test_mla_cplusplus_entry(cuda):
    """LaunchFlashMlaForwardBf16Kernel (BSHD, default stream)."""
    import ctypes

    import torch
    fg = _fg()
    L = fg.lib()
    print("mla C++ entry", flush=True)
    B, S, Hq, Hkv = 1, 260, 4, 2
    q, k, v = _inputs(2400, B, S, S, Hq, Hkv)
    o_ref, l_ref = oracle.prefill_mla(q, k, v, SCALE, causal=True)
    qd, kd, vd = (to_torch_bf16(x, cuda) for x in (q, k, v))
    od = torch.zeros((B, S, Hq, DV), dtype=torch.bfloat16, device=cuda)
    ld = torch.zeros((B, Hq, S), dtype=torch.float32, device=cuda)
    fn = getattr(L, "_Z31LaunchFlashMlaForwardBf16KernelPK6bf16_tS1_S1_fPS_Pfiiiiiiib")
    fn.restype = None
    st = getattr(L, "_Z21FlashGqaGetLastStatusv")
    st.restype = ctypes.c_int
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    torch.cuda.synchronize()
    fn(p(qd), p(kd), p(vd), ctypes.c_float(SCALE), p(od), p(ld), B, S, S, Hq, Hkv, DQK, DV, True)
    assert st() == 0
    torch.cuda.synchronize()
    _check(from_torch_bf16(od), ld.cpu().numpy(), o_ref, l_ref, "C++ MLA")
    # (192, 64): the 192 kernels on V zero-padded to 128
    v64 = vd[..., :64].contiguous()
    o64 = torch.zeros((B, S, Hq, 64), dtype=torch.bfloat16, device=cuda)
    fn(p(qd), p(kd), p(v64), ctypes.c_float(SCALE), p(o64), p(ld), B, S, S, Hq, Hkv, DQK, 64, True)
    assert st() == 0
    torch.cuda.synchronize()
    o_ref64, l_ref64 = oracle.prefill_mla(q, k, np.ascontiguousarray(v[..., :64]), SCALE, causal=True)
    _check(from_torch_bf16(o64), ld.cpu().numpy(), o_ref64, l_ref64, "C++ (192, 64)")
    # V rows above 256 are not built: refused before any launch
    fn(p(qd), p(kd), p(vd), ctypes.c_float(SCALE), p(od), p(ld), B, S, S, Hq, Hkv, DQK, 320, True)
    assert st() == -2
