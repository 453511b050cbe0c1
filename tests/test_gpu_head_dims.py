"""GPU tests of the prefill at head dims other than the built (128, 128),
(192, 128) and (256, 128) against the CPU oracle.

The reference's Triton launcher takes any head dim and pads its head-dim
blocks to a power of two (src/python/Triton/flash_gqa_kernel.py:266-269);
this library runs such calls on copies of Q and K zero-padded to 128, 192 or
256 and of V to 128 or 256 (two launches of 128 columns), and copies the
first head_dim_v columns of O back.  The oracle
(oracle/fgqa_oracle.c: fgqa_oracle_prefill_bf16, _mla_bf16, _swa_bf16) takes
the head dims as they are, so these tests check the padding against the
unpadded maths.  Bar: max-abs 2e-2 and mean-abs 2e-3 on bf16 outputs, LSE
within 1e-3.
"""
import ctypes
import math

import numpy as np
import pytest

import oracle
from tests._helpers import assert_close, from_torch_bf16, to_torch_bf16

pytestmark = pytest.mark.gpu

LSE_TOL = 1e-3


def _fg():
    import cuda_llm_ops_amd as fg
    return fg


def _check(o, lse, o_ref, l_ref, what):
    assert_close(oracle.bf16_to_f32(o), oracle.bf16_to_f32(o_ref), what)
    fin = np.isfinite(l_ref)
    assert np.array_equal(np.isfinite(lse), fin), f"{what}: lse finiteness"
    assert np.max(np.abs(lse[fin] - l_ref[fin]), initial=0.0) <= LSE_TOL, f"{what}: lse"


def _inputs(seed, B, Sq, Skv, Hq, Hkv, dqk, dv):
    q = oracle.normal_bf16(seed, (B, Sq, Hq, dqk))
    k = oracle.normal_bf16(seed, (B, Skv, Hkv, dqk), stream=1)
    v = oracle.normal_bf16(seed, (B, Skv, Hkv, dv), stream=2)
    return q, k, v


DIMS = [(64, 64), (32, 32), (96, 96), (100, 100), (64, 128), (128, 64), (72, 40), (1, 8),
        (256, 256), (256, 128), (192, 64), (128, 192), (200, 72), (160, 160), (192, 192), (8, 256)]


def _kernels(dqk):
    """The kernel shapes a pair runs on: Q/K above 128 (other than 192) pads
    to 256, which only the whole-range kernel is built for."""
    return ["auto", "whole"] if dqk > 128 and dqk != 192 else ["auto", "whole", "split", "wide"]


@pytest.mark.parametrize("dqk,dv,kernel", [(a, b, k) for a, b in DIMS for k in _kernels(a)])
@pytest.mark.parametrize("B,Sq,Skv,Hq,Hkv,causal", [
    (1, 300, 300, 8, 2, True),
    (2, 200, 330, 4, 1, False),
    (1, 330, 200, 6, 3, True),
])
def test_padded_head_dims(cuda, kernel, dqk, dv, B, Sq, Skv, Hq, Hkv, causal):
    what = f"D=({dqk},{dv}) kernel={kernel} B{B} Sq{Sq} Skv{Skv} Hq{Hq} Hkv{Hkv} causal={causal}"
    print(what, flush=True)
    scale = 1.0 / math.sqrt(dqk)
    q, k, v = _inputs(3000 + dqk + dv + Sq, B, Sq, Skv, Hq, Hkv, dqk, dv)
    o_ref, l_ref = oracle.prefill_mla(q, k, v, scale, causal=causal)
    qd, kd, vd = (to_torch_bf16(x, cuda) for x in (q, k, v))
    out, lse = _fg().flash_gqa_forward_bshd(qd, kd, vd, scale, causal=causal, kernel=kernel)
    assert out.shape == (B, Sq, Hq, dv)
    _check(from_torch_bf16(out), lse.cpu().numpy(), o_ref, l_ref, what)


def test_padded_equal_dims_match_the_gqa_oracle(cuda):
    """D = 64 against the GQA oracle itself (fgqa_oracle_prefill_bf16), and
    against the (128, 128) kernels on inputs zero-padded by hand: bit-identical."""
    import torch
    fg = _fg()
    print("D=64 vs gqa oracle and hand-padded 128", flush=True)
    B, S, Hq, Hkv = 1, 520, 16, 1
    scale = 0.125
    q, k, v = _inputs(3100, B, S, S, Hq, Hkv, 64, 64)
    o_ref, l_ref = oracle.prefill(q, k, v, scale, causal=True)
    qd, kd, vd = (to_torch_bf16(x, cuda) for x in (q, k, v))
    out, lse = fg.flash_gqa_forward_bshd(qd, kd, vd, scale, causal=True)
    _check(from_torch_bf16(out), lse.cpu().numpy(), o_ref, l_ref, "D=64 gqa oracle")
    pad = lambda t: torch.nn.functional.pad(t, (0, 64)).contiguous()  # noqa: E731
    o128, l128 = fg.flash_gqa_forward_bshd(pad(qd), pad(kd), pad(vd), scale, causal=True)
    torch.cuda.synchronize()
    assert torch.equal(o128[..., :64].contiguous().view(torch.int16), out.view(torch.int16))
    assert torch.equal(l128, lse)
    assert not bool(o128[..., 64:].any())


@pytest.mark.parametrize("D", [64, 256, 200])
def test_padded_window_and_sink(cuda, D):
    """The sliding-window form with a sink at D = 64 (on the 128 kernels),
    256 (the 256 whole-range kernel, V in two launches) and 200."""
    import torch
    fg = _fg()
    print(f"D={D} window+sink", flush=True)
    B, S, Hq, Hkv, W = 1, 700, 8, 2, 96
    scale = 1.0 / math.sqrt(D)
    q, k, v = _inputs(3200 + D, B, S, S, Hq, Hkv, D, D)
    sink = np.random.default_rng(5).random(Hq, dtype=np.float32) + 1e-6
    o_ref, l_ref = oracle.prefill_swa(q, k, v, scale, W, sink)
    qd, kd, vd = (to_torch_bf16(x, cuda) for x in (q, k, v))
    out, lse = fg.flash_gqa_forward_bshd(qd, kd, vd, scale, causal=True, window_size=W,
                                         sink=torch.from_numpy(sink).to(cuda))
    _check(from_torch_bf16(out), lse.cpu().numpy(), o_ref, l_ref, f"D={D} window+sink")


def test_padded_strided_unaligned_tensors(cuda):
    """D = 100 (200-byte rows, so no row after the first is 16-byte aligned),
    Q and K views with a head stride wider than the row, O written into a
    strided view: the copies read and write element by element."""
    import torch
    fg = _fg()
    print("D=100 strided views", flush=True)
    B, S, Hq, Hkv, D = 1, 150, 4, 2, 100
    scale = 0.1
    q, k, v = _inputs(3300, B, S, S, Hq, Hkv, D, D)
    o_ref, l_ref = oracle.prefill(q, k, v, scale, causal=True)
    qd, kd, vd = (to_torch_bf16(x, cuda) for x in (q, k, v))
    qw = torch.zeros((B, S, Hq, D + 3), dtype=torch.bfloat16, device=cuda)
    qw[..., :D] = qd
    kw = torch.zeros((B, S, Hkv, D + 5), dtype=torch.bfloat16, device=cuda)
    kw[..., :D] = kd
    ow = torch.full((B, S, Hq, D + 7), 7.0, dtype=torch.bfloat16, device=cuda)
    out, lse = fg.flash_gqa_forward_bshd(qw[..., :D], kw[..., :D], vd, scale, causal=True, out=ow[..., :D])
    torch.cuda.synchronize()
    _check(from_torch_bf16(out), lse.cpu().numpy(), o_ref, l_ref, "D=100 strided")
    assert bool((ow[..., D:] == 7.0).all()), "columns past D of the output view were written"


def test_padded_config4_shape_every_kernel(cuda):
    """BASELINE config 4's shape (B=1, S=4096, Hq=16, Hkv=1, causal) at D = 64:
    the wide kernel's split pairs on the copies; rows sampled against the oracle."""
    import torch
    from tests._helpers import gpu_normal_bf16
    fg = _fg()
    B, S, Hq, Hkv, D = 1, 4096, 16, 1, 64
    scale = 1.0 / 8
    q = gpu_normal_bf16((B, S, Hq, D), 81, 1.0, cuda)
    k = gpu_normal_bf16((B, S, Hkv, D), 82, 1.0, cuda)
    v = gpu_normal_bf16((B, S, Hkv, D), 83, 1.0, cuda)
    assert fg.prefill_kernel_name(q, k, v, causal=True) == "prefill_wide_kernel"
    # (the calls share this stream's cached workspace: a call whose kernel
    # merges nothing must leave its counter prefix zero for the merging calls
    # after it)
    for kern in ("auto", "split", "tall", "auto"):
        print(f"D=64 config 4 shape kernel={kern}", flush=True)
        out, lse = fg.flash_gqa_forward_bshd(q, k, v, scale, causal=True, kernel=kern)
        torch.cuda.synchronize()
        for r0, r1 in ((0, 64), (1000, 1064), (S - 64, S)):
            o_ref, l_ref = oracle.prefill(from_torch_bf16(q[:, r0:r1]), from_torch_bf16(k[:, :r1]),
                                          from_torch_bf16(v[:, :r1]), scale, causal=True, q_offset=r0)
            _check(from_torch_bf16(out[:, r0:r1]), lse[:, :, r0:r1].cpu().numpy(), o_ref, l_ref,
                   f"D=64 config 4 kernel={kern} rows {r0}:{r1}")


def test_padded_library_workspace_and_caller_workspace(cuda):
    """The C ABI with no workspace (the library's cached buffer for the
    copies, its per-device merge scratch) and with a caller workspace of
    fgqa_prefill_workspace_bytes: the same bits; a workspace one byte short
    is refused."""
    import torch
    import cuda_llm_ops_amd._lib as L
    fg = _fg()
    from cuda_llm_ops_amd import flash_gqa as impl
    print("D=64 workspaces", flush=True)
    B, S, Hq, Hkv, D = 1, 4096, 16, 1, 64
    q, k, v = _inputs(3400, B, S, S, Hq, Hkv, D, D)
    qd, kd, vd = (to_torch_bf16(x, cuda) for x in (q, k, v))
    outs = []
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for mode in ("none", "caller", "short"):
        out = torch.empty((B, S, Hq, D), dtype=torch.bfloat16, device=cuda)
        lse = torch.empty((B, Hq, S), dtype=torch.float32, device=cuda)
        a = impl._prefill_args(qd, kd, vd, out, lse, 0.125, True, "bshd")
        n = ctypes.c_size_t(0)
        assert L.lib().fgqa_prefill_workspace_bytes(ctypes.byref(a), ctypes.byref(n)) == 0
        assert n.value >= 2 * (B * S * Hq + B * S * Hkv) * 128 * 2
        ws = None
        if mode != "none":
            ws = torch.zeros(n.value - (1 if mode == "short" else 0), dtype=torch.uint8, device=cuda)
            a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
        st = L.lib().fgqa_prefill_bf16(ctypes.byref(a), s)
        if mode == "short":
            assert st == L.FGQA_ERR_WORKSPACE
            continue
        assert st == 0
        torch.cuda.synchronize()
        outs.append((out, lse))
    assert torch.equal(outs[0][0].view(torch.int16), outs[1][0].view(torch.int16))
    assert torch.equal(outs[0][1], outs[1][1])
    o_ref, l_ref = oracle.prefill(q[:, -64:], k, v, 0.125, causal=True, q_offset=S - 64)
    _check(from_torch_bf16(outs[0][0][:, -64:]), outs[0][1][:, :, -64:].cpu().numpy(), o_ref, l_ref,
           "D=64 library workspace, last rows")
    del fg


def test_padded_reference_mirror_bhsd(cuda):
    """launch_flash_gqa_forward_bf16_kernel (the reference launcher's
    signature, BHSD, 3-D and 4-D) at D = 64 with its default 1/sqrt(D) scale."""
    import torch
    fg = _fg()
    print("D=64 bhsd mirror", flush=True)
    B, S, Hq, Hkv, D = 2, 200, 4, 2, 64
    q, k, v = _inputs(3500, B, S, S, Hq, Hkv, D, D)
    o_ref, l_ref = oracle.prefill(q, k, v, 1.0 / math.sqrt(D), causal=True)
    t = lambda x: to_torch_bf16(np.ascontiguousarray(x.transpose(0, 2, 1, 3)), cuda)  # noqa: E731
    out, lse = fg.launch_flash_gqa_forward_bf16_kernel(t(q), t(k), t(v))
    torch.cuda.synchronize()
    _check(from_torch_bf16(out.transpose(1, 2)), lse.cpu().numpy(), o_ref, l_ref, "D=64 bhsd 4-D")
    out3, lse3 = fg.launch_flash_gqa_forward_bf16_kernel(t(q)[0], t(k)[0], t(v)[0])
    torch.cuda.synchronize()
    assert torch.equal(out3.view(torch.int16), out[0].view(torch.int16))
    assert torch.equal(lse3, lse[0])
