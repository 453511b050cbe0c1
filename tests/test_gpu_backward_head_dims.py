"""GPU tests of the prefill backward at head dims the kernels are not built for.

The reference's Triton backward pads its head-dim blocks to a power of two
(src/python/Triton/flash_gqa_backward_kernel.py:312-478 passes
BLOCK_DMODEL = next_power_of_2(head_dim)); this library runs Q/K head dims up
to 128 (or 192) with V/O head dims up to 128 on copies of Q, K, V, O and dO
zero-padded to the built (128, 128) or (192, 128) and copies the first
columns of dQ, dK and dV back.  The oracle (oracle/fgqa_oracle.c
fgqa_oracle_prefill_backward_bf16 and _mla_backward_bf16) takes the head dims
as they are.  Bar: the gradients within 2e-2 of max(1, |ref|) per element
and 2e-3 on average (tests/_helpers.py assert_grad_close).
"""
import math

import numpy as np
import pytest

import oracle
from tests._helpers import assert_grad_close, from_torch_bf16, to_torch_bf16

pytestmark = pytest.mark.gpu


def _fg():
    import cuda_llm_ops_amd as fg
    return fg


def _inputs(seed, B, Sq, Skv, Hq, Hkv, dqk, dv, scale, causal=True):
    q = oracle.normal_bf16(seed, (B, Sq, Hq, dqk))
    k = oracle.normal_bf16(seed, (B, Skv, Hkv, dqk), stream=1)
    v = oracle.normal_bf16(seed, (B, Skv, Hkv, dv), stream=2)
    do = oracle.normal_bf16(seed, (B, Sq, Hq, dv), stream=3)
    o, lse = oracle.prefill_mla(q, k, v, scale, causal=causal)
    return q, k, v, o, lse, do


def _check(grads, refs, what):
    for name, g, r in zip(("dq", "dk", "dv"), grads, refs):
        ref = oracle.bf16_to_f32(oracle.f32_to_bf16(r))
        assert_grad_close(oracle.bf16_to_f32(g), ref, f"{what} {name}")


@pytest.mark.parametrize("dqk,dv", [(64, 64), (32, 32), (100, 100), (64, 128), (128, 64), (72, 40), (192, 64),
                                    (8, 8)])
@pytest.mark.parametrize("B,Sq,Skv,Hq,Hkv,causal", [
    (1, 256, 256, 16, 1, True),
    (2, 200, 330, 4, 2, False),
    (1, 161, 97, 6, 3, True),
])
def test_backward_padded_head_dims(cuda, dqk, dv, B, Sq, Skv, Hq, Hkv, causal):
    import torch
    what = f"backward D=({dqk},{dv}) B{B} Sq{Sq} Skv{Skv} Hq{Hq} Hkv{Hkv} causal={causal}"
    print(what, flush=True)
    scale = 1.0 / math.sqrt(dqk)
    q, k, v, o, lse, do = _inputs(4000 + dqk + dv + Sq, B, Sq, Skv, Hq, Hkv, dqk, dv, scale, causal)
    refs = oracle.prefill_backward(q, k, v, o, lse, do, scale, causal=causal)
    t = [to_torch_bf16(x, cuda) for x in (q, k, v, o, do)]
    lsed = torch.from_numpy(np.ascontiguousarray(lse)).to(cuda)
    grads = _fg().flash_gqa_backward_bshd(t[0], t[1], t[2], t[3], lsed, t[4], scale, causal=causal)
    torch.cuda.synchronize()
    assert grads[0].shape == q.shape and grads[1].shape == k.shape and grads[2].shape == v.shape
    _check([from_torch_bf16(g) for g in grads], refs, what)


def test_backward_padded_matches_hand_padded_128(cuda):
    """D = 64 against the (128, 128) kernels on inputs zero-padded by hand:
    bit-identical gradients, zero in the padded columns; the window form too."""
    import torch
    fg = _fg()
    print("backward D=64 vs hand-padded 128", flush=True)
    B, S, Hq, Hkv, D = 1, 520, 16, 1, 64
    scale = 0.125
    q, k, v, o, lse, do = _inputs(4100, B, S, S, Hq, Hkv, D, D, scale)
    t = [to_torch_bf16(x, cuda) for x in (q, k, v, o, do)]
    lsed = torch.from_numpy(np.ascontiguousarray(lse)).to(cuda)
    pad = lambda x: torch.nn.functional.pad(x, (0, 128 - D)).contiguous()  # noqa: E731
    for window in (0, 100):
        g = fg.flash_gqa_backward_bshd(t[0], t[1], t[2], t[3], lsed, t[4], scale, causal=True, window_size=window)
        g128 = fg.flash_gqa_backward_bshd(*(pad(x) for x in t[:4]), lsed, pad(t[4]), scale, causal=True,
                                          window_size=window)
        torch.cuda.synchronize()
        for a, b in zip(g, g128):
            assert torch.equal(b[..., :D].contiguous().view(torch.int16), a.view(torch.int16)), f"window {window}"
            assert not bool(b[..., D:].any())
    refs = oracle.prefill_backward(q, k, v, o, lse, do, scale, causal=True, window=100)
    _check([from_torch_bf16(x) for x in g], refs, "backward D=64 window 100")


def test_backward_padded_config4_shape_and_workspaces(cuda):
    """Config 4's shape (B=1, S=4096, Hq=16, Hkv=1, causal) at D = 64: the
    16-way head split and its reduce on the copies, sampled rows and keys
    against the oracle; the library's buffer and a caller workspace of
    backward_workspace_bytes give the same bits, and one byte short is refused."""
    import ctypes
    import torch
    import cuda_llm_ops_amd._lib as L
    from cuda_llm_ops_amd import flash_gqa as impl
    from tests._helpers import gpu_normal_bf16
    fg = _fg()
    print("backward D=64 config 4 shape", flush=True)
    B, S, Hq, Hkv, D = 1, 4096, 16, 1, 64
    scale = 0.125
    q = gpu_normal_bf16((B, S, Hq, D), 91, 1.0, cuda)
    k = gpu_normal_bf16((B, S, Hkv, D), 92, 1.0, cuda)
    v = gpu_normal_bf16((B, S, Hkv, D), 93, 1.0, cuda)
    do = gpu_normal_bf16((B, S, Hq, D), 94, 1.0, cuda)
    o, lse = fg.flash_gqa_forward_bshd(q, k, v, scale, causal=True)
    n = fg.backward_workspace_bytes(B, S, S, Hq, Hkv, head_dim=D)
    assert n >= (2 * B * S * Hq + B * S * Hkv) * 128 * 2 * 2
    ws = torch.empty(n, dtype=torch.uint8, device=cuda)
    g_caller = fg.flash_gqa_backward_bshd(q, k, v, o, lse, do, scale, causal=True, workspace=ws)
    g_lib = fg.flash_gqa_backward_bshd(q, k, v, o, lse, do, scale, causal=True)
    torch.cuda.synchronize()
    for a, b in zip(g_caller, g_lib):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    grads = [from_torch_bf16(x) for x in g_caller]
    h = [from_torch_bf16(x) for x in (q, k, v, o, do)]
    lse_h = lse.cpu().numpy()
    rows, keys = (S - 64, S), (0, 64)
    refs = oracle.prefill_backward(h[0], h[1], h[2], h[3], lse_h, h[4], scale, causal=True, rows=rows, keys=keys)
    assert_grad_close(oracle.bf16_to_f32(grads[0][:, rows[0]:rows[1]]),
                      oracle.bf16_to_f32(oracle.f32_to_bf16(refs[0][:, rows[0]:rows[1]])), "config 4 D=64 dq")
    for name, g, r in zip(("dk", "dv"), grads[1:], refs[1:]):
        assert_grad_close(oracle.bf16_to_f32(g[:, keys[0]:keys[1]]),
                          oracle.bf16_to_f32(oracle.f32_to_bf16(r[:, keys[0]:keys[1]])), f"config 4 D=64 {name}")
    gq, gk, gv = (torch.empty_like(x) for x in (q, k, v))
    a = impl._backward_args(q, k, v, o, lse, do, gq, gk, gv, scale, True, "bshd", ws)
    a.workspace_bytes = n - 1
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert L.lib().fgqa_prefill_backward_bf16(ctypes.byref(a), s) == L.FGQA_ERR_WORKSPACE
