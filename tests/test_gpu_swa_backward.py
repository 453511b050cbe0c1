"""GPU parity tests of the sliding-window (+ sink) prefill backward against the
CPU oracle.

The oracle (oracle/fgqa_oracle.c fgqa_oracle_prefill_swa_backward_bf16)
restates src/python/Triton/SWA/flash_swa_backward_kernel.py:157-321: the
causal backward restricted to keys [i - window + 1, i], driven by the forward's
sink-adjusted LSE.  Inputs come from the SWA forward oracle (O, LSE with the
sink), so the GPU and the oracle see the same O and LSE.  Bar: the backward's
relative 2e-2 / 2e-3 (tests/_helpers.py assert_grad_close).
"""
import ctypes
import math

import numpy as np
import pytest

import oracle
from tests._helpers import assert_grad_close, from_torch_bf16, gpu_normal_bf16, to_torch_bf16

pytestmark = pytest.mark.gpu

SCALE = 1.0 / math.sqrt(128)


def _fg():
    import cuda_llm_ops_amd as fg
    return fg


def _sync():
    import torch
    torch.cuda.synchronize()


def _sink(seed, Hq, with_sink):
    if not with_sink:
        return None
    return np.random.default_rng(seed).random(Hq).astype(np.float32) * 4 + 1e-6


def _inputs(seed, B, Sq, Skv, Hq, Hkv, window, with_sink=True, scale=SCALE):
    q = oracle.normal_bf16(seed, (B, Sq, Hq, 128))
    k = oracle.normal_bf16(seed, (B, Skv, Hkv, 128), stream=1)
    v = oracle.normal_bf16(seed, (B, Skv, Hkv, 128), stream=2)
    do = oracle.normal_bf16(seed, (B, Sq, Hq, 128), stream=3)
    sink = _sink(seed, Hq, with_sink)
    o, lse = oracle.prefill_swa(q, k, v, scale, window, sink)
    return q, k, v, o, lse, do


def _check(grads, refs, what):
    for name, g, r in zip(("dq", "dk", "dv"), grads, refs):
        ref = oracle.bf16_to_f32(oracle.f32_to_bf16(r))
        assert_grad_close(oracle.bf16_to_f32(g), ref, f"{what} {name}")


def _gpu_backward(cuda, q, k, v, o, lse, do, window, scale=SCALE, **plan):
    import torch
    t = [to_torch_bf16(x, cuda) for x in (q, k, v, o, do)]
    lsed = torch.from_numpy(np.ascontiguousarray(lse)).to(cuda)
    dq, dk, dv = _fg().flash_gqa_backward_bshd(t[0], t[1], t[2], t[3], lsed, t[4], scale, causal=True,
                                               window_size=window, **plan)
    _sync()
    return from_torch_bf16(dq), from_torch_bf16(dk), from_torch_bf16(dv)


@pytest.mark.parametrize("B,S,Hq,Hkv,window,with_sink", [
    (1, 300, 16, 1, 64, True),     # G=16, window = one key tile
    (2, 500, 8, 2, 17, True),      # window not a multiple of any tile
    (1, 400, 6, 3, 1, True),       # each row sees itself only
    (1, 257, 4, 4, 100, False),    # no sink: plain windowed softmax
    (1, 700, 4, 1, 4096, True),    # window past the sequence: causal + sink
    (1, 640, 2, 1, 200, True),     # several key blocks fully outside a row block's window
])
def test_swa_backward_shapes(cuda, B, S, Hq, Hkv, window, with_sink):
    what = f"swa backward B{B} S{S} Hq{Hq} Hkv{Hkv} W{window} sink={with_sink}"
    print(what, flush=True)
    q, k, v, o, lse, do = _inputs(1300 + S + window, B, S, S, Hq, Hkv, window, with_sink)
    refs = oracle.prefill_backward(q, k, v, o, lse, do, SCALE, causal=True, window=window)
    _check(_gpu_backward(cuda, q, k, v, o, lse, do, window), refs, what)


@pytest.mark.parametrize("scale", [-0.07, 0.0])
def test_swa_backward_scale_values(cuda, scale):
    """The window's two mask edges with a negative scale (S masked by +inf) and
    with scale 0 (the dK/dV kernel's select form)."""
    what = f"swa backward scale={scale}"
    print(what, flush=True)
    q, k, v, o, lse, do = _inputs(1500, 1, 300, 300, 8, 2, 40, True, scale=scale)
    refs = oracle.prefill_backward(q, k, v, o, lse, do, scale, causal=True, window=40)
    _check(_gpu_backward(cuda, q, k, v, o, lse, do, 40, scale=scale), refs, what)


@pytest.mark.parametrize("B,Sq,Skv,Hq,Hkv,window", [
    (1, 161, 97, 4, 1, 40),        # Sq > Skv: rows past the last key's window get zero dQ
    (2, 64, 640, 16, 4, 48),       # Sq < Skv: keys >= Sq get zero dK / dV
])
def test_swa_backward_unequal_lengths(cuda, B, Sq, Skv, Hq, Hkv, window):
    what = f"swa backward B{B} Sq{Sq} Skv{Skv} Hq{Hq} Hkv{Hkv} W{window}"
    print(what, flush=True)
    q, k, v, o, lse, do = _inputs(1400 + Sq, B, Sq, Skv, Hq, Hkv, window)
    refs = oracle.prefill_backward(q, k, v, o, lse, do, SCALE, causal=True, window=window)
    grads = _gpu_backward(cuda, q, k, v, o, lse, do, window)
    _check(grads, refs, what)
    if Sq > Skv:
        assert np.all(oracle.bf16_to_f32(grads[0])[:, Skv - 1 + window:] == 0)
    else:
        assert np.all(oracle.bf16_to_f32(grads[1])[:, Sq:] == 0)
        assert np.all(oracle.bf16_to_f32(grads[2])[:, Sq:] == 0)


@pytest.mark.parametrize("hsplit", [1, 2, 8])
def test_swa_backward_head_split_modes(cuda, hsplit):
    """Heads of a KV group in one workgroup or split over workgroups."""
    print(f"swa backward hsplit={hsplit}", flush=True)
    q, k, v, o, lse, do = _inputs(1510, 1, 384, 384, 16, 2, 96)
    refs = oracle.prefill_backward(q, k, v, o, lse, do, SCALE, causal=True, window=96)
    _check(_gpu_backward(cuda, q, k, v, o, lse, do, 96, kv_head_split=hsplit), refs, f"swa hsplit={hsplit}")


@pytest.mark.parametrize("split", ["whole", "split"])
@pytest.mark.parametrize("B,S,Hq,Hkv,window", [
    (1, 320, 16, 1, 70), (2, 200, 4, 2, 33), (1, 64, 3, 1, 5), (1, 600, 2, 1, 300)])
def test_swa_backward_dq_whole_and_split_kernels(cuda, split, B, S, Hq, Hkv, window):
    """The dQ kernel over a unit's windowed key range, whole or split over two
    wave groups."""
    what = f"swa dq kernel={split} B{B} S{S} Hq{Hq} Hkv{Hkv} W{window}"
    print(what, flush=True)
    q, k, v, o, lse, do = _inputs(1560 + S + window, B, S, S, Hq, Hkv, window)
    refs = oracle.prefill_backward(q, k, v, o, lse, do, SCALE, causal=True, window=window)
    _check(_gpu_backward(cuda, q, k, v, o, lse, do, window, dq_kernel=split), refs, what)


def test_swa_backward_window_past_sequence_equals_causal_without_sink(cuda):
    """A window at least the sequence length and no sink is the causal backward
    (bit for bit, with the same work split: the plans differ by default)."""
    print("swa backward == causal backward", flush=True)
    q, k, v, o, lse, do = _inputs(1600, 1, 256, 256, 8, 2, 256, with_sink=False)
    plan = dict(kv_head_split=2, dq_kernel="split")
    g_w = _gpu_backward(cuda, q, k, v, o, lse, do, 256, **plan)
    g_c = _gpu_backward(cuda, q, k, v, o, lse, do, 0, **plan)
    for a, b in zip(g_w, g_c):
        assert np.array_equal(a, b)


def test_swa_backward_forward_chain_reference_mirror(cuda):
    """The reference's call sequence (test_flash_swa_kernel.py:520-570): the
    SWA forward mirror's O and LSE into the SWA backward mirror, BHSD, 4-D
    and 3-D."""
    import torch
    fg = _fg()
    print("swa backward mirror chain", flush=True)
    B, S, Hq, Hkv, W = 2, 200, 8, 2, 48
    q = oracle.normal_bf16(1610, (B, S, Hq, 128))
    k = oracle.normal_bf16(1610, (B, S, Hkv, 128), stream=1)
    v = oracle.normal_bf16(1610, (B, S, Hkv, 128), stream=2)
    do = oracle.normal_bf16(1610, (B, S, Hq, 128), stream=3)
    sink = np.linspace(0.1, 3.0, Hq).astype(np.float32)
    t = lambda x: to_torch_bf16(np.ascontiguousarray(x.transpose(0, 2, 1, 3)), cuda)  # noqa: E731
    back = lambda x: from_torch_bf16(x).transpose(0, 2, 1, 3)  # noqa: E731
    sd = torch.from_numpy(sink).to(cuda)
    qd, kd, vd, dod = t(q), t(k), t(v), t(do)
    out, lse = fg.launch_flash_swa_forward_bf16_kernel(qd, kd, vd, window_size=W, sink_value=sd)
    dq, dk, dv = fg.launch_flash_swa_backward_bf16_kernel(qd, kd, vd, out, lse, dod, window_size=W)
    _sync()
    o_np = back(out)
    lse_np = lse.cpu().numpy()
    refs = oracle.prefill_backward(q, k, v, o_np, lse_np, do, SCALE, causal=True, window=W)
    _check((back(dq), back(dk), back(dv)), refs, "swa mirror 4-D")
    dq3, dk3, dv3 = fg.launch_flash_swa_backward_bf16_kernel(qd[1], kd[1], vd[1], out[1], lse[1], dod[1],
                                                             window_size=W)
    _sync()
    assert dq3.shape == (Hq, S, 128) and dk3.shape == (Hkv, S, 128)
    back3 = lambda x: from_torch_bf16(x)[None].transpose(0, 2, 1, 3)  # noqa: E731
    _check((back3(dq3), back3(dk3), back3(dv3)), tuple(r[1:] for r in refs), "swa mirror 3-D")


def test_swa_backward_reference_shape_full_size(cuda):
    """The reference's SWA benchmark shape (test_flash_swa_kernel.py:26-36:
    B=1, S=4096, Hq=16, Hkv=1, W=512, sink U[0,1)), N(0,1) inputs: GPU forward
    then backward; sampled rows / keys against the oracle, plus two identities
    over every key with p_i = sink_h * exp(-lse_i) the sink's share of row i:
    sum_j dV_j = sum_i (1 - p_i) dO_i and sum_j dK_j = scale * sum_i p_i delta_i q_i
    (delta_i = O_i . dO_i)."""
    import torch
    fg = _fg()
    print("swa backward reference shape", flush=True)
    B, S, Hq, Hkv, W = 1, 4096, 16, 1, 512
    q = gpu_normal_bf16((B, S, Hq, 128), 51, 1.0, cuda)
    k = gpu_normal_bf16((B, S, Hkv, 128), 52, 1.0, cuda)
    v = gpu_normal_bf16((B, S, Hkv, 128), 53, 1.0, cuda)
    do = gpu_normal_bf16((B, S, Hq, 128), 54, 1.0, cuda)
    sink = torch.rand(Hq, generator=torch.Generator().manual_seed(65)).to(cuda) + 1e-6
    out, lse = fg.flash_gqa_forward_bshd(q, k, v, SCALE, causal=True, window_size=W, sink=sink)
    dq, dk, dv = fg.flash_gqa_backward_bshd(q, k, v, out, lse, do, SCALE, causal=True, window_size=W)
    _sync()
    for g in (dq, dk, dv):
        assert bool(g.isfinite().all())
    h = [from_torch_bf16(x) for x in (q, k, v, out, do)]
    lse_np = lse.cpu().numpy()
    gq, gk, gv = (from_torch_bf16(x) for x in (dq, dk, dv))
    for rows in ((0, 64), (1000, 1064), (S - 64, S)):
        rq, _, _ = oracle.prefill_backward(*h[:4], lse_np, h[4], SCALE, causal=True, rows=rows, want=("dq",),
                                           window=W)
        assert_grad_close(oracle.bf16_to_f32(gq[:, rows[0]:rows[1]]),
                          oracle.bf16_to_f32(oracle.f32_to_bf16(rq[:, rows[0]:rows[1]])), f"swa dq rows {rows}")
    for keys in ((0, 8), (2000, 2008), (S - 64, S)):
        _, rk, rv = oracle.prefill_backward(*h[:4], lse_np, h[4], SCALE, causal=True, keys=keys,
                                            want=("dk", "dv"), window=W)
        for name, g, r in (("dk", gk, rk), ("dv", gv, rv)):
            assert_grad_close(oracle.bf16_to_f32(g[:, keys[0]:keys[1]]),
                              oracle.bf16_to_f32(oracle.f32_to_bf16(r[:, keys[0]:keys[1]])),
                              f"swa {name} keys {keys}")
    # identities over every key
    p = sink.double()[None, :, None] * torch.exp(-lse.double())          # [B, Hq, S]
    p = p.transpose(1, 2)                                                # [B, S, Hq]
    dod, od, qd = do.double(), out.double(), q.double()
    dv_sum = dv.double().sum(1)[:, 0]                                    # [B, D]
    dv_expect = ((1 - p)[..., None] * dod).sum(dim=(1, 2))
    assert float((dv_sum - dv_expect).abs().max()) < 2e-3 * float(dv_expect.abs().max())
    delta = (od * dod).sum(-1)                                           # [B, S, Hq]
    dk_expect = SCALE * ((p * delta)[..., None] * qd).sum(dim=(1, 2))
    dk_sum = dk.double().sum(1)[:, 0]
    assert float((dk_sum - dk_expect).abs().max()) < 5e-3 * float(dk.double().abs().sum(1).mean())


def test_swa_backward_caller_workspace(cuda):
    """A caller workspace sized for the window (at most the causal size; one
    byte short is rejected), and the gradients it gives."""
    import torch
    fg = _fg()
    print("swa backward caller workspace", flush=True)
    B, S, Hq, Hkv, W = 1, 384, 16, 1, 96
    q, k, v, o, lse, do = _inputs(1660, B, S, S, Hq, Hkv, W)
    refs = oracle.prefill_backward(q, k, v, o, lse, do, SCALE, causal=True, window=W)
    n_w = fg.backward_workspace_bytes(B, S, S, Hq, Hkv, window_size=W)
    n_c = fg.backward_workspace_bytes(B, S, S, Hq, Hkv)
    assert 0 < n_w <= n_c
    qd, kd, vd, od, dod = (to_torch_bf16(x, cuda) for x in (q, k, v, o, do))
    lsed = torch.from_numpy(lse).to(cuda)
    small = torch.empty(n_w - 1, dtype=torch.uint8, device=cuda)
    with pytest.raises(fg.FgqaError):
        fg.flash_gqa_backward_bshd(qd, kd, vd, od, lsed, dod, SCALE, workspace=small, window_size=W)
    ws = torch.empty(n_w, dtype=torch.uint8, device=cuda)
    g = fg.flash_gqa_backward_bshd(qd, kd, vd, od, lsed, dod, SCALE, workspace=ws, window_size=W)
    _sync()
    _check(tuple(from_torch_bf16(x) for x in g), refs, "swa caller workspace")


def test_swa_backward_cplusplus_dropin(cuda):
    """LaunchFlashSwaBackwardBf16Kernel (BSHD, default stream)."""
    import torch
    fg = _fg()
    L = fg.lib()
    print("swa backward C++ entry point", flush=True)
    B, S, Hq, Hkv, W = 1, 192, 4, 1, 40
    q, k, v, o, lse, do = _inputs(1650, B, S, S, Hq, Hkv, W)
    refs = oracle.prefill_backward(q, k, v, o, lse, do, SCALE, causal=True, window=W)
    qd, kd, vd, od, dod = (to_torch_bf16(x, cuda) for x in (q, k, v, o, do))
    lsed = torch.from_numpy(lse).to(cuda)
    gq, gk, gv = torch.zeros_like(qd), torch.zeros_like(kd), torch.zeros_like(vd)
    fn = getattr(L, "_Z32LaunchFlashSwaBackwardBf16KernelPK6bf16_tS1_S1_S1_PKfS1_fPS_S4_S4_iiiiiii")
    fn.restype = None
    torch.cuda.synchronize()
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    fn(p(qd), p(kd), p(vd), p(od), p(lsed), p(dod), ctypes.c_float(SCALE), p(gq), p(gk), p(gv),
       B, S, S, Hq, Hkv, 128, W)
    st = getattr(L, "_Z21FlashGqaGetLastStatusv")
    st.restype = ctypes.c_int
    assert st() == 0
    torch.cuda.synchronize()
    _check((from_torch_bf16(gq), from_torch_bf16(gk), from_torch_bf16(gv)), refs, "C++ swa backward")
