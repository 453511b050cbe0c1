"""GPU parity tests of the prefill backward (dQ, dK, dV) against the CPU oracle.

Bar: bf16 gradients within 2e-2 of the oracle's elementwise, relative to
max(1, |ref|), and mean error within 2e-3 relative to max(1, mean |ref|) --
the forward's 2e-2 / 2e-3 taken relative, since gradients exceed 1 in
magnitude where a single bf16 ulp is already above 2e-2 (tests/_helpers.py).
The oracle restates src/python/Triton/flash_gqa_backward_kernel.py and is fed
the same O and LSE as the GPU.  Full-size configurations are checked on sampled
query rows and keys plus size-independent properties.
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


def _inputs(seed, B, Sq, Skv, Hq, Hkv, scale=SCALE, causal=True, sigma=1.0):
    q = oracle.normal_bf16(seed, (B, Sq, Hq, 128), sigma)
    k = oracle.normal_bf16(seed, (B, Skv, Hkv, 128), sigma, stream=1)
    v = oracle.normal_bf16(seed, (B, Skv, Hkv, 128), sigma, stream=2)
    do = oracle.normal_bf16(seed, (B, Sq, Hq, 128), 1.0, stream=3)
    o, lse = oracle.prefill(q, k, v, scale, causal=causal)
    return q, k, v, o, lse, do


def _check(grads, refs, what):
    for name, g, r in zip(("dq", "dk", "dv"), grads, refs):
        ref = oracle.bf16_to_f32(oracle.f32_to_bf16(r))
        assert_grad_close(oracle.bf16_to_f32(g), ref, f"{what} {name}")


def _gpu_backward(cuda, q, k, v, o, lse, do, scale=SCALE, causal=True, workspace=None, **plan):
    import torch
    t = [to_torch_bf16(x, cuda) for x in (q, k, v, o)]
    dod = to_torch_bf16(do, cuda)
    lsed = torch.from_numpy(np.ascontiguousarray(lse)).to(cuda)
    dq, dk, dv = _fg().flash_gqa_backward_bshd(t[0], t[1], t[2], t[3], lsed, dod, scale, causal=causal,
                                               workspace=workspace, **plan)
    _sync()
    return from_torch_bf16(dq), from_torch_bf16(dk), from_torch_bf16(dv)


@pytest.mark.parametrize("B,Sq,Skv,Hq,Hkv,causal", [
    (1, 256, 256, 16, 1, True),     # G=16 (config 4's grouping)
    (2, 300, 300, 8, 2, True),      # G=4, ragged query and key tails
    (1, 200, 200, 6, 3, True),      # G=2
    (1, 130, 130, 3, 3, True),      # G=1
    (1, 1, 1, 4, 1, True),          # one row, one key
    (1, 97, 161, 4, 2, False),      # non-causal, Sq != Skv
    (1, 161, 97, 4, 1, True),       # causal, Sq > Skv
    (2, 64, 640, 16, 4, True),      # causal, Sq < Skv: keys >= Sq get zero gradients
    (1, 33, 33, 2, 1, False),
])
def test_backward_shapes(cuda, B, Sq, Skv, Hq, Hkv, causal):
    what = f"backward B{B} Sq{Sq} Skv{Skv} Hq{Hq} Hkv{Hkv} causal{causal}"
    print(what, flush=True)
    q, k, v, o, lse, do = _inputs(700 + Sq, B, Sq, Skv, Hq, Hkv, causal=causal)
    refs = oracle.prefill_backward(q, k, v, o, lse, do, SCALE, causal=causal)
    grads = _gpu_backward(cuda, q, k, v, o, lse, do, causal=causal)
    _check(grads, refs, what)
    if causal and Skv > Sq:
        assert np.all(oracle.bf16_to_f32(grads[1])[:, Sq:] == 0)
        assert np.all(oracle.bf16_to_f32(grads[2])[:, Sq:] == 0)


@pytest.mark.parametrize("hsplit", [1, 2, 8])
def test_backward_head_split_modes(cuda, hsplit):
    """Heads of a KV group in one workgroup (dK/dV written from registers) or
    split over workgroups (fp32 dK/dV accumulators) give the same gradients."""
    print(f"backward hsplit={hsplit}", flush=True)
    q, k, v, o, lse, do = _inputs(810, 1, 384, 384, 16, 2)
    refs = oracle.prefill_backward(q, k, v, o, lse, do, SCALE, causal=True)
    _check(_gpu_backward(cuda, q, k, v, o, lse, do, kv_head_split=hsplit), refs, f"hsplit={hsplit}")


@pytest.mark.parametrize("split", ["whole", "split"])
@pytest.mark.parametrize("B,Sq,Skv,Hq,Hkv,causal", [
    (1, 320, 320, 16, 1, True), (2, 200, 200, 4, 2, True), (1, 130, 250, 2, 1, False), (1, 64, 64, 3, 1, True)])
def test_backward_dq_whole_and_split_kernels(cuda, split, B, Sq, Skv, Hq, Hkv, causal):
    """The dQ kernel over a unit's whole key range, or split over two wave
    groups whose dQ is summed through LDS."""
    what = f"dq kernel={split} B{B} Sq{Sq} Skv{Skv} Hq{Hq} Hkv{Hkv} causal{causal}"
    print(what, flush=True)
    q, k, v, o, lse, do = _inputs(860 + Sq, B, Sq, Skv, Hq, Hkv, causal=causal)
    refs = oracle.prefill_backward(q, k, v, o, lse, do, SCALE, causal=causal)
    _check(_gpu_backward(cuda, q, k, v, o, lse, do, causal=causal, dq_kernel=split), refs, what)


@pytest.mark.parametrize("Skv", [64, 128, 192, 320, 448, 704, 832])
def test_backward_dq_split_tile_counts(cuda, Skv):
    """The split dQ kernel's two groups cycle three K buffers and two V
    buffers over their half of the key range: non-causal rows over 1 to 13
    key tiles give each group 1 to 7 tiles (every position of the cycle,
    and a second half that is partly or wholly past the keys)."""
    what = f"dq split tile counts Skv={Skv}"
    print(what, flush=True)
    q, k, v, o, lse, do = _inputs(1700 + Skv, 1, 128, Skv, 4, 1, causal=False)
    refs = oracle.prefill_backward(q, k, v, o, lse, do, SCALE, causal=False)
    _check(_gpu_backward(cuda, q, k, v, o, lse, do, causal=False, dq_kernel="split"), refs, what)


# a negative scale masks S with +inf (S * scale is then -inf); a zero scale
# runs the dK/dV kernel's select form of the mask
@pytest.mark.parametrize("scale", [0.2, -0.05, 0.0])
def test_backward_scale_values(cuda, scale):
    print(f"backward scale={scale}", flush=True)
    q, k, v, o, lse, do = _inputs(820, 1, 200, 200, 4, 1, scale=scale)
    refs = oracle.prefill_backward(q, k, v, o, lse, do, scale, causal=True)
    _check(_gpu_backward(cuda, q, k, v, o, lse, do, scale=scale), refs, f"scale={scale}")


def test_backward_reference_mirror_bhsd(cuda):
    """launch_flash_gqa_backward_bf16_kernel with the reference's BHSD tensors,
    4-D and 3-D (flash_gqa_backward_kernel.py:312-478)."""
    import torch
    fg = _fg()
    print("backward mirror bhsd", flush=True)
    q, k, v, o, lse, do = _inputs(830, 2, 160, 160, 8, 2)
    refs = oracle.prefill_backward(q, k, v, o, lse, do, SCALE, causal=True)
    t = lambda x: to_torch_bf16(np.ascontiguousarray(x.transpose(0, 2, 1, 3)), cuda)  # noqa: E731
    lsed = torch.from_numpy(lse).to(cuda)
    dq, dk, dv = fg.launch_flash_gqa_backward_bf16_kernel(t(q), t(k), t(v), t(o), lsed, t(do))
    _sync()
    back = lambda x: from_torch_bf16(x).transpose(0, 2, 1, 3)  # noqa: E731
    _check((back(dq), back(dk), back(dv)), refs, "mirror 4-D")
    # 3-D (unbatched) tensors of batch 1
    dq3, dk3, dv3 = fg.launch_flash_gqa_backward_bf16_kernel(t(q)[1], t(k)[1], t(v)[1], t(o)[1], lsed[1],
                                                             t(do)[1])
    _sync()
    assert dq3.shape == (8, 160, 128) and dk3.shape == (2, 160, 128)
    # fp32 atomics sum in no fixed order (as the reference's atomic_add,
    # flash_gqa_backward_kernel.py:293-310), so equal up to rounding, not bits
    r1 = tuple(r[1:] for r in refs)
    back3 = lambda x: from_torch_bf16(x)[None].transpose(0, 2, 1, 3)  # noqa: E731
    _check((back3(dq3), back3(dk3), back3(dv3)), r1, "mirror 3-D")


def test_backward_caller_workspace_and_forward_chain(cuda):
    """Caller workspace (too small -> error), and the backward of the GPU
    forward's own O and LSE."""
    import torch
    fg = _fg()
    print("backward workspace + forward chain", flush=True)
    B, S, Hq, Hkv = 1, 256, 8, 1
    q, k, v, _, _, do = _inputs(840, B, S, S, Hq, Hkv)
    qd, kd, vd, dod = (to_torch_bf16(x, cuda) for x in (q, k, v, do))
    out, lse = fg.flash_gqa_forward_bshd(qd, kd, vd, SCALE)
    n = fg.backward_workspace_bytes(B, S, S, Hq, Hkv)
    small = torch.empty(n - 256, dtype=torch.uint8, device=cuda)
    with pytest.raises(fg.FgqaError):
        fg.flash_gqa_backward_bshd(qd, kd, vd, out, lse, dod, SCALE, workspace=small)
    ws = torch.empty(n, dtype=torch.uint8, device=cuda)
    dq, dk, dv = fg.flash_gqa_backward_bshd(qd, kd, vd, out, lse, dod, SCALE, workspace=ws)
    _sync()
    o_np, lse_np = from_torch_bf16(out), lse.cpu().numpy()
    refs = oracle.prefill_backward(q, k, v, o_np, lse_np, do, SCALE, causal=True)
    _check((from_torch_bf16(dq), from_torch_bf16(dk), from_torch_bf16(dv)), refs, "forward chain")
    # a prepared launch repeats the same work
    pl = fg.prepare_backward(qd, kd, vd, out, lse, dod, SCALE, workspace=ws)
    g2 = pl()
    _sync()
    _check(tuple(from_torch_bf16(x) for x in g2), refs, "prepared launch")


def test_backward_config4_full_size(cuda):
    """BASELINE config 4 shape (B=1, S=4096, Hq=16, Hkv=1, causal, N(0,1)):
    forward then backward on the GPU; sampled rows / keys against the oracle,
    plus sum_j dK_j ~ 0 and sum_j dV_j ~ sum dO over all keys."""
    import torch
    fg = _fg()
    print("backward config4 full size", flush=True)
    B, S, Hq, Hkv = 1, 4096, 16, 1
    q = gpu_normal_bf16((B, S, Hq, 128), 41, 1.0, cuda)
    k = gpu_normal_bf16((B, S, Hkv, 128), 42, 1.0, cuda)
    v = gpu_normal_bf16((B, S, Hkv, 128), 43, 1.0, cuda)
    do = gpu_normal_bf16((B, S, Hq, 128), 44, 1.0, cuda)
    out, lse = fg.flash_gqa_forward_bshd(q, k, v, SCALE)
    dq, dk, dv = fg.flash_gqa_backward_bshd(q, k, v, out, lse, do, SCALE)
    _sync()
    for g in (dq, dk, dv):
        assert bool(g.isfinite().all())
    h = [from_torch_bf16(x) for x in (q, k, v, out, do)]
    lse_np = lse.cpu().numpy()
    gq, gk, gv = (from_torch_bf16(x) for x in (dq, dk, dv))
    for rows in ((0, 64), (S - 64, S)):
        rq, _, _ = oracle.prefill_backward(*h[:4], lse_np, h[4], SCALE, causal=True, rows=rows, want=("dq",))
        assert_grad_close(oracle.bf16_to_f32(gq[:, rows[0]:rows[1]]),
                          oracle.bf16_to_f32(oracle.f32_to_bf16(rq[:, rows[0]:rows[1]])), f"config4 dq rows {rows}")
    for keys in ((0, 8), (2000, 2008), (S - 64, S)):
        _, rk, rv = oracle.prefill_backward(*h[:4], lse_np, h[4], SCALE, causal=True, keys=keys,
                                            want=("dk", "dv"))
        for name, g, r in (("dk", gk, rk), ("dv", gv, rv)):
            assert_grad_close(oracle.bf16_to_f32(g[:, keys[0]:keys[1]]),
                              oracle.bf16_to_f32(oracle.f32_to_bf16(r[:, keys[0]:keys[1]])),
                              f"config4 {name} keys {keys}")
    # size-independent properties over every key
    sk = dk.double().sum(1)
    assert float(sk.abs().max()) < 5e-3 * float(dk.double().abs().sum(1).mean())
    dosum = do.double().sum(dim=(1, 2), keepdim=False)
    err = (dv.double().sum(1)[:, 0] - dosum).abs().max()
    assert float(err) < 2e-3 * float(dosum.abs().max())



def test_backward_cplusplus_dropin(cuda):
    """LaunchFlashGqaBackwardBf16Kernel (BSHD, default stream)."""
    import torch
    fg = _fg()
    L = fg.lib()
    print("backward C++ entry point", flush=True)
    B, S, Hq, Hkv = 1, 192, 4, 1
    q, k, v, o, lse, do = _inputs(850, B, S, S, Hq, Hkv)
    refs = oracle.prefill_backward(q, k, v, o, lse, do, SCALE, causal=True)
    qd, kd, vd, od, dod = (to_torch_bf16(x, cuda) for x in (q, k, v, o, do))
    lsed = torch.from_numpy(lse).to(cuda)
    gq, gk, gv = torch.zeros_like(qd), torch.zeros_like(kd), torch.zeros_like(vd)
    fn = getattr(L, "_Z32LaunchFlashGqaBackwardBf16KernelPK6bf16_tS1_S1_S1_PKfS1_fPS_S4_S4_iiiiiib")
    fn.restype = None
    torch.cuda.synchronize()
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    fn(p(qd), p(kd), p(vd), p(od), p(lsed), p(dod), ctypes.c_float(SCALE), p(gq), p(gk), p(gv),
       B, S, S, Hq, Hkv, 128, ctypes.c_bool(True))
    st = getattr(L, "_Z21FlashGqaGetLastStatusv")
    st.restype = ctypes.c_int
    assert st() == 0
    torch.cuda.synchronize()
    _check((from_torch_bf16(gq), from_torch_bf16(gk), from_torch_bf16(gv)), refs, "C++ backward")


_NO_QUERY_ROWS_SCRIPT = r"""
import ctypes, sys
sys.path.insert(0, sys.argv[1])
import torch
import cuda_llm_ops_amd._lib as L
dev = torch.device("cuda:0")
B, Skv, H, D = 2, 200, 3, 128
k = torch.randn(B, Skv, H, D, device=dev).to(torch.bfloat16)
v = torch.randn(B, Skv, H, D, device=dev).to(torch.bfloat16)
dk = torch.full((B, Skv, H, D), float("nan"), device=dev, dtype=torch.bfloat16)
dv = torch.full((B, Skv, H, D), float("nan"), device=dev, dtype=torch.bfloat16)
a = L.BackwardArgs()
a.k, a.v, a.grad_k, a.grad_v = k.data_ptr(), v.data_ptr(), dk.data_ptr(), dv.data_ptr()
a.batch, a.seqlen_q, a.seqlen_kv, a.num_q_heads, a.num_kv_heads, a.head_dim = B, 0, Skv, H, H, D
a.causal, a.scale = 1, D ** -0.5
for name in ("q_stride", "o_stride", "grad_o_stride", "grad_q_stride"):
    getattr(a, name)[:] = [H * D, H * D, D]
for name in ("k_stride", "v_stride", "grad_k_stride", "grad_v_stride"):
    getattr(a, name)[:] = [Skv * H * D, H * D, D]
n = ctypes.c_size_t(1)
assert L.lib().fgqa_prefill_backward_workspace_bytes(ctypes.byref(a), ctypes.byref(n)) == 0 and n.value == 0
st = L.lib().fgqa_prefill_backward_bf16(ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
torch.cuda.synchronize()
assert st == 0, st
assert bool((dk == 0).all()) and bool((dv == 0).all()), "dK / dV not zeroed"
print("no-query-rows backward ok", flush=True)
"""


@pytest.mark.parametrize("split", ["whole", "split"])
def test_backward_without_keys_zeroes_dq(cuda, split):
    """Sq > 0 with Skv = 0: no dQ unit has a key tile, so each writes dQ = 0
    (and still stores its rows' statistics; no dK/dV kernel runs to read
    them), for both dQ kernels."""
    import torch
    print(f"backward Sq=100 Skv=0 dq={split}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(77)
    q = torch.randn(1, 100, 4, 128, generator=g).to(torch.bfloat16).to(cuda)
    o = torch.randn(1, 100, 4, 128, generator=g).to(torch.bfloat16).to(cuda)
    do = torch.randn(1, 100, 4, 128, generator=g).to(torch.bfloat16).to(cuda)
    k = torch.empty(1, 0, 1, 128, dtype=torch.bfloat16, device=cuda)
    v = torch.empty_like(k)
    lse = torch.zeros(1, 4, 100, device=cuda)
    dq, dk, dv = _fg().flash_gqa_backward_bshd(q, k, v, o, lse, do, SCALE, causal=False, dq_kernel=split)
    _sync()
    assert dk.shape == (1, 0, 1, 128) and dv.shape == (1, 0, 1, 128)
    assert torch.count_nonzero(dq.float()).item() == 0


def test_backward_without_query_rows_zeroes_key_gradients(cuda):
    """Sq = 0 with Skv > 0 and G = 1: the call needs no workspace, and no query
    row sees any key, so dK = dV = 0 must still be written -- in a fresh process,
    where the library's own buffer has never been allocated (q, o, lse, grad_o
    and grad_q are NULL: nothing reads them)."""
    import os
    import subprocess
    import sys
    print("backward Sq=0 Skv=200 G=1 (fresh process)", flush=True)
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _NO_QUERY_ROWS_SCRIPT, root], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "no-query-rows backward ok" in r.stdout
