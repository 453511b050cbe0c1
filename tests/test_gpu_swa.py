"""GPU tests of the sliding-window (+ sink) prefill against the CPU oracle.

The oracle (oracle/fgqa_oracle.c fgqa_oracle_prefill_swa_bf16) restates the
reference's torch SWA reference, examples/python/Triton/test_flash_swa_kernel.py:97-116.
Bar: max-abs 2e-2 and mean-abs 2e-3 on bf16 outputs, LSE within 1e-3.
"""
import math

import numpy as np
import pytest

import oracle
from tests._helpers import assert_close, from_torch_bf16, gpu_normal_bf16, to_torch_bf16

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


def _case(cuda, seed, B, Sq, Skv, Hq, Hkv, window, with_sink, kernel="auto"):
    import torch
    q = oracle.normal_bf16(seed, (B, Sq, Hq, 128))
    k = oracle.normal_bf16(seed, (B, Skv, Hkv, 128), stream=1)
    v = oracle.normal_bf16(seed, (B, Skv, Hkv, 128), stream=2)
    sink = (np.random.default_rng(seed).random(Hq).astype(np.float32) * 4 + 1e-6) if with_sink else None
    o_ref, l_ref = oracle.prefill_swa(q, k, v, SCALE, window, sink)
    qd, kd, vd = (to_torch_bf16(x, cuda) for x in (q, k, v))
    sd = None if sink is None else torch.from_numpy(sink).to(cuda)
    out, lse = _fg().flash_gqa_forward_bshd(qd, kd, vd, SCALE, causal=True, window_size=window, sink=sd,
                                            kernel=kernel)
    torch.cuda.synchronize()
    return from_torch_bf16(out), lse.cpu().numpy(), o_ref, l_ref


@pytest.mark.parametrize("kernel", ["auto", "whole", "wide"])
@pytest.mark.parametrize("B,S,Hq,Hkv,window,with_sink", [
    (1, 300, 16, 1, 64, True),
    (2, 500, 8, 2, 17, True),     # window not a multiple of the tile
    (1, 400, 6, 3, 1, True),      # each row sees itself only
    (1, 257, 4, 4, 100, False),   # no sink: plain windowed softmax
    (1, 700, 4, 1, 4096, True),   # window past the sequence: causal + sink
    (1, 2048, 16, 1, 300, True),  # wide kernel: early units shorter, their pairs split
    (1, 1500, 8, 1, 1000, True),
])
def test_swa_shapes(cuda, kernel, B, S, Hq, Hkv, window, with_sink):
    what = f"swa kernel={kernel} B{B} S{S} Hq{Hq} Hkv{Hkv} W{window} sink={with_sink}"
    print(what, flush=True)
    _check(*_case(cuda, 1000 + S + window, B, S, S, Hq, Hkv, window, with_sink, kernel), what)


@pytest.mark.parametrize("window", [0, 2048])
def test_swa_long_window_and_sink_only_config4_shape(cuda, window):
    """Config 4's shape (B=1, S=4096, Hq=16, Hkv=1) with a sink and no window,
    and with a 2048-key window: AUTO runs the 256-row kernel there; its rows
    (first, middle, last blocks) and the whole-range kernel's match the
    oracle (a window of S keys stands for none)."""
    import torch
    fg = _fg()
    B, S, Hq, Hkv = 1, 4096, 16, 1
    q = gpu_normal_bf16((B, S, Hq, 128), 61, 1.0, cuda)
    k = gpu_normal_bf16((B, S, Hkv, 128), 62, 1.0, cuda)
    v = gpu_normal_bf16((B, S, Hkv, 128), 63, 1.0, cuda)
    sink = np.random.default_rng(7).random(Hq).astype(np.float32) * 4 + 1e-6
    sd = torch.from_numpy(sink).to(cuda)
    if torch.cuda.get_device_properties(cuda).multi_processor_count == 256:
        assert fg.prefill_kernel_choice(q, k, v, window_size=window, sink=sd) == "wide"
    h = [from_torch_bf16(x) for x in (q, k, v)]
    for kern in ("auto", "whole"):
        print(f"swa config 4 shape window={window} kernel={kern}", flush=True)
        out, lse = fg.flash_gqa_forward_bshd(q, k, v, SCALE, causal=True, window_size=window, sink=sd, kernel=kern)
        torch.cuda.synchronize()
        for r0, r1 in ((0, 64), (2000, 2064), (S - 64, S)):
            o_ref, l_ref = oracle.prefill_swa(h[0][:, r0:r1], h[1][:, :r1], h[2][:, :r1], SCALE, window or S, sink,
                                              q_offset=r0)
            _check(from_torch_bf16(out[:, r0:r1]), lse[:, :, r0:r1].cpu().numpy(), o_ref, l_ref,
                   f"swa window={window} kernel={kern} rows {r0}:{r1}")


def test_swa_split_kernel_request_is_unsupported(cuda):
    """The window / sink variant has no split form: asking for it is an error
    (FGQA_ERR_UNSUPPORTED), not a silent fallback."""
    import torch
    fg = _fg()
    q = torch.zeros((1, 64, 4, 128), device=cuda, dtype=torch.bfloat16)
    k = torch.zeros((1, 64, 1, 128), device=cuda, dtype=torch.bfloat16)
    with pytest.raises(fg.FgqaError) as e:
        fg.flash_gqa_forward_bshd(q, k, k, SCALE, causal=True, window_size=16, kernel="split")
    assert e.value.status == -2


def test_swa_rows_past_the_keys(cuda):
    """Sq > Skv: rows past the last key's window see nothing (O = 0, lse = log(max(sink, 1e-9)))."""
    print("swa Sq > Skv", flush=True)
    o, lse, o_ref, l_ref = _case(cuda, 1100, 1, 200, 90, 4, 1, 32, True)
    _check(o, lse, o_ref, l_ref, "swa Sq > Skv")
    assert np.all(oracle.bf16_to_f32(o)[:, 90 + 31:] == 0)


def test_swa_reference_mirror_bhsd(cuda):
    """launch_flash_swa_forward_bf16_kernel with the reference's BHSD tensors, 4-D and 3-D."""
    import torch
    fg = _fg()
    print("swa mirror", flush=True)
    B, S, Hq, Hkv, W = 2, 260, 8, 2, 48
    q = oracle.normal_bf16(1200, (B, S, Hq, 128))
    k = oracle.normal_bf16(1200, (B, S, Hkv, 128), stream=1)
    v = oracle.normal_bf16(1200, (B, S, Hkv, 128), stream=2)
    sink = np.linspace(0.1, 3.0, Hq).astype(np.float32)
    o_ref, l_ref = oracle.prefill_swa(q, k, v, SCALE, W, sink)
    t = lambda x: to_torch_bf16(np.ascontiguousarray(x.transpose(0, 2, 1, 3)), cuda)  # noqa: E731
    sd = torch.from_numpy(sink).to(cuda)
    out, lse = fg.launch_flash_swa_forward_bf16_kernel(t(q), t(k), t(v), window_size=W, sink_value=sd)
    torch.cuda.synchronize()
    _check(from_torch_bf16(out).transpose(0, 2, 1, 3), lse.cpu().numpy(), o_ref, l_ref, "swa mirror 4-D")
    o3, l3 = fg.launch_flash_swa_forward_bf16_kernel(t(q)[1], t(k)[1], t(v)[1], window_size=W, sink_value=sd)
    torch.cuda.synchronize()
    assert torch.equal(o3, out[1]) and torch.equal(l3, lse[1])
    with pytest.raises(ValueError, match="window_size must be provided"):
        fg.launch_flash_swa_forward_bf16_kernel(t(q), t(k), t(v), sink_value=sd)
    with pytest.raises(ValueError, match="elements"):
        fg.launch_flash_swa_forward_bf16_kernel(t(q), t(k), t(v), window_size=W, sink_value=sd[:3])


def test_swa_reference_shape_full_size(cuda):
    """The reference's SWA benchmark shape (B=1, S=4096, Hq=16, Hkv=1, window 512,
    sink U[0,1)), N(0,1) inputs: sampled row blocks against the oracle."""
    import torch
    fg = _fg()
    print("swa full size", flush=True)
    B, S, Hq, Hkv, W = 1, 4096, 16, 1, 512
    q = gpu_normal_bf16((B, S, Hq, 128), 61, 1.0, cuda)
    k = gpu_normal_bf16((B, S, Hkv, 128), 62, 1.0, cuda)
    v = gpu_normal_bf16((B, S, Hkv, 128), 63, 1.0, cuda)
    sink = torch.rand(Hq, generator=torch.Generator().manual_seed(64)).to(cuda) + 1e-6
    out, lse = fg.flash_gqa_forward_bshd(q, k, v, SCALE, causal=True, window_size=W, sink=sink)
    torch.cuda.synchronize()
    assert bool(out.isfinite().all())
    sk = sink.cpu().numpy()
    for r0, r1 in ((0, 64), (1500, 1564), (S - 64, S)):
        k0 = max(0, r0 - W + 1)
        o_ref, l_ref = oracle.prefill_swa(from_torch_bf16(q[:, r0:r1]), from_torch_bf16(k[:, k0:r1]),
                                          from_torch_bf16(v[:, k0:r1]), SCALE, W, sk, q_offset=r0 - k0)
        _check(from_torch_bf16(out[:, r0:r1]), lse[:, :, r0:r1].cpu().numpy(), o_ref, l_ref,
               f"swa full size rows {r0}:{r1}")


def test_swa_cplusplus_entry(cuda):
    """LaunchFlashSwaForwardBf16Kernel (BSHD, default stream)."""
    import ctypes

    import torch
    fg = _fg()
    L = fg.lib()
    print("swa C++ entry", flush=True)
    B, S, Hq, Hkv, W = 1, 320, 8, 1, 40
    q = oracle.normal_bf16(1300, (B, S, Hq, 128))
    k = oracle.normal_bf16(1300, (B, S, Hkv, 128), stream=1)
    v = oracle.normal_bf16(1300, (B, S, Hkv, 128), stream=2)
    sink = np.linspace(0.5, 2.0, Hq).astype(np.float32)
    o_ref, l_ref = oracle.prefill_swa(q, k, v, SCALE, W, sink)
    qd, kd, vd = (to_torch_bf16(x, cuda) for x in (q, k, v))
    sd = torch.from_numpy(sink).to(cuda)
    od = torch.zeros_like(qd)
    ld = torch.zeros((B, Hq, S), dtype=torch.float32, device=cuda)
    fn = getattr(L, "_Z31LaunchFlashSwaForwardBf16KernelPK6bf16_tS1_S1_fPS_PfiiiiiiiPKf")
    fn.restype = None
    st = getattr(L, "_Z21FlashGqaGetLastStatusv")
    st.restype = ctypes.c_int
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    torch.cuda.synchronize()
    fn(p(qd), p(kd), p(vd), ctypes.c_float(SCALE), p(od), p(ld), B, S, S, Hq, Hkv, 128, W, p(sd))
    assert st() == 0
    torch.cuda.synchronize()
    _check(from_torch_bf16(od), ld.cpu().numpy(), o_ref, l_ref, "C++ SWA")
    fn(p(qd), p(kd), p(vd), ctypes.c_float(SCALE), p(od), p(ld), B, S, S, Hq, Hkv, 128, 0, p(sd))
    assert st() == -1
