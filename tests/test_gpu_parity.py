"""GPU parity tests: the HIP path (through the C ABI) against the CPU oracle.

Bar (stated for this path): bf16 outputs within max-abs 2e-2 and mean-abs 2e-3
of the oracle on the same seeded inputs.  LSE outputs within 1e-3 absolute.
Full-size configurations are checked on sampled batches / rows (the oracle
would take minutes on all of them) plus size-independent properties.
"""
import ctypes
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


def _sync():
    import torch
    torch.cuda.synchronize()


# ------------------------------------------------------------------ decode
def _decode_case(cuda, seed, B, Hq, Hkv, S, seqlens=None, split_tokens=0, nan_pad=False, workspace=False):
    import torch
    q = oracle.normal_bf16(seed, (B, Hq, 128))
    k = oracle.normal_bf16(seed, (B, S, Hkv, 128), stream=1)
    v = oracle.normal_bf16(seed, (B, S, Hkv, 128), stream=2)
    if nan_pad and seqlens is not None:
        for b, n in enumerate(seqlens):
            k[b, n:] = 0x7FC0
            v[b, n:] = 0x7FC0
    o_ref, lse_ref = oracle.decode(q, k, v, SCALE, seqlens=seqlens)
    qd, kd, vd = (to_torch_bf16(x, cuda) for x in (q, k, v))
    sl = None if seqlens is None else torch.tensor(seqlens, dtype=torch.int32, device=cuda)
    lse = torch.empty((B, Hq), dtype=torch.float32, device=cuda)
    ws = None
    if workspace:
        n = _fg().decode_workspace_bytes(B, S, Hq, Hkv, split_tokens=split_tokens, ragged=seqlens is not None)
        ws = torch.empty(max(n, 16), dtype=torch.uint8, device=cuda)
    out = _fg().decode_flash_gqa_bshd(qd, kd, vd, SCALE, seqlens=sl, lse=lse, split_tokens=split_tokens,
                                      workspace=ws)
    _sync()
    return from_torch_bf16(out), lse.cpu().numpy(), o_ref, lse_ref


def _check_decode(o, lse, o_ref, lse_ref, what):
    assert_close(oracle.bf16_to_f32(o), oracle.bf16_to_f32(o_ref), what)
    fin = np.isfinite(lse_ref)
    assert np.array_equal(np.isfinite(lse), fin), f"{what}: lse finiteness"
    assert np.max(np.abs(lse[fin] - lse_ref[fin]), initial=0.0) <= LSE_TOL, f"{what}: lse"


def test_decode_config1(cuda):
    """B=2, Hq=16, Hkv=2 (G=8), S=512, N(0,1)."""
    for split in (0, 128, 512):
        o, lse, o_ref, lse_ref = _decode_case(cuda, 101, 2, 16, 2, 512, split_tokens=split)
        _check_decode(o, lse, o_ref, lse_ref, f"config1 split={split}")


@pytest.mark.parametrize("G", [1, 2, 4, 8, 16])
def test_decode_group_sizes_and_tail(cuda, G):
    o, lse, o_ref, lse_ref = _decode_case(cuda, 200 + G, 3, 2 * G, 2, 1000)
    _check_decode(o, lse, o_ref, lse_ref, f"G={G} S=1000")


def test_decode_split_invariance_and_workspace(cuda):
    outs = []
    for split, ws in ((128, False), (256, True), (1024, False), (4096, True)):
        o, lse, o_ref, lse_ref = _decode_case(cuda, 300, 2, 32, 2, 4096, split_tokens=split, workspace=ws)
        _check_decode(o, lse, o_ref, lse_ref, f"split={split}")
        outs.append(oracle.bf16_to_f32(o))
    for x in outs[1:]:
        assert_close(x, outs[0], "split invariance", max_abs=8e-3)


def test_decode_ragged_nan_padding(cuda):
    sl = [0, 1, 2, 31, 32, 127, 128, 129, 500, 1024, 2047, 2048]
    o, lse, o_ref, lse_ref = _decode_case(cuda, 400, len(sl), 16, 2, 2048, seqlens=sl, nan_pad=True)
    assert np.all(np.isfinite(oracle.bf16_to_f32(o)))
    _check_decode(o, lse, o_ref, lse_ref, "ragged with NaN padding")
    assert np.all(oracle.bf16_to_f32(o[0]) == 0) and np.all(np.isneginf(lse[0]))
    # single split: the pass-1 kernel writes the output itself
    o, lse, o_ref, lse_ref = _decode_case(cuda, 401, len(sl), 16, 2, 2048, seqlens=sl, nan_pad=True,
                                          split_tokens=4096)
    _check_decode(o, lse, o_ref, lse_ref, "ragged, one split")
    # caller workspace, several split lengths of the ragged work list
    for split in (128, 384, 1024):
        o, lse, o_ref, lse_ref = _decode_case(cuda, 402 + split, len(sl), 16, 2, 2048, seqlens=sl, nan_pad=True,
                                              split_tokens=split, workspace=True)
        _check_decode(o, lse, o_ref, lse_ref, f"ragged, split {split}, caller workspace")
        assert np.all(oracle.bf16_to_f32(o[0]) == 0) and np.all(np.isneginf(lse[0]))


@pytest.mark.parametrize("Hkv", [1, 3, 4])
def test_decode_ragged_kv_head_counts(cuda, Hkv):
    """The ragged work list with odd kv head counts (one head per workgroup)
    and an even one (two heads per 8-wave workgroup), one split and several."""
    sl = [0, 1, 129, 500, 2047, 2048, 700]
    for split in (4096, 256):
        what = f"ragged Hkv={Hkv} split={split}"
        print(what, flush=True)
        o, lse, o_ref, lse_ref = _decode_case(cuda, 420 + Hkv, len(sl), 4 * Hkv, Hkv, 2048, seqlens=sl,
                                              nan_pad=True, split_tokens=split)
        _check_decode(o, lse, o_ref, lse_ref, what)
        assert np.all(oracle.bf16_to_f32(o[0]) == 0) and np.all(np.isneginf(lse[0]))


def test_decode_known_answers(cuda):
    import torch
    B, Hq, Hkv, S = 2, 16, 1, 3000
    fg = _fg()
    k = gpu_normal_bf16((B, S, Hkv, 128), 5, 1.0, cuda)
    v = gpu_normal_bf16((B, S, Hkv, 128), 6, 1.0, cuda)
    # Q = 0: every logit equal -> O = mean(V), lse = log S
    q = torch.zeros((B, Hq, 128), dtype=torch.bfloat16, device=cuda)
    lse = torch.empty((B, Hq), dtype=torch.float32, device=cuda)
    out = fg.decode_flash_gqa_bshd(q, k, v, SCALE, lse=lse)
    _sync()
    vm = v.float().mean(dim=1)[:, 0, :].cpu().numpy()
    assert_close(out.float().cpu().numpy(), np.repeat(vm[:, None, :], Hq, axis=1), "Q=0 -> mean(V)", max_abs=4e-3)
    assert np.allclose(lse.cpu().numpy(), math.log(S), atol=1e-4)
    # one token -> V[0] exactly
    out = fg.decode_flash_gqa_bshd(gpu_normal_bf16((B, Hq, 128), 7, 1.0, cuda), k[:, :1], v[:, :1], SCALE)
    _sync()
    assert torch.equal(out, v[:, 0, 0:1, :].expand(B, Hq, 128))


def test_decode_config2_full_size(cuda):
    """BASELINE config 2 at full size (B=60, S=4096, Hq=128, Hkv=8): sampled batches vs oracle."""
    import torch
    B, S, Hq, Hkv = 60, 4096, 128, 8
    fg = _fg()
    q = gpu_normal_bf16((B, Hq, 128), 21, 1.0, cuda)
    k = gpu_normal_bf16((B, S, Hkv, 128), 22, 1.0, cuda)
    v = gpu_normal_bf16((B, S, Hkv, 128), 23, 1.0, cuda)
    lse = torch.empty((B, Hq), dtype=torch.float32, device=cuda)
    out = fg.decode_flash_gqa_bshd(q, k, v, SCALE, lse=lse)
    _sync()
    o_np = from_torch_bf16(out)
    assert np.all(np.isfinite(oracle.bf16_to_f32(o_np)))
    for b in (0, 31, 59):
        o_ref, lse_ref = oracle.decode(from_torch_bf16(q[b:b + 1]), from_torch_bf16(k[b:b + 1]),
                                       from_torch_bf16(v[b:b + 1]), SCALE)
        _check_decode(o_np[b:b + 1], lse[b:b + 1].cpu().numpy(), o_ref, lse_ref, f"config2 batch {b}")
    # the reference's C++ layout through the Triton-layout mirror gives the same bytes
    out2 = fg.launch_decode_flash_gqa_bf16_kernel(q[:, :, None, :].contiguous(),
                                                  k.permute(0, 2, 1, 3).contiguous(),
                                                  v.permute(0, 2, 1, 3).contiguous())
    _sync()
    assert torch.equal(out2[:, :, 0, :], out)
    # split-KV over kv head pairs (960 items, combine pass) on the same inputs
    for split in (1024, 2048):
        lse2 = torch.empty_like(lse)
        out3 = fg.decode_flash_gqa_bshd(q, k, v, SCALE, lse=lse2, split_tokens=split)
        _sync()
        o3 = from_torch_bf16(out3)
        for b in (0, 59):
            o_ref, lse_ref = oracle.decode(from_torch_bf16(q[b:b + 1]), from_torch_bf16(k[b:b + 1]),
                                           from_torch_bf16(v[b:b + 1]), SCALE)
            _check_decode(o3[b:b + 1], lse2[b:b + 1].cpu().numpy(), o_ref, lse_ref, f"config2 split {split} batch {b}")


def test_decode_config3_ragged_full_size(cuda):
    """B=64, len ~ U{1..32768}, Hq=64, Hkv=8, NaN padding; sampled batches vs oracle."""
    import torch
    B, Smax, Hq, Hkv = 64, 32768, 64, 8
    rng = np.random.default_rng(3)
    lens = (1 + rng.integers(0, 32768, size=B)).astype(np.int32)
    fg = _fg()
    q = gpu_normal_bf16((B, Hq, 128), 31, 1.0, cuda)
    k = gpu_normal_bf16((B, Smax, Hkv, 128), 32, 1.0, cuda)
    v = gpu_normal_bf16((B, Smax, Hkv, 128), 33, 1.0, cuda)
    nan = torch.tensor(float("nan"), dtype=torch.bfloat16, device=cuda)
    for b in range(B):
        k[b, int(lens[b]):] = nan
        v[b, int(lens[b]):] = nan
    sl = torch.from_numpy(lens).to(cuda)
    lse = torch.empty((B, Hq), dtype=torch.float32, device=cuda)
    out = fg.decode_flash_gqa_bshd(q, k, v, SCALE, seqlens=sl, lse=lse)
    _sync()
    o_np = from_torch_bf16(out)
    assert np.all(np.isfinite(oracle.bf16_to_f32(o_np)))
    picks = [int(np.argmin(lens)), int(np.argmax(lens)), 7, 40]
    for b in picks:
        n = int(lens[b])
        o_ref, lse_ref = oracle.decode(from_torch_bf16(q[b:b + 1]), from_torch_bf16(k[b:b + 1, :n]),
                                       from_torch_bf16(v[b:b + 1, :n]), SCALE)
        _check_decode(o_np[b:b + 1], lse[b:b + 1].cpu().numpy(), o_ref, lse_ref, f"config3 batch {b} len {n}")


def test_decode_cplusplus_dropin(cuda):
    """The reference-signature C++ entry point LaunchFlashGqaBf16Kernel (default
    stream), twice in a row at two shapes whose split plans differ: both match
    the oracle, and oIntermediate is left untouched (the partials live in the
    library's fixed device scratch, so the call allocates nothing)."""
    import torch
    fg = _fg()
    L = fg.lib()
    fn = getattr(L, "_Z24LaunchFlashGqaBf16KernelPK6bf16_tS1_S1_fPS_Pfiiiii")
    fn.restype = None
    st = getattr(L, "_Z21FlashGqaGetLastStatusv")
    st.restype = ctypes.c_int
    for seed, (B, S, Hq, Hkv) in ((500, (2, 512, 32, 2)), (501, (1, 8192, 16, 1))):
        need = fg.decode_workspace_bytes(B, S, Hq, Hkv)
        assert 0 < need <= 32 << 20, need
        q = oracle.normal_bf16(seed, (B, Hq, 128))
        k = oracle.normal_bf16(seed, (B, S, Hkv, 128), stream=1)
        v = oracle.normal_bf16(seed, (B, S, Hkv, 128), stream=2)
        o_ref, _ = oracle.decode(q, k, v, SCALE)
        qd, kd, vd = (to_torch_bf16(x, cuda) for x in (q, k, v))
        od = torch.zeros((B, Hq, 128), dtype=torch.bfloat16, device=cuda)
        oi = torch.full((B, Hq, 128), 7.0, dtype=torch.float32, device=cuda)
        torch.cuda.synchronize()
        fn(ctypes.c_void_p(qd.data_ptr()), ctypes.c_void_p(kd.data_ptr()), ctypes.c_void_p(vd.data_ptr()),
           ctypes.c_float(SCALE), ctypes.c_void_p(od.data_ptr()), ctypes.c_void_p(oi.data_ptr()),
           B, S, Hq, Hkv, 128)
        assert st() == 0
        torch.cuda.synchronize()
        assert_close(od.float().cpu().numpy(), oracle.bf16_to_f32(o_ref), f"C++ drop-in decode B={B} S={S}")
        assert bool((oi == 7.0).all().item()), "oIntermediate was written"
    # unsupported head_dim: silent no-op, status says why
    fn(ctypes.c_void_p(qd.data_ptr()), ctypes.c_void_p(kd.data_ptr()), ctypes.c_void_p(vd.data_ptr()),
       ctypes.c_float(SCALE), ctypes.c_void_p(od.data_ptr()), ctypes.c_void_p(oi.data_ptr()), B, S, Hq, Hkv, 64)
    assert st() == -2


# ------------------------------------------------------------------ prefill
def _prefill_case(cuda, seed, B, Sq, Skv, Hq, Hkv, causal=True, sigma=1.0, kernel="auto"):
    q = oracle.normal_bf16(seed, (B, Sq, Hq, 128), sigma)
    k = oracle.normal_bf16(seed, (B, Skv, Hkv, 128), sigma, stream=1)
    v = oracle.normal_bf16(seed, (B, Skv, Hkv, 128), sigma, stream=2)
    o_ref, lse_ref = oracle.prefill(q, k, v, SCALE, causal=causal)
    qd, kd, vd = (to_torch_bf16(x, cuda) for x in (q, k, v))
    out, lse = _fg().flash_gqa_forward_bshd(qd, kd, vd, SCALE, causal=causal, kernel=kernel)
    _sync()
    return from_torch_bf16(out), lse.cpu().numpy(), o_ref, lse_ref


def _check_prefill(o, lse, o_ref, lse_ref, what):
    assert_close(oracle.bf16_to_f32(o), oracle.bf16_to_f32(o_ref), what)
    fin = np.isfinite(lse_ref)
    assert np.array_equal(np.isfinite(lse), fin), f"{what}: lse finiteness"
    assert np.max(np.abs(lse[fin] - lse_ref[fin]), initial=0.0) <= LSE_TOL, f"{what}: lse"


@pytest.mark.parametrize("B,Sq,Skv,Hq,Hkv,causal", [
    (1, 256, 256, 16, 1, True),
    (2, 300, 300, 8, 2, True),      # G=4, ragged tail
    (1, 200, 200, 6, 3, True),      # G=2
    (1, 130, 130, 3, 3, True),      # G=1
    (1, 1, 1, 4, 1, True),
    (1, 97, 161, 4, 2, False),      # non-causal, Sq != Skv
    (1, 161, 97, 4, 1, True),       # causal, Sq > Skv
    (2, 64, 640, 16, 4, True),      # causal, Sq < Skv (top-left aligned)
])
def test_prefill_shapes(cuda, B, Sq, Skv, Hq, Hkv, causal):
    o, lse, o_ref, lse_ref = _prefill_case(cuda, 600 + Sq, B, Sq, Skv, Hq, Hkv, causal)
    _check_prefill(o, lse, o_ref, lse_ref, f"prefill B{B} Sq{Sq} Skv{Skv} Hq{Hq} Hkv{Hkv} causal{causal}")


@pytest.mark.parametrize("kernel", ["whole", "split", "wide", "tall"])
@pytest.mark.parametrize("B,Sq,Skv,Hq,Hkv,causal", [
    (1, 256, 256, 16, 1, True),
    (2, 300, 300, 8, 2, True),      # odd tile counts per unit
    (1, 130, 130, 3, 3, True),
    (1, 97, 161, 4, 2, False),
    (1, 161, 97, 4, 1, True),
    (2, 64, 640, 16, 4, True),
    (1, 1111, 1111, 16, 2, True),   # up to 18 tiles per unit
    (1, 700, 900, 4, 4, False),
    (1, 2048, 2048, 16, 1, True),   # 128 wide units of 8 heads: every pair but the lightest split
    (3, 1000, 1000, 8, 1, True),    # odd number of wide units (the middle one alone)
    (1, 1500, 1500, 4, 2, True),    # wide units of 4 heads x 64 positions
    (1, 900, 900, 2, 1, True),      # 2 heads x 128 positions
    (1, 1300, 1300, 1, 1, True),    # 1 head x 256 positions
    (16, 512, 512, 16, 1, True),    # 256 unit pairs: the wide kernel runs whole units, persistent
    (4, 600, 600, 8, 2, False),     # the same, non-causal
])
def test_prefill_whole_and_split_kernels(cuda, kernel, B, Sq, Skv, Hq, Hkv, causal):
    """The prefill kernels: one workgroup per unit over its whole KV range, the
    split kernel (two wave groups on the halves of the range, merged), the
    wide kernel (two wave groups on one tile, a unit's range split over two
    workgroups that merge through device memory), and the tall kernel (the
    wide kernel's units on four waves of 64 rows each)."""
    o, lse, o_ref, lse_ref = _prefill_case(cuda, 650 + Sq, B, Sq, Skv, Hq, Hkv, causal, kernel=kernel)
    _check_prefill(o, lse, o_ref, lse_ref,
                   f"kernel={kernel} B{B} Sq{Sq} Skv{Skv} Hq{Hq} Hkv{Hkv} causal{causal}")


@pytest.mark.parametrize("kernel", ["whole", "split", "wide", "tall"])
@pytest.mark.parametrize("case,scale", [("climb", 0.5), ("fall", 0.5), ("sharp", 2.0)])
def test_prefill_running_max_moves(cuda, kernel, case, scale):
    """Score distributions that move the running max: keys scaled up along the
    sequence (each row's max climbs from tile to tile by far more than the
    rescale slack, so both kernels rescale, and the split kernel's row-sum
    check fires), scaled down (the first tile holds the max), and logits in
    the hundreds (exp2 against a stale max would overflow fp32)."""
    B, S, Hq, Hkv = 1, 640, 8, 1
    what = f"running max {case} scale={scale} kernel={kernel}"
    print(what, flush=True)
    q = oracle.normal_bf16(900, (B, S, Hq, 128))
    k = oracle.bf16_to_f32(oracle.normal_bf16(900, (B, S, Hkv, 128), stream=1))
    v = oracle.normal_bf16(900, (B, S, Hkv, 128), stream=2)
    ramp = np.arange(S, dtype=np.float32) / S
    f = {"climb": 0.25 + 3.0 * ramp, "fall": 3.25 - 3.0 * ramp, "sharp": np.ones(S, np.float32)}[case]
    k = oracle.f32_to_bf16(k * f[None, :, None, None])
    o_ref, lse_ref = oracle.prefill(q, k, v, scale, causal=True)
    qd, kd, vd = (to_torch_bf16(x, cuda) for x in (q, k, v))
    out, lse = _fg().flash_gqa_forward_bshd(qd, kd, vd, scale, causal=True, kernel=kernel)
    _sync()
    o = from_torch_bf16(out)
    if case == "sharp":
        # Logits in the hundreds make each output one V value scaled by its
        # bf16 P; how the kernels round P against a running max that trails
        # the row max by up to 2^8 moves some outputs by one bf16 step, which
        # is 0.031 at |O| >= 4, above the 2e-2 bar: here the bar is
        # max(2e-2, one bf16 step of the expected value) per element.
        got, ref = oracle.bf16_to_f32(o), oracle.bf16_to_f32(o_ref)
        step = np.exp2(np.floor(np.log2(np.maximum(np.abs(ref), 1e-30))) - 7)
        assert np.all(np.abs(got - ref) <= np.maximum(2e-2, step)), what
        assert_close(got, ref, what, max_abs=np.inf)   # mean-abs bar unchanged
        fin = np.isfinite(lse_ref)
        assert np.array_equal(np.isfinite(lse.cpu().numpy()), fin)
        assert np.max(np.abs(lse.cpu().numpy()[fin] - lse_ref[fin]), initial=0.0) <= LSE_TOL
        return
    _check_prefill(o, lse.cpu().numpy(), o_ref, lse_ref, what)


@pytest.mark.parametrize("scale", [0.2, -0.05])
def test_scale_values(cuda, scale):
    """Non-default and negative softmax scales (the prefill kernel folds the
    sign into Q, the decode kernel into the exponent argument)."""
    import torch
    fg = _fg()
    B, S, Hq, Hkv = 2, 300, 8, 2
    q = oracle.normal_bf16(910, (B, S, Hq, 128))
    k = oracle.normal_bf16(910, (B, S, Hkv, 128), stream=1)
    v = oracle.normal_bf16(910, (B, S, Hkv, 128), stream=2)
    o_ref, lse_ref = oracle.prefill(q, k, v, scale, causal=True)
    qd, kd, vd = (to_torch_bf16(x, cuda) for x in (q, k, v))
    out, lse = fg.flash_gqa_forward_bshd(qd, kd, vd, scale, causal=True)
    _sync()
    _check_prefill(from_torch_bf16(out), lse.cpu().numpy(), o_ref, lse_ref, f"prefill scale {scale}")
    qdec = q[:, -1].copy()
    od_ref, ld_ref = oracle.decode(qdec, k, v, scale)
    ld = torch.empty((B, Hq), dtype=torch.float32, device=cuda)
    od = fg.decode_flash_gqa_bshd(to_torch_bf16(qdec, cuda), kd, vd, scale, lse=ld)
    _sync()
    _check_decode(from_torch_bf16(od), ld.cpu().numpy(), od_ref, ld_ref, f"decode scale {scale}")


def test_prefill_row0_and_triton_layout(cuda):
    import torch
    fg = _fg()
    B, S, Hq, Hkv = 2, 384, 8, 2
    q = oracle.normal_bf16(700, (B, Hq, S, 128))
    k = oracle.normal_bf16(700, (B, Hkv, S, 128), stream=1)
    v = oracle.normal_bf16(700, (B, Hkv, S, 128), stream=2)
    o_ref, lse_ref = oracle.prefill(q, k, v, SCALE, causal=True, layout="bhsd")
    qd, kd, vd = (to_torch_bf16(x, cuda) for x in (q, k, v))
    out, lse = fg.launch_flash_gqa_forward_bf16_kernel(qd, kd, vd)
    _sync()
    _check_prefill(from_torch_bf16(out), lse.cpu().numpy(), o_ref, lse_ref, "Triton-layout prefill")
    # causal row 0 sees key 0 only: O = V[0] exactly
    G = Hq // Hkv
    for h in range(Hq):
        assert torch.equal(out[:, h, 0], vd[:, h // G, 0])
    # 3-D unbatched form, provided out/lse written in place
    o3 = torch.empty_like(qd[0])
    l3 = torch.empty((Hq, S), dtype=torch.float32, device=cuda)
    r_o, r_l = fg.launch_flash_gqa_forward_bf16_kernel(qd[0], kd[0], vd[0], out=o3, lse=l3)
    _sync()
    assert r_o.data_ptr() == o3.data_ptr() and r_l.data_ptr() == l3.data_ptr()
    assert torch.equal(o3, out[0])


def test_prefill_decode_consistency(cuda):
    """Decode of the last token == last row of causal prefill (same K/V)."""
    import torch
    fg = _fg()
    S, Hq, Hkv = 1000, 16, 2
    q = gpu_normal_bf16((1, S, Hq, 128), 801, 1.0, cuda)
    k = gpu_normal_bf16((1, S, Hkv, 128), 802, 1.0, cuda)
    v = gpu_normal_bf16((1, S, Hkv, 128), 803, 1.0, cuda)
    out, lse = fg.flash_gqa_forward_bshd(q, k, v, SCALE)
    lse_d = torch.empty((1, Hq), dtype=torch.float32, device=cuda)
    od = fg.decode_flash_gqa_bshd(q[:, -1].contiguous(), k, v, SCALE, lse=lse_d)
    _sync()
    assert_close(od.float().cpu().numpy(), out[:, -1].float().cpu().numpy(), "decode vs prefill last row",
                 max_abs=8e-3)
    assert np.max(np.abs(lse_d.cpu().numpy() - lse[:, :, -1].cpu().numpy())) <= LSE_TOL


def _sampled_prefill_check(q, k, v, out, lse, rows, b, what):
    """Oracle on rows `rows` (a contiguous range) of batch b via q_offset."""
    r0, r1 = rows
    o_ref, lse_ref = oracle.prefill(from_torch_bf16(q[b:b + 1, r0:r1]), from_torch_bf16(k[b:b + 1, :r1]),
                                    from_torch_bf16(v[b:b + 1, :r1]), SCALE, causal=True, q_offset=r0)
    _check_prefill(from_torch_bf16(out[b:b + 1, r0:r1]), lse[b:b + 1, :, r0:r1].cpu().numpy(), o_ref, lse_ref,
                   f"{what} batch {b} rows {r0}:{r1}")


def test_prefill_config4_full_size(cuda):
    """B=1, S=4096, Hq=16, Hkv=1, causal, N(0,1)."""
    fg = _fg()
    B, S, Hq, Hkv = 1, 4096, 16, 1
    q = gpu_normal_bf16((B, S, Hq, 128), 41, 1.0, cuda)
    k = gpu_normal_bf16((B, S, Hkv, 128), 42, 1.0, cuda)
    v = gpu_normal_bf16((B, S, Hkv, 128), 43, 1.0, cuda)
    out, lse = fg.flash_gqa_forward_bshd(q, k, v, SCALE)
    _sync()
    assert bool(out.isfinite().all())
    for rows in ((0, 128), (1000, 1064), (4096 - 128, 4096)):
        _sampled_prefill_check(q, k, v, out, lse, rows, 0, "config4")


def test_prefill_auto_kernel_choice(cuda):
    """What AUTO resolves to on this device: the wide kernel at BASELINE
    config 4 (its 128 unit pairs fill the 256 CUs), at config 5 and at other
    causal grids of 2 or more 128-row units per CU (whole units, persistent),
    for both head-dim shapes; the split kernel for a small grid and for a
    non-causal grid below 4 units per CU; the whole-range kernel with a
    sliding window and for large non-causal grids."""
    import torch
    fg = _fg()
    cus = torch.cuda.get_device_properties(cuda).multi_processor_count

    def choice(B, S, Hq, Hkv, dk=128, **kw):
        q = torch.empty((B, S, Hq, dk), dtype=torch.bfloat16, device=cuda)
        k = torch.empty((B, S, Hkv, dk), dtype=torch.bfloat16, device=cuda)
        v = torch.empty((B, S, Hkv, 128), dtype=torch.bfloat16, device=cuda)
        return fg.prefill_kernel_choice(q, k, v, **kw)

    if cus == 256:
        assert choice(1, 4096, 16, 1) == "wide"
        assert choice(1, 4096, 16, 16, dk=192) == "wide"
        assert choice(8, 1024, 32, 8) == "wide"          # 2048 units
        assert choice(2, 1024, 16, 4) == "split"         # 256 units
    assert choice(1, 1024, 16, 1) == "split"
    assert choice(4, 16384, 32, 8) == "wide"
    assert choice(4, 8192, 16, 16, dk=192) == "wide"
    assert choice(1, 1024, 16, 16, dk=192) == "split"
    assert choice(4, 16384, 32, 8, causal=False) == "whole"
    assert choice(1, 4096, 16, 1, window_size=128) == "whole"
    assert choice(1, 4096, 16, 1, window_size=1024) == "whole"
    assert choice(1, 4096, 16, 1, window_size=2048) == "wide"   # long windows: the 256-row kernels
    sink = torch.ones(16, dtype=torch.float32, device=cuda)
    if cus == 256:
        assert choice(1, 4096, 16, 1, sink=sink) == "wide"     # a sink alone, a unit per CU or more
        assert choice(1, 2048, 16, 1, sink=sink) == "wide"
    assert choice(1, 1024, 16, 1, sink=sink) == "whole"
    assert choice(1, 4096, 16, 1, kernel="split") == "split"


@pytest.mark.parametrize("kernel", ["wide", "tall"])
def test_prefill_wide_config4_repeatable(cuda, kernel):
    """The wide (and tall) kernel at BASELINE config 4, where every pair of its
    256-row units but one splits its heavy unit over two workgroups: 200
    launches in a row, each compared bit for bit with the first (the arrival
    counters return to 0, and the merge does not depend on which workgroup
    finishes first), and sampled rows of split units match the oracle."""
    import torch
    fg = _fg()
    B, S, Hq, Hkv = 1, 4096, 16, 1
    q = gpu_normal_bf16((B, S, Hq, 128), 44, 1.0, cuda)
    k = gpu_normal_bf16((B, S, Hkv, 128), 45, 1.0, cuda)
    v = gpu_normal_bf16((B, S, Hkv, 128), 46, 1.0, cuda)
    out0, lse0 = fg.flash_gqa_forward_bshd(q, k, v, SCALE, kernel=kernel)
    out, lse = torch.empty_like(out0), torch.empty_like(lse0)
    step = fg.prepare_prefill(q, k, v, SCALE, out=out, lse=lse, causal=True, kernel=kernel)
    diff = torch.zeros((), dtype=torch.int32, device=cuda)
    for i in range(200):
        step()
        # count launches that differ, on the device (no synchronisation per launch)
        same = (out.view(torch.int16) == out0.view(torch.int16)).all() & (lse.view(torch.int32) ==
                                                                          lse0.view(torch.int32)).all()
        diff += (~same).to(torch.int32)
        if i % 50 == 49:
            assert int(diff.item()) == 0, f"{kernel} kernel: a launch before {i + 1} differs from the first"
    assert bool(out0.isfinite().all())
    for rows in ((0, 64), (2016, 2080), (4096 - 96, 4096)):
        _sampled_prefill_check(q, k, v, out0, lse0, rows, 0, f"config4 {kernel}")


def test_prefill_concurrent_streams_config4(cuda):
    """Config-4 prefills on two streams of the same priority at once: the
    kernels that merge a unit's two halves through device memory get a
    workspace per stream from the Python mirror, so each stream's output is
    bit-identical to its serial run (a shared merge slot would mix them)."""
    import torch
    fg = _fg()
    B, S, Hq, Hkv = 1, 4096, 16, 1
    ins = [tuple(gpu_normal_bf16(shape, seed, 1.0, cuda) for shape, seed in
                 (((B, S, Hq, 128), 60 + 3 * i), ((B, S, Hkv, 128), 61 + 3 * i), ((B, S, Hkv, 128), 62 + 3 * i)))
           for i in range(2)]
    assert fg.prefill_kernel_choice(*ins[0]) in ("wide", "split")
    serial = [fg.flash_gqa_forward_bshd(*x, SCALE) for x in ins]
    _sync()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [[None] * 2 for _ in range(20)]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    for r in range(20):
        for i, s in enumerate(streams):
            with torch.cuda.stream(s):
                outs[r][i] = fg.flash_gqa_forward_bshd(*ins[i], SCALE)
    for s in streams:
        torch.cuda.current_stream().wait_stream(s)
    _sync()
    for r in range(20):
        for i in range(2):
            o, l = outs[r][i]
            assert torch.equal(o, serial[i][0]) and torch.equal(l, serial[i][1]), f"round {r} stream {i}"


def test_prefill_caller_workspace(cuda):
    """The merge workspace through the C ABI: the size query at config 4, a
    caller workspace (zeroed counter prefix) giving the library scratch's
    output bit for bit, twice in a row without clearing, and the refusals (too
    small, NULL with a size, misaligned) before any launch."""
    import torch
    from cuda_llm_ops_amd import _lib
    from cuda_llm_ops_amd import flash_gqa as fgm
    fg = _fg()
    L = fg.lib()
    B, S, Hq, Hkv = 1, 4096, 16, 1
    q = gpu_normal_bf16((B, S, Hq, 128), 70, 1.0, cuda)
    k = gpu_normal_bf16((B, S, Hkv, 128), 71, 1.0, cuda)
    v = gpu_normal_bf16((B, S, Hkv, 128), 72, 1.0, cuda)
    out = torch.empty_like(q)
    lse = torch.empty((B, Hq, S), dtype=torch.float32, device=cuda)
    a = fgm._prefill_args(q, k, v, out, lse, SCALE, True, "bshd", kernel="wide")
    n = ctypes.c_size_t(0)
    assert L.fgqa_prefill_workspace_bytes(ctypes.byref(a), ctypes.byref(n)) == 0
    cus = torch.cuda.get_device_properties(cuda).multi_processor_count
    pairs = (2 * (S // 32) + 1) // 2   # 256-row units: 8 heads x 32 positions, 2 head groups
    if 2 * pairs <= cus:
        assert n.value == 4096 + pairs * 2 * (2 * 4 * 66 * 64) * 4
    else:
        assert n.value == 0
    st = torch.cuda.current_stream().cuda_stream
    assert L.fgqa_prefill_bf16(ctypes.byref(a), ctypes.c_void_p(st)) == 0   # library scratch
    _sync()
    ref_o, ref_l = out.clone(), lse.clone()
    if n.value == 0:
        return
    ws = torch.empty(n.value + 512, dtype=torch.uint8, device=cuda)
    ws[:4096].zero_()
    a.workspace, a.workspace_bytes = ws.data_ptr(), n.value
    for _ in range(2):
        out.zero_()
        assert L.fgqa_prefill_bf16(ctypes.byref(a), ctypes.c_void_p(st)) == 0
        _sync()
        assert torch.equal(out, ref_o) and torch.equal(lse, ref_l)
    assert int(ws[:4096].to(torch.int32).abs().sum()) == 0, "counters left nonzero"
    a.workspace_bytes = n.value - 1
    assert L.fgqa_prefill_bf16(ctypes.byref(a), ctypes.c_void_p(st)) == _lib.FGQA_ERR_WORKSPACE
    a.workspace, a.workspace_bytes = None, n.value
    assert L.fgqa_prefill_bf16(ctypes.byref(a), ctypes.c_void_p(st)) == _lib.FGQA_ERR_WORKSPACE
    a.workspace, a.workspace_bytes = ws.data_ptr() + 16, n.value
    assert L.fgqa_prefill_bf16(ctypes.byref(a), ctypes.c_void_p(st)) == _lib.FGQA_ERR_UNSUPPORTED
    # shapes whose kernels merge nothing need no workspace
    a2 = fgm._prefill_args(q, k, v, out, lse, SCALE, False, "bshd", kernel="wide")
    assert L.fgqa_prefill_workspace_bytes(ctypes.byref(a2), ctypes.byref(n)) == 0 and n.value == 0
    a3 = fgm._prefill_args(q, k, v, out, lse, SCALE, True, "bshd", kernel="split")
    assert L.fgqa_prefill_workspace_bytes(ctypes.byref(a3), ctypes.byref(n)) == 0 and n.value == 0


def test_prefill_kernel_names(cuda):
    """The kernel function the library reports for a call: the grid form of
    the 256-row kernels follows the pair count."""
    import torch
    fg = _fg()
    cus = torch.cuda.get_device_properties(cuda).multi_processor_count

    def name(B, S, Hq, Hkv, **kw):
        q = torch.empty((B, S, Hq, 128), dtype=torch.bfloat16, device=cuda)
        k = torch.empty((B, S, Hkv, 128), dtype=torch.bfloat16, device=cuda)
        return fg.prefill_kernel_name(q, k, k, **kw)

    assert name(4, 16384, 32, 8) == "prefill_wide_persistent_kernel"
    assert name(4, 16384, 32, 8, kernel="tall") == "prefill_tall_persistent_kernel"
    assert name(1, 1024, 16, 1, kernel="split") == "prefill_split_kernel"
    assert name(1, 1024, 16, 1, kernel="whole") == "prefill_kernel"
    if cus == 256:
        assert name(1, 4096, 16, 1) == "prefill_wide_kernel"
        assert name(1, 4096, 16, 1, kernel="tall") == "prefill_tall_pairs_kernel"
        assert name(1, 4096, 16, 1, causal=False, kernel="tall") == "prefill_tall_persistent_kernel"


def test_prefill_wide_graph_replays(cuda):
    """The wide kernel (split units merging through the library's device
    memory) captured in a HIP graph: every launch leaves the arrival counters
    at 0 and no memset is recorded, so each replay, with eager launches and
    synchronizations between replays, must match the eager result exactly."""
    import torch
    fg = _fg()
    B, S, Hq, Hkv = 1, 2048, 16, 1   # 64 unit pairs, all but the lightest split
    q = gpu_normal_bf16((B, S, Hq, 128), 47, 1.0, cuda)
    k = gpu_normal_bf16((B, S, Hkv, 128), 48, 1.0, cuda)
    v = gpu_normal_bf16((B, S, Hkv, 128), 49, 1.0, cuda)
    out = torch.empty_like(q)
    lse = torch.empty((B, Hq, S), dtype=torch.float32, device=cuda)
    step = fg.prepare_prefill(q, k, v, SCALE, out=out, lse=lse, causal=True, kernel="wide")
    step()   # one-time set-up (kernel attributes, device memory lookup) outside the capture
    _sync()
    ref_o, ref_l = out.clone(), lse.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            step()
    torch.cuda.current_stream().wait_stream(s)
    for i in range(4):
        out.zero_()
        lse.zero_()
        g.replay()
        _sync()
        assert torch.equal(out, ref_o) and torch.equal(lse, ref_l), f"replay {i}"
        step()   # an eager launch between replays
        _sync()
        assert torch.equal(out, ref_o), f"eager launch after replay {i}"
    _sampled_prefill_check(q, k, v, out, lse, (S - 64, S), 0, "wide kernel after graph replays")


def test_prefill_config5_full_size(cuda):
    """B=4, S=16384, Hq=32, Hkv=8, causal, N(0, 0.5^2): sampled rows."""
    fg = _fg()
    B, S, Hq, Hkv = 4, 16384, 32, 8
    q = gpu_normal_bf16((B, S, Hq, 128), 51, 0.5, cuda)
    k = gpu_normal_bf16((B, S, Hkv, 128), 52, 0.5, cuda)
    v = gpu_normal_bf16((B, S, Hkv, 128), 53, 0.5, cuda)
    out, lse = fg.flash_gqa_forward_bshd(q, k, v, SCALE)
    _sync()
    assert bool(out.isfinite().all())
    _sampled_prefill_check(q, k, v, out, lse, (0, 128), 0, "config5")
    _sampled_prefill_check(q, k, v, out, lse, (S - 64, S), 0, "config5")
    _sampled_prefill_check(q, k, v, out, lse, (9000, 9032), 3, "config5")


def test_prefill_cplusplus_dropin(cuda):
    import torch
    fg = _fg()
    L = fg.lib()
    B, S, Hq, Hkv = 1, 256, 16, 1
    q = oracle.normal_bf16(900, (B, S, Hq, 128))
    k = oracle.normal_bf16(900, (B, S, Hkv, 128), stream=1)
    v = oracle.normal_bf16(900, (B, S, Hkv, 128), stream=2)
    o_ref, lse_ref = oracle.prefill(q, k, v, SCALE, causal=True)
    qd, kd, vd = (to_torch_bf16(x, cuda) for x in (q, k, v))
    od = torch.zeros_like(qd)
    ld = torch.zeros((B, Hq, S), dtype=torch.float32, device=cuda)
    fn = getattr(L, "_Z31LaunchFlashGqaForwardBf16KernelPK6bf16_tS1_S1_fPS_Pfiiiiiib")
    fn.restype = None
    torch.cuda.synchronize()
    fn(ctypes.c_void_p(qd.data_ptr()), ctypes.c_void_p(kd.data_ptr()), ctypes.c_void_p(vd.data_ptr()),
       ctypes.c_float(SCALE), ctypes.c_void_p(od.data_ptr()), ctypes.c_void_p(ld.data_ptr()),
       B, S, S, Hq, Hkv, 128, ctypes.c_bool(True))
    torch.cuda.synchronize()
    _check_prefill(from_torch_bf16(od), ld.cpu().numpy(), o_ref, lse_ref, "C++ drop-in prefill")
