"""GPU tests of the paged-KV decode (block table; bf16 or OCP fp8 e4m3 caches).

No reference counterpart: the checks are the paged oracle
(oracle/fgqa_oracle.c fgqa_oracle_decode_paged, itself pinned bit-for-bit to
the contiguous decode oracle) at the decode bar (max-abs 2e-2, mean-abs 2e-3),
and two bit-exact identities at BASELINE config 3's size: paged bf16 against
the contiguous decode of the same K/V, and fp8 against bf16 pages holding the
decoded values (the arithmetic after staging is the same in each pair).
"""
import math

import numpy as np
import pytest

import oracle
from tests._helpers import assert_close, fp8_quantize, from_torch_bf16, make_paged, to_torch_bf16

pytestmark = pytest.mark.gpu

SCALE = 1.0 / math.sqrt(128)
LSE_TOL = 1e-3


def _fg():
    import cuda_llm_ops_amd as fg
    return fg


def _case(cuda, seed, B, Hq, Hkv, S, lens, page_size, fp8, split_tokens=0):
    import torch
    rng = np.random.default_rng(seed)
    q = oracle.normal_bf16(seed, (B, Hq, 128))
    if fp8:
        kf = rng.standard_normal((B, S, Hkv, 128)).astype(np.float32)
        vf = rng.standard_normal((B, S, Hkv, 128)).astype(np.float32)
        ks, vs = float(np.abs(kf).max() / 448), float(np.abs(vf).max() / 448)
        k, v = fp8_quantize(kf, ks), fp8_quantize(vf, vs)
    else:
        k = oracle.normal_bf16(seed, (B, S, Hkv, 128), stream=1)
        v = oracle.normal_bf16(seed, (B, S, Hkv, 128), stream=2)
        ks = vs = 1.0
    lens = np.asarray(lens, dtype=np.int32)
    kc, vc, bt = make_paged(k, v, lens, page_size, rng)
    o_ref, l_ref = oracle.decode_paged(q, kc, vc, bt, lens, SCALE, k_scale=ks, v_scale=vs)
    if fp8:
        kd = torch.from_numpy(kc).to(cuda).view(torch.float8_e4m3fn)
        vd = torch.from_numpy(vc).to(cuda).view(torch.float8_e4m3fn)
    else:
        kd, vd = to_torch_bf16(kc, cuda), to_torch_bf16(vc, cuda)
    qd = to_torch_bf16(q, cuda)
    btd = torch.from_numpy(bt).to(cuda)
    sld = torch.from_numpy(lens).to(cuda)
    lse = torch.empty((B, Hq), dtype=torch.float32, device=cuda)
    out = _fg().decode_flash_gqa_paged(qd, kd, vd, btd, sld, SCALE, k_scale=ks, v_scale=vs, lse=lse,
                                       split_tokens=split_tokens)
    torch.cuda.synchronize()
    return from_torch_bf16(out), lse.cpu().numpy(), o_ref, l_ref


def _check(o, lse, o_ref, l_ref, what):
    assert_close(oracle.bf16_to_f32(o), oracle.bf16_to_f32(o_ref), what)
    fin = np.isfinite(l_ref)
    assert np.array_equal(np.isfinite(lse), fin), f"{what}: lse finiteness"
    assert np.max(np.abs(lse[fin] - l_ref[fin]), initial=0.0) <= LSE_TOL, f"{what}: lse"


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("page_size", [1, 2, 4, 8, 16, 32, 64, 256])
def test_paged_page_sizes(cuda, page_size, fp8):
    what = f"paged page={page_size} fp8={fp8}"
    print(what, flush=True)
    o, lse, o_ref, l_ref = _case(cuda, 900 + page_size, 3, 16, 2, 700, [700, 1, 333], page_size, fp8)
    _check(o, lse, o_ref, l_ref, what)


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("Hkv", [1, 3])
def test_paged_odd_kv_heads(cuda, Hkv, fp8):
    """Odd kv head counts run the one-head-per-workgroup list kernel (even
    counts pair two heads in an 8-wave workgroup)."""
    what = f"paged Hkv={Hkv} fp8={fp8}"
    print(what, flush=True)
    for page_size in (2, 16):
        o, lse, o_ref, l_ref = _case(cuda, 970 + Hkv + page_size, 3, 4 * Hkv, Hkv, 700, [700, 1, 333], page_size,
                                     fp8)
        _check(o, lse, o_ref, l_ref, f"{what} page={page_size}")


@pytest.mark.parametrize("page_size", [4, 8, 16, 32, 128])
def test_paged_segments_split_inside_pages(cuda, page_size):
    """Pages read by page segment, with 128-token splits (a split ends
    inside a page for pages of 256) and lengths that end inside a segment, a
    load instruction and a page; bf16 and fp8 (fp8 segments start at 8 rows)."""
    lens = [1023, 131, 5, 1024, 769]
    for fp8 in (False, True):
        what = f"paged segments page={page_size} fp8={fp8}"
        print(what, flush=True)
        o, lse, o_ref, l_ref = _case(cuda, 950 + page_size, 5, 16, 2, 1024, lens, page_size, fp8, split_tokens=128)
        _check(o, lse, o_ref, l_ref, what)


@pytest.mark.parametrize("G", [1, 4, 16])
@pytest.mark.parametrize("fp8", [False, True])
def test_paged_groups_splits_and_empty(cuda, G, fp8):
    what = f"paged G={G} fp8={fp8}"
    print(what, flush=True)
    for split in (0, 128, 512):
        o, lse, o_ref, l_ref = _case(cuda, 950 + G, 4, 2 * G, 2, 1200, [1200, 0, 129, 640], 16, fp8,
                                     split_tokens=split)
        _check(o, lse, o_ref, l_ref, f"{what} split={split}")
        assert np.all(o[1] == 0) and np.all(np.isneginf(lse[1]))


def _config3_inputs(cuda, seed=3):
    import torch
    B, S, Hq, Hkv = 64, 32768, 64, 8
    rng = np.random.default_rng(seed)
    lens = (1 + rng.integers(0, S, size=B)).astype(np.int32)
    g = torch.Generator(device=cuda)
    g.manual_seed(seed)
    q = torch.randn((B, Hq, 128), generator=g, device=cuda).to(torch.bfloat16)
    return B, S, Hq, Hkv, lens, q, g


def _paginate(cuda, k, lens, page_size, perm_seed):
    """[B, S, Hkv, D] contiguous -> (pages [n, page_size, Hkv, D], block table) with pages in random order."""
    import torch
    B, S, Hkv, D = k.shape
    max_pages = S // page_size
    n = B * max_pages
    perm = torch.from_numpy(np.random.default_rng(perm_seed).permutation(n).astype(np.int64)).to(cuda)
    pages = torch.empty((n, page_size, Hkv, D), dtype=k.dtype, device=cuda)
    pages[perm] = k.reshape(n, page_size, Hkv, D)
    table = perm.view(B, max_pages).to(torch.int32)
    return pages, table


def test_paged_config3_bf16_bit_identical_to_contiguous(cuda):
    """BASELINE config 3 (ragged B=64, lengths U{1..32768}, Hq=64, Hkv=8) in 16-token
    pages: the same bits as the contiguous ragged decode of the same K/V."""
    import torch
    fg = _fg()
    print("paged config3 bf16", flush=True)
    B, S, Hq, Hkv, lens, q, g = _config3_inputs(cuda)
    k = torch.randn((B, S, Hkv, 128), generator=g, device=cuda).to(torch.bfloat16)
    v = torch.randn((B, S, Hkv, 128), generator=g, device=cuda).to(torch.bfloat16)
    sl = torch.from_numpy(lens).to(cuda)
    ref = fg.decode_flash_gqa_bshd(q, k, v, SCALE, seqlens=sl)
    kc, bt = _paginate(cuda, k, lens, 16, 5)
    vc, _ = _paginate(cuda, v, lens, 16, 5)
    del k, v
    out = fg.decode_flash_gqa_paged(q, kc, vc, bt, sl, SCALE)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def test_paged_config3_fp8_matches_decoded_bf16(cuda):
    """fp8 pages at config 3's shape: bit-identical to bf16 pages holding the
    decoded values with the same scales, and within the bar of the oracle on
    two sampled sequences."""
    import torch
    fg = _fg()
    print("paged config3 fp8", flush=True)
    B, S, Hq, Hkv, lens, q, g = _config3_inputs(cuda, seed=4)
    ks, vs = 0.011, 0.009
    # the cast turns values beyond the e4m3 range (448) into NaN, so clamp first
    k8 = (torch.randn((B, S, Hkv, 128), generator=g, device=cuda) / ks).clamp_(-448, 448).to(torch.float8_e4m3fn)
    v8 = (torch.randn((B, S, Hkv, 128), generator=g, device=cuda) / vs).clamp_(-448, 448).to(torch.float8_e4m3fn)
    kc, bt = _paginate(cuda, k8, lens, 64, 6)
    vc, _ = _paginate(cuda, v8, lens, 64, 6)
    del k8, v8
    sl = torch.from_numpy(lens).to(cuda)
    out = fg.decode_flash_gqa_paged(q, kc, vc, bt, sl, SCALE, k_scale=ks, v_scale=vs)
    ref = fg.decode_flash_gqa_paged(q, kc.to(torch.bfloat16), vc.to(torch.bfloat16), bt, sl, SCALE,
                                    k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    assert bool(out.isfinite().all())
    assert torch.equal(out, ref)
    for b in (int(np.argmin(lens)), int(np.argmax(lens))):
        n = int(lens[b])
        rows = bt[b, : -(-n // 64)].long()
        kb = kc[rows].view(torch.uint8).cpu().numpy()[None].reshape(1, -1, 64, Hkv, 128)[0]
        vb = vc[rows].view(torch.uint8).cpu().numpy()[None].reshape(1, -1, 64, Hkv, 128)[0]
        tab = np.arange(kb.shape[0], dtype=np.int32)[None]
        o_ref, _ = oracle.decode_paged(from_torch_bf16(q[b:b + 1]), kb, vb, tab, np.array([n], np.int32), SCALE,
                                       k_scale=ks, v_scale=vs)
        assert_close(oracle.bf16_to_f32(from_torch_bf16(out[b:b + 1])), oracle.bf16_to_f32(o_ref),
                     f"config3 fp8 sequence {b} (len {n})")


def test_paged_rejections(cuda):
    import torch
    fg = _fg()
    q = torch.zeros((2, 8, 128), dtype=torch.bfloat16, device=cuda)
    kc = torch.zeros((4, 24, 1, 128), dtype=torch.bfloat16, device=cuda)
    bt = torch.zeros((2, 4), dtype=torch.int32, device=cuda)
    sl = torch.zeros(2, dtype=torch.int32, device=cuda)
    with pytest.raises(fg.FgqaError):   # page size not a power of two
        fg.decode_flash_gqa_paged(q, kc, kc, bt, sl)
    kc = torch.zeros((4, 16, 1, 128), dtype=torch.bfloat16, device=cuda)
    with pytest.raises(fg.FgqaError):   # max_seqlen beyond what the table covers
        fg.decode_flash_gqa_paged(q, kc, kc, bt, sl, max_seqlen=65)
    with pytest.raises(ValueError):
        fg.decode_flash_gqa_paged(q, kc, kc.float(), bt, sl)


def test_paged_cplusplus_entry(cuda):
    """LaunchFlashGqaBf16KernelPaged (default stream), bf16 and fp8 caches."""
    import ctypes

    import torch
    fg = _fg()
    L = fg.lib()
    fn = getattr(L, "_Z29LaunchFlashGqaBf16KernelPagedPK6bf16_tPKvS3_bfffPS_PKiS6_iiiiiii")
    fn.restype = None
    st = getattr(L, "_Z21FlashGqaGetLastStatusv")
    st.restype = ctypes.c_int
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    for fp8 in (False, True):
        print(f"paged C++ entry fp8={fp8}", flush=True)
        rng = np.random.default_rng(5)
        B, Hq, Hkv, S, ps = 2, 16, 2, 256, 32
        q = oracle.normal_bf16(970, (B, Hq, 128))
        if fp8:
            k = fp8_quantize(rng.standard_normal((B, S, Hkv, 128)), 0.02)
            v = fp8_quantize(rng.standard_normal((B, S, Hkv, 128)), 0.02)
            ks = vs = 0.02
        else:
            k = oracle.normal_bf16(970, (B, S, Hkv, 128), stream=1)
            v = oracle.normal_bf16(970, (B, S, Hkv, 128), stream=2)
            ks = vs = 1.0
        lens = np.array([256, 77], dtype=np.int32)
        kc, vc, bt = make_paged(k, v, lens, ps, rng)
        o_ref, _ = oracle.decode_paged(q, kc, vc, bt, lens, SCALE, k_scale=ks, v_scale=vs)
        kd = torch.from_numpy(kc).to(cuda)
        vd = torch.from_numpy(vc).to(cuda)
        qd = to_torch_bf16(q, cuda)
        btd = torch.from_numpy(bt).to(cuda)
        sld = torch.from_numpy(lens).to(cuda)
        od = torch.zeros_like(qd)
        torch.cuda.synchronize()
        fn(p(qd), p(kd), p(vd), ctypes.c_bool(fp8), ctypes.c_float(SCALE), ctypes.c_float(ks), ctypes.c_float(vs),
           p(od), p(btd), p(sld), B, bt.shape[1], ps, kc.shape[0], Hq, Hkv, 128)
        assert st() == 0
        torch.cuda.synchronize()
        assert_close(oracle.bf16_to_f32(from_torch_bf16(od)), oracle.bf16_to_f32(o_ref), f"C++ paged fp8={fp8}")
