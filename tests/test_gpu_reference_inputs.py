"""GPU parity at the reference harnesses' own input distribution, U[0,1) for
Q, K and V (examples/cplusplus/test_decode_flash_gqa.cu:162-177,
examples/python/Triton/test_flash_gqa_kernel.py:390-418), at BASELINE config
2's and config 4's shapes; the BHSD decode mirror checked against the oracle
directly; and BASELINE config 5 on 256 seeded random rows of every batch.

With U[0,1) inputs every score is ~2.8 +- 0.3, so the softmax is nearly flat
over thousands of keys and O sits near 0.5: a test of long fp32 sums of
similar terms rather than of a few dominant keys.  Bar: max-abs 2e-2,
mean-abs 2e-3 on bf16 outputs, LSE within 1e-3 (tests/_helpers.py)."""
import math

import numpy as np
import pytest

import oracle
from tests._helpers import assert_close, from_torch_bf16, gpu_normal_bf16

pytestmark = pytest.mark.gpu

SCALE = 1.0 / math.sqrt(128)
LSE_TOL = 1e-3


def _fg():
    import cuda_llm_ops_amd as fg
    return fg


def _uniform(shape, seed, dev):
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    return torch.rand(shape, generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)


def _check(o, lse, o_ref, lse_ref, what):
    assert_close(oracle.bf16_to_f32(o), oracle.bf16_to_f32(o_ref), what)
    fin = np.isfinite(lse_ref)
    assert np.array_equal(np.isfinite(lse), fin), f"{what}: lse finiteness"
    assert np.max(np.abs(lse[fin] - lse_ref[fin]), initial=0.0) <= LSE_TOL, f"{what}: lse"


def test_decode_config2_uniform_inputs_and_bhsd_mirror(cuda):
    """Config 2's shape (B=60, S=4096, Hq=128, Hkv=8) with U[0,1) inputs: the
    BSHD decode and the Triton-layout mirror launch_decode_flash_gqa_bf16_kernel
    (BHSD, scale 1/sqrt(D)), each against the oracle on sampled batches."""
    import torch
    fg = _fg()
    print("decode config 2 shape, U[0,1) inputs", flush=True)
    B, S, Hq, Hkv = 60, 4096, 128, 8
    q = _uniform((B, Hq, 128), 61, cuda)
    k = _uniform((B, S, Hkv, 128), 62, cuda)
    v = _uniform((B, S, Hkv, 128), 63, cuda)
    lse = torch.empty((B, Hq), dtype=torch.float32, device=cuda)
    out = fg.decode_flash_gqa_bshd(q, k, v, SCALE, lse=lse)
    mirror = fg.launch_decode_flash_gqa_bf16_kernel(q[:, :, None, :].contiguous(),
                                                    k.permute(0, 2, 1, 3).contiguous(),
                                                    v.permute(0, 2, 1, 3).contiguous())
    torch.cuda.synchronize()
    o_np, m_np = from_torch_bf16(out), from_torch_bf16(mirror[:, :, 0, :])
    for b in (0, 17, 42, 59):
        o_ref, lse_ref = oracle.decode(from_torch_bf16(q[b:b + 1]), from_torch_bf16(k[b:b + 1]),
                                       from_torch_bf16(v[b:b + 1]), SCALE)
        _check(o_np[b:b + 1], lse[b:b + 1].cpu().numpy(), o_ref, lse_ref, f"U[0,1) decode batch {b}")
        assert_close(oracle.bf16_to_f32(m_np[b:b + 1]), oracle.bf16_to_f32(o_ref), f"BHSD mirror batch {b}")


def test_prefill_config4_uniform_inputs_every_row(cuda):
    """Config 4's shape (B=1, S=4096, Hq=16, Hkv=1, causal) with U[0,1) inputs,
    every row and head against the oracle."""
    fg = _fg()
    print("prefill config 4 shape, U[0,1) inputs, all rows", flush=True)
    B, S, Hq, Hkv = 1, 4096, 16, 1
    q = _uniform((B, S, Hq, 128), 64, cuda)
    k = _uniform((B, S, Hkv, 128), 65, cuda)
    v = _uniform((B, S, Hkv, 128), 66, cuda)
    out, lse = fg.flash_gqa_forward_bshd(q, k, v, SCALE, causal=True)
    o_ref, lse_ref = oracle.prefill(from_torch_bf16(q), from_torch_bf16(k), from_torch_bf16(v), SCALE, causal=True)
    _check(from_torch_bf16(out), lse.cpu().numpy(), o_ref, lse_ref, "U[0,1) prefill config 4")


def test_prefill_config5_random_rows_every_batch(cuda):
    """BASELINE config 5 (B=4, S=16384, Hq=32, Hkv=8, causal, N(0, 0.5^2)):
    256 seeded random rows of every batch, each row's 32 heads against the oracle."""
    fg = _fg()
    print("prefill config 5, 256 random rows per batch", flush=True)
    B, S, Hq, Hkv = 4, 16384, 32, 8
    q = gpu_normal_bf16((B, S, Hq, 128), 51, 0.5, cuda)
    k = gpu_normal_bf16((B, S, Hkv, 128), 52, 0.5, cuda)
    v = gpu_normal_bf16((B, S, Hkv, 128), 53, 0.5, cuda)
    out, lse = fg.flash_gqa_forward_bshd(q, k, v, SCALE, causal=True)
    lse_np = lse.cpu().numpy()
    rng = np.random.default_rng(55)
    for b in range(B):
        qh, kh, vh, oh = (from_torch_bf16(t[b:b + 1]) for t in (q, k, v, out))
        rows = np.sort(rng.choice(S, size=256, replace=False))
        got_o, got_l, ref_o, ref_l = [], [], [], []
        for r in rows:
            r = int(r)
            o_ref, l_ref = oracle.prefill(qh[:, r:r + 1], kh[:, :r + 1], vh[:, :r + 1], SCALE, causal=True, q_offset=r)
            got_o.append(oh[:, r:r + 1]); got_l.append(lse_np[b:b + 1, :, r:r + 1])
            ref_o.append(o_ref); ref_l.append(l_ref)
        _check(np.concatenate(got_o, 1), np.concatenate(got_l, 2), np.concatenate(ref_o, 1),
               np.concatenate(ref_l, 2), f"config5 batch {b}, 256 random rows")
