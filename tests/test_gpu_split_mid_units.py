"""GPU parity of the split prefill kernel at ragged shapes with between one
and two 128-row units per CU (the range config 4 sits in: 512 units on 256
CUs), where the dispatcher hands every CU a heavy unit and then a light one.

The shapes are derived from the device's CU count so that the unit count
lands in that range.  A unit is 128 query rows: 4 heads x 32 positions here,
so units = ceil(Sq / 32) x (Hq / 4).  Cases: a ragged last query block, an
odd unit count, and a non-causal launch over a short, ragged KV range (the
last K/V tile is clamped).  Checked against the oracle in 32-row blocks: the
first and last blocks, and seeded random ones in between."""
import math

import numpy as np
import pytest

import oracle
from tests._helpers import assert_close, from_torch_bf16, gpu_normal_bf16

pytestmark = pytest.mark.gpu

SCALE = 1.0 / math.sqrt(128)
LSE_TOL = 1e-3


def _cus():
    import torch
    return torch.cuda.get_device_properties(0).multi_processor_count


def _run_and_check(B, Sq, Skv, Hq, Hkv, causal, seed, n_blocks, cuda):
    import cuda_llm_ops_amd as fg
    cus = _cus()
    units = B * Hkv * (Hq // Hkv // 4) * math.ceil(Sq / 32)
    if not cus < units <= 2 * cus:
        pytest.skip(f"{units} units is not in ({cus}, {2 * cus}] on this device")
    print(f"split kernel: B={B} Sq={Sq} Skv={Skv} Hq={Hq} Hkv={Hkv} causal={causal} units={units} cus={cus}", flush=True)
    q = gpu_normal_bf16((B, Sq, Hq, 128), seed, 1.0, cuda)
    k = gpu_normal_bf16((B, Skv, Hkv, 128), seed + 1, 1.0, cuda)
    v = gpu_normal_bf16((B, Skv, Hkv, 128), seed + 2, 1.0, cuda)
    out, lse = fg.flash_gqa_forward_bshd(q, k, v, SCALE, causal=causal, kernel="split")
    o_np, lse_np = from_torch_bf16(out), lse.cpu().numpy()
    qh, kh, vh = from_torch_bf16(q), from_torch_bf16(k), from_torch_bf16(v)
    rng = np.random.default_rng(seed)
    starts = {0, max(0, Sq - 32)} | {int(s) for s in rng.integers(0, Sq, size=n_blocks)}
    for r0 in sorted(starts):
        r1 = min(Sq, r0 + 32)
        kv = min(Skv, r1) if causal else Skv
        o_ref, l_ref = oracle.prefill(qh[:, r0:r1], kh[:, :kv], vh[:, :kv], SCALE, causal=causal, q_offset=r0)
        what = f"rows [{r0}, {r1})"
        assert_close(oracle.bf16_to_f32(o_np[:, r0:r1]), oracle.bf16_to_f32(o_ref), what)
        got = lse_np[:, :, r0:r1]
        fin = np.isfinite(l_ref)
        assert np.array_equal(np.isfinite(got), fin), f"{what}: lse finiteness"
        assert np.max(np.abs(got[fin] - l_ref[fin]), initial=0.0) <= LSE_TOL, f"{what}: lse"


def test_split_causal_ragged(cuda):
    """Causal, Hq=16 over one KV head (4 units per 32 positions), a ragged
    last query block."""
    n_q = _cus() // 4 + 37
    S = 32 * n_q - 13
    _run_and_check(1, S, S, 16, 1, True, 301, 24, cuda)


def test_split_causal_odd_unit_count(cuda):
    """Causal, Hq=4 over one KV head (1 unit per 32 positions), an odd unit
    count."""
    n_q = _cus() + 45
    S = 32 * n_q - 7
    _run_and_check(1, S, S, 4, 1, True, 311, 24, cuda)


def test_split_noncausal_short_kv(cuda):
    """Non-causal, two batches, Skv = 777 (the last K/V tile is clamped)."""
    n_q = _cus() // 4 + 11
    Sq = 32 * n_q - 3
    _run_and_check(2, Sq, 777, 8, 2, False, 321, 24, cuda)
