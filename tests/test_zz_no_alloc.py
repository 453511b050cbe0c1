"""The decode entry point that allocates nothing (fgqa_decode_bf16_noalloc),
called through the C ABI and checked against fgqa_decode_bf16 on the same
inputs: same kernels and plan, so the outputs must agree bit for bit.  Two calls
in a row, the second smaller, so stale scratch from the first cannot leak into
the second.  Also: a plan larger than the built-in scratch is refused before any
launch, and so is a caller workspace."""
import ctypes
import math

import numpy as np
import pytest

import oracle
from tests._helpers import assert_close, from_torch_bf16, gpu_normal_bf16, to_torch_bf16

pytestmark = pytest.mark.gpu

SCALE = 1.0 / math.sqrt(128)
SCRATCH_BYTES = 32 << 20   # FGQA_DECODE_NOALLOC_SCRATCH_BYTES


def _args(q, k, v, o, lse, seqlens, max_seqlen):
    import cuda_llm_ops_amd._lib as L
    a = L.DecodeArgs()
    B, Hq, D = q.shape
    Hkv = k.shape[2]
    a.q, a.k, a.v, a.o, a.lse = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr()
    a.seqlens = seqlens.data_ptr() if seqlens is not None else None
    a.batch, a.max_seqlen, a.num_q_heads, a.num_kv_heads, a.head_dim = B, max_seqlen, Hq, Hkv, D
    a.scale = SCALE
    a.q_stride[:] = [q.stride(0), q.stride(1)]
    a.k_stride[:] = [k.stride(0), k.stride(1), k.stride(2)]
    a.v_stride[:] = [v.stride(0), v.stride(1), v.stride(2)]
    a.o_stride[:] = [o.stride(0), o.stride(1)]
    return a


def _both(q, k, v, seqlens, max_seqlen, what):
    """(noalloc out, lse), (fgqa_decode_bf16 out, lse) on the same inputs."""
    import torch
    import cuda_llm_ops_amd._lib as L
    B, Hq, D = q.shape
    res = []
    for fn in (L.lib().fgqa_decode_bf16_noalloc, L.lib().fgqa_decode_bf16):
        o = torch.full((B, Hq, D), float("nan"), dtype=torch.bfloat16, device=q.device)
        lse = torch.full((B, Hq), float("nan"), dtype=torch.float32, device=q.device)
        a = _args(q, k, v, o, lse, seqlens, max_seqlen)
        ws = ctypes.c_size_t(0)
        assert L.lib().fgqa_decode_workspace_bytes(ctypes.byref(a), ctypes.byref(ws)) == 0
        print(f"{what}: {fn.__name__}, plan workspace {ws.value} B", flush=True)
        st = fn(ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        assert st == 0, (what, fn.__name__, st)
        torch.cuda.synchronize()
        res.append((o, lse))
    return res


def test_noalloc_decode_matches_allocating_entry_twice(cuda):
    import torch
    # call 1: BASELINE config 3 (ragged B=64, lengths U{1..32768}, Hq=64, Hkv=8, NaN padding):
    # split partials plus the work list, about half of the scratch
    B, Smax, Hq, Hkv = 64, 32768, 64, 8
    lens = (1 + np.random.default_rng(3).integers(0, 32768, size=B)).astype(np.int32)
    q = gpu_normal_bf16((B, Hq, 128), 41, 1.0, cuda)
    k = gpu_normal_bf16((B, Smax, Hkv, 128), 42, 1.0, cuda)
    v = gpu_normal_bf16((B, Smax, Hkv, 128), 43, 1.0, cuda)
    nan = torch.tensor(float("nan"), dtype=torch.bfloat16, device=cuda)
    for b in range(B):
        k[b, int(lens[b]):] = nan
        v[b, int(lens[b]):] = nan
    sl = torch.from_numpy(lens).to(cuda)
    (o1, l1), (r1, rl1) = _both(q, k, v, sl, Smax, "config 3 ragged")
    assert torch.equal(o1.view(torch.int16), r1.view(torch.int16)), "config 3: O differs from fgqa_decode_bf16"
    assert torch.equal(l1, rl1), "config 3: LSE differs from fgqa_decode_bf16"
    assert bool(o1.isfinite().all())
    del k, v
    # call 2, smaller: BASELINE config 1 (B=2, S=512, Hq=16, Hkv=2, uniform length: split partials)
    qn = oracle.normal_bf16(44, (2, 16, 128))
    kn = oracle.normal_bf16(44, (2, 512, 2, 128), stream=1)
    vn = oracle.normal_bf16(44, (2, 512, 2, 128), stream=2)
    q2, k2, v2 = (to_torch_bf16(x, cuda) for x in (qn, kn, vn))
    (o2, l2), (r2, rl2) = _both(q2, k2, v2, None, 512, "config 1")
    assert torch.equal(o2.view(torch.int16), r2.view(torch.int16)), "config 1: O differs from fgqa_decode_bf16"
    assert torch.equal(l2, rl2), "config 1: LSE differs from fgqa_decode_bf16"
    o_ref, _ = oracle.decode(qn, kn, vn, SCALE)
    assert_close(oracle.bf16_to_f32(from_torch_bf16(o2)), oracle.bf16_to_f32(o_ref), "noalloc config 1 vs oracle")


def test_noalloc_decode_refuses_oversize_plan_and_caller_workspace(cuda):
    """Nothing is launched: the statuses come back before any GPU work."""
    import torch
    import cuda_llm_ops_amd._lib as L
    print("noalloc refusals", flush=True)
    # B=256, Hq=64, Hkv=8, 512 tokens in splits of 128: 4 splits per sequence,
    # 32.5 MiB of partials.  Every tensor has the shape the struct describes
    # (K and V 256 MiB each), so even a launch would stay inside them.
    B, Hq, Hkv, S = 256, 64, 8, 512
    q = torch.zeros((B, Hq, 128), dtype=torch.bfloat16, device=cuda)
    k = torch.zeros((B, S, Hkv, 128), dtype=torch.bfloat16, device=cuda)
    o = torch.zeros_like(q)
    lse = torch.zeros((B, Hq), dtype=torch.float32, device=cuda)
    sl = torch.full((B,), S, dtype=torch.int32, device=cuda)
    a = _args(q, k, k, o, lse, sl, S)
    a.split_tokens = 128
    ws = ctypes.c_size_t(0)
    assert L.lib().fgqa_decode_workspace_bytes(ctypes.byref(a), ctypes.byref(ws)) == 0
    assert ws.value > SCRATCH_BYTES
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert L.lib().fgqa_decode_bf16_noalloc(ctypes.byref(a), s) == L.FGQA_ERR_WORKSPACE
    torch.cuda.synchronize()
    assert torch.isfinite(lse).all() and bool((lse == 0).all()), "a refused call wrote its outputs"
    b = _args(q, k, k, o, lse, sl, S)
    b.workspace, b.workspace_bytes = o.data_ptr(), 1 << 20
    assert L.lib().fgqa_decode_bf16_noalloc(ctypes.byref(b), s) == L.FGQA_ERR_INVALID_ARGUMENT
    torch.cuda.synchronize()
