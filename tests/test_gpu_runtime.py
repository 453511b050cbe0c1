"""GPU tests of the host runtime: the library-owned workspace under host
threads, and kernel attributes that are set per device.

Calls that pass no workspace share one per-device buffer that grows (freeing
the old one after draining the device).  A call holds the buffer's lock until
its kernels are launched, so host threads may call concurrently; these tests
drive decode and the prefill backward from several threads at once, with
sizes that make the buffer grow while other calls are in flight, and check
every result against a single-threaded run of the same inputs."""
import math
import threading

import pytest

pytestmark = pytest.mark.gpu

SCALE = 1.0 / math.sqrt(128)


def _fg():
    import cuda_llm_ops_amd as fg
    return fg


def test_internal_workspace_concurrent_host_threads(cuda):
    import torch
    fg = _fg()
    print("internal workspace: 4 threads x 12 decodes, growing split counts", flush=True)
    B, S, Hq, Hkv = 4, 4096, 32, 4
    g = torch.Generator(device=cuda)
    g.manual_seed(11)
    q = torch.randn(B, Hq, 128, device=cuda, generator=g).to(torch.bfloat16)
    k = torch.randn(B, S, Hkv, 128, device=cuda, generator=g).to(torch.bfloat16)
    v = torch.randn(B, S, Hkv, 128, device=cuda, generator=g).to(torch.bfloat16)
    # split sizes from large to small: each smaller split needs a larger workspace
    splits = [4096, 2048, 1024, 512, 256, 128]
    ref = {}
    for st in splits:
        ref[st] = fg.decode_flash_gqa_bshd(q, k, v, SCALE, split_tokens=st)
    torch.cuda.synchronize()
    errors = []
    results = []

    def worker(tid):
        try:
            for it in range(12):
                st = splits[(tid + it) % len(splits)]
                out = fg.decode_flash_gqa_bshd(q, k, v, SCALE, split_tokens=st)
                results.append((st, out))
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(repr(e))

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    torch.cuda.synchronize()
    assert not errors, errors
    assert len(results) == 48
    for st, out in results:
        assert torch.equal(out, ref[st]), f"split_tokens={st}: result differs from the single-threaded run"


def test_backward_concurrent_host_threads_internal_workspace(cuda):
    """Prefill backward from two threads with the library-owned workspace
    (different shapes, so the buffer grows while the other thread calls)."""
    import torch
    fg = _fg()
    print("internal workspace: backward from 2 threads", flush=True)
    shapes = [(1, 256, 8, 1), (1, 640, 16, 2)]
    inputs, refs = [], []
    g = torch.Generator(device=cuda)
    g.manual_seed(12)
    for B, S, Hq, Hkv in shapes:
        q = torch.randn(B, S, Hq, 128, device=cuda, generator=g).to(torch.bfloat16)
        k = torch.randn(B, S, Hkv, 128, device=cuda, generator=g).to(torch.bfloat16)
        v = torch.randn(B, S, Hkv, 128, device=cuda, generator=g).to(torch.bfloat16)
        do = torch.randn(B, S, Hq, 128, device=cuda, generator=g).to(torch.bfloat16)
        o, lse = fg.flash_gqa_forward_bshd(q, k, v, SCALE)
        inputs.append((q, k, v, o, lse, do))
        refs.append(fg.flash_gqa_backward_bshd(q, k, v, o, lse, do, SCALE))
    torch.cuda.synchronize()
    errors, results = [], []

    def worker(i):
        try:
            for _ in range(8):
                results.append((i, fg.flash_gqa_backward_bshd(*inputs[i][:6], SCALE)))
        except Exception as e:  # noqa: BLE001
            errors.append(repr(e))

    threads = [threading.Thread(target=worker, args=(i,)) for i in (0, 1, 0, 1)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    torch.cuda.synchronize()
    assert not errors, errors
    assert len(results) == 32
    for i, grads in results:
        for a, b in zip(grads, refs[i]):
            assert torch.equal(a, b)
