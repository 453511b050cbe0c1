"""Benchmark of the MI355X flash-GQA hot path.

Default (the driver's contract): BASELINE config 2, GQA decode at B=60,
S=4096, Hq=128, Hkv=8, D=128, bf16 in/out, fp32 accumulation, inputs resident
in HBM.  One "step" = one decode over the whole batch.  Prints ONE JSON line:
value = decode KV-read throughput in GB/s (decimal), with the roofline of the
decode kernel against 8 TB/s HBM.  Beside it: the other BASELINE configs (1
and 3 decode, 4 and 5 causal prefill, each with its roofline: TFLOPS against
2.5 PFLOP/s bf16 dense MFMA for prefill), the paged-KV decode (bf16 and fp8
caches) at config 3's lengths, the sliding-window, MLA and sparse-index
prefill and the backward passes; max-abs / mean-abs of each BASELINE
config's output against the CPU oracle (sampled batches or rows, outside the
timed regions); and the CPU oracle timed on a bounded sample of the decode
workload (`cpu_baseline`) and on all of config 4 (`cpu_baseline_prefill`).

    python bench.py [--steps K] [--warmup W] [--split-tokens N] [--no-cpu] [--no-configs] [--no-check]

Only one GPU is used: --gpus N with N > 1 exits with a message.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, 8 TB/s
BF16_PEAK_TFLOPS = 2516.6      # 256 CU x 2.4 GHz x 4096 dense bf16 FLOP/clk/CU
PEAK_SCLK_MHZ = 2400.0         # the shader clock that figure assumes
SCALE = 1.0 / math.sqrt(128)

# HBM bytes per launch of the dominant kernel, from rocprofv3 --pmc FETCH_SIZE and
# WRITE_SIZE runs of `bench.py --mode decode|prefill` (KiB per dispatch x 1024).
# FETCH_SIZE is scaled by 2.0: on this GPU it reads 524,302 KiB for a 1 GiB
# buffer copy whose WRITE_SIZE reads the exact 1,048,576 KiB.  The summaries
# with the commands are profiles/*_hbm_traffic.md.  Re-measure when a kernel
# changes.
# HBM bytes per dispatch of the dominant kernel, from rocprofv3 FETCH_SIZE (x 2.0,
# the factor a 1 GiB copy calibrates) + WRITE_SIZE, on the current kernels
# (decode_split_kernel with KV head pairs; the prefill's re-measurement read
# 83,495,424 B, within 0.06 % of the figure below).
TRAFFIC_BYTES = {
    "decode_cfg2": 1010671543,   # = Q+K+V+O (1,010,565,120 B) + 0.01 %
    "prefill_cfg4": 83448320,    # Q+O+LSE 32.25 MiB, K/V per XCD, split units' partials written and read back
}

DECODE_CONFIGS = {
    1: dict(B=2, S=512, Hq=16, Hkv=2, ragged=False, sigma=1.0),
    2: dict(B=60, S=4096, Hq=128, Hkv=8, ragged=False, sigma=1.0),
    3: dict(B=64, S=32768, Hq=64, Hkv=8, ragged=True, sigma=1.0),
}
PREFILL_CONFIGS = {
    4: dict(B=1, S=4096, Hq=16, Hkv=1, sigma=1.0),
    5: dict(B=4, S=16384, Hq=32, Hkv=8, sigma=0.5),
}


def _normal(shape, seed, sigma, dev):
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    x = torch.randn(shape, generator=g, device=dev, dtype=torch.float32)
    if sigma != 1.0:
        x.mul_(sigma)
    return x.to(torch.bfloat16)


# The auxiliary measurements each follow an idle gap (the CPU baseline, the
# previous mode's setup): they warm up for at least this long.  After an idle
# second, config 4's prefill ran 73-85 us per launch in its first 10 ms, 70-71
# us at 25 ms and settled at 68.0 us from about 60 ms on (the same in three
# trials on one MI355X), so a shorter warm-up times the clock's ramp, not the
# kernel.
AUX_WARM_MS = 150.0


def _time_calls(fn, steps, warmup, min_warm_ms=0.0):
    """Times `steps` calls issued back to back between two HIP events on
    torch's current stream (the stream every launch of the library goes to),
    with a synchronize on both sides: the total (ms) over the timed region, so
    total / steps is the average launch duration.  Then the same number of
    calls again, each between events of its own, for the sorted per-call
    durations (median and minimum; those events add a gap per call, so they
    are not used for the average).  Before the timed region: `warmup`
    untimed calls, then more until `min_warm_ms` of them have run (an idle GPU
    takes milliseconds to bring its clock back up)."""
    import time
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    if min_warm_ms > 0:
        t0 = time.perf_counter()
        while (time.perf_counter() - t0) * 1e3 < min_warm_ms:
            for _ in range(4):
                fn()
            torch.cuda.synchronize()
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record()
    for _ in range(steps):
        fn()
    t_end.record()
    torch.cuda.synchronize()
    total = t_start.elapsed_time(t_end)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for a, b in evs:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    per = sorted(a.elapsed_time(b) for a, b in evs)
    # then `steps` calls more between two clock samples, for _clock_fields
    global _LAST_SCLK_MHZ
    _LAST_SCLK_MHZ = _sclk_mhz(fn, steps)
    return total, per


# Shader clock (MHz) averaged over the last `_time_calls` call's extra pass
# (None when the two samples ran on different XCDs or the entry is missing).
_LAST_SCLK_MHZ = None


def _sclk_mhz(fn, n, samples=1024):
    """Average shader clock over n back-to-back calls: fgqa_clock_sample
    before and after them on torch's current stream (the launch stream)
    reads, from `samples` workgroups spread over the CUs, each CU's
    shader-clock counter and the 100 MHz real-time counter; the median over
    the CUs sampled both times."""
    import ctypes

    import torch

    from cuda_llm_ops_amd import _lib
    buf = torch.zeros((2, samples, 3), dtype=torch.int64, device="cuda")
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    L = _lib.lib()
    if L.fgqa_clock_sample(ctypes.c_void_p(buf[0].data_ptr()), samples, s) != 0:
        return None
    for _ in range(n):
        fn()
    if L.fgqa_clock_sample(ctypes.c_void_p(buf[1].data_ptr()), samples, s) != 0:
        return None
    torch.cuda.synchronize()
    first = {}
    for t, r, cu in buf[0].tolist():
        first.setdefault(cu, (t, r))
    mhz = []
    for t, r, cu in buf[1].tolist():
        if cu in first and r > first[cu][1] and t > first[cu][0]:
            mhz.append((t - first[cu][0]) / (r - first[cu][1]) * 100.0)
            del first[cu]
    if not mhz:
        return None
    mhz.sort()
    return round(mhz[len(mhz) // 2], 1)


def _clock_fields(tflops):
    """The MFMA roofline's clock fields: the shader clock the kernel sustained
    over its measurement, and the fraction of the dense peak scaled to that
    clock (the 2,516.6 TFLOP/s figure assumes 2.4 GHz)."""
    if not _LAST_SCLK_MHZ:
        return {"sclk_mhz": None, "frac_at_sclk": None}
    return {"sclk_mhz": _LAST_SCLK_MHZ,
            "frac_at_sclk": round(tflops / (BF16_PEAK_TFLOPS * _LAST_SCLK_MHZ / PEAK_SCLK_MHZ), 4)}


def _decode_setup(cfg, dev, seed=2):
    import numpy as np
    import torch
    B, S, Hq, Hkv = cfg["B"], cfg["S"], cfg["Hq"], cfg["Hkv"]
    q = _normal((B, Hq, 128), seed, cfg["sigma"], dev)
    k = _normal((B, S, Hkv, 128), seed + 1, cfg["sigma"], dev)
    v = _normal((B, S, Hkv, 128), seed + 2, cfg["sigma"], dev)
    lens = None
    if cfg["ragged"]:
        rng = np.random.default_rng(seed)
        lens = (1 + rng.integers(0, S, size=B)).astype(np.int32)
    sl = None if lens is None else torch.from_numpy(lens).to(dev)
    valid_tokens = B * S if lens is None else int(lens.sum())
    kv_bytes = 2 * valid_tokens * Hkv * 128 * 2
    return q, k, v, sl, lens, kv_bytes


def bench_decode(cfg_id, steps, warmup, split_tokens, dev):
    import torch

    import cuda_llm_ops_amd as fg
    cfg = DECODE_CONFIGS[cfg_id]
    q, k, v, sl, lens, kv_bytes = _decode_setup(cfg, dev)
    out = torch.empty_like(q)
    n_ws = fg.decode_workspace_bytes(cfg["B"], cfg["S"], cfg["Hq"], cfg["Hkv"], split_tokens=split_tokens,
                                     ragged=cfg["ragged"])
    ws = torch.empty(max(n_ws, 256), dtype=torch.uint8, device=dev)

    # validated once; each step is one call of the C ABI on torch's current stream
    step = fg.prepare_decode(q, k, v, SCALE, out=out, seqlens=sl, split_tokens=split_tokens, workspace=ws)

    total_ms, per = _time_calls(step, steps, warmup)
    ms_step = total_ms / steps
    avg_launch_ms = total_ms / steps
    qo_bytes = 2 * cfg["B"] * cfg["Hq"] * 128 * 2
    # no workspace: one split per (batch, KV head) stream, no combine pass
    kernel = ("decode_split_kernel, one split per (batch, KV head), KV head pairs per workgroup, no combine"
              if n_ws == 0 else
              "decode_list_kernel + decode_combine_kernel (device-built ragged work list, split-KV)"
              if cfg["ragged"] else "decode_split_kernel + decode_combine_kernel (split-KV)")
    return dict(cfg=cfg, q=q, k=k, v=v, lens=lens, out=out, kv_bytes=kv_bytes, qo_bytes=qo_bytes,
                ms_step=ms_step, avg_launch_ms=avg_launch_ms, median_ms=per[len(per) // 2], min_ms=per[0],
                kernel=kernel, sclk_mhz=_LAST_SCLK_MHZ)


def _host_u16(t):
    import numpy as np
    import torch
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _err(out_u16, ref_u16):
    """max-abs and mean-abs of a bf16 output against the oracle's (the parity
    figures of the reference harness, test_decode_flash_gqa.cu:311-319)."""
    import numpy as np

    import oracle
    d = np.abs(oracle.bf16_to_f32(out_u16).astype(np.float64) - oracle.bf16_to_f32(ref_u16))
    return float(d.max()), float(d.sum()), int(d.size)


def decode_check(res, batches, threads):
    """GPU decode output (the last timed step's) against the C oracle on the
    listed batches, all heads; outside the timed region."""
    import numpy as np

    import oracle
    mx, sm, n = 0.0, 0.0, 0
    for b in batches:
        L = res["cfg"]["S"] if res["lens"] is None else int(res["lens"][b])
        ref, _ = oracle.decode(_host_u16(res["q"][b:b + 1]), _host_u16(res["k"][b:b + 1, :L]),
                               _host_u16(res["v"][b:b + 1, :L]), SCALE, nthreads=threads, with_lse=False)
        m, s, c = _err(_host_u16(res["out"][b:b + 1]), ref)
        mx, sm, n = max(mx, m), sm + s, n + c
    return dict(max_abs=mx, mean_abs=sm / n, tol={"max_abs": 2e-2, "mean_abs": 2e-3},
                sample=f"batches {list(batches)}, all heads, against the C oracle")


def decode_block(cfg_id, steps, warmup, dev, check_batches, threads):
    """A decode config beside the default line: timing, HBM roofline and the
    oracle check (check_batches None: the shortest and longest sequences and
    two fixed ones)."""
    import numpy as np
    res = bench_decode(cfg_id, steps, warmup, 0, dev)
    if check_batches is None:
        check_batches = sorted({int(np.argmin(res["lens"])), int(np.argmax(res["lens"])), 7, 40})
    cfg = res["cfg"]
    achieved = res["kv_bytes"] / (res["avg_launch_ms"] * 1e-3) / 1e9
    block = dict(
        config=f"GQA decode B={cfg['B']} S={'<=' if cfg['ragged'] else ''}{cfg['S']} Hq={cfg['Hq']} "
               f"Hkv={cfg['Hkv']} D=128{' ragged lengths' if cfg['ragged'] else ''} (BASELINE config {cfg_id})",
        us_avg=round(res["avg_launch_ms"] * 1e3, 2), us_median=round(res["median_ms"] * 1e3, 2),
        us_min=round(res["min_ms"] * 1e3, 2), GBs=round(achieved, 2),
        roofline={"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                  "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": TRAFFIC_BYTES.get(f"decode_cfg{cfg_id}"),
                  "algorithmic_bytes": res["kv_bytes"]},
        error=decode_check(res, check_batches, threads))
    if cfg_id == 1:
        block["note"] = "1 MiB of KV stays in the caches: a latency figure, not an HBM-bound one"
    return block


def prefill_check(t, row_blocks, threads):
    """GPU prefill output against the C oracle on row blocks (b, r0, r1) of
    every query head; outside the timed region."""
    mx, sm, n = 0.0, 0.0, 0
    import oracle
    for b, r0, r1 in row_blocks:
        ref, _ = oracle.prefill(_host_u16(t["q"][b:b + 1, r0:r1]), _host_u16(t["k"][b:b + 1, :r1]),
                                _host_u16(t["v"][b:b + 1, :r1]), SCALE, causal=True, q_offset=r0,
                                nthreads=threads)
        m, s, c = _err(_host_u16(t["out"][b:b + 1, r0:r1]), ref)
        mx, sm, n = max(mx, m), sm + s, n + c
    return dict(max_abs=mx, mean_abs=sm / n, tol={"max_abs": 2e-2, "mean_abs": 2e-3})


def cpu_baseline_prefill(t, threads):
    """The C oracle (OpenMP over batch x head x query block) on all of BASELINE
    config 4, timed on the host cores; its output also gives config 4's
    max-abs / mean-abs over every row and head."""
    import oracle
    qh, kh, vh = _host_u16(t["q"]), _host_u16(t["k"]), _host_u16(t["v"])
    B, S, Hq = qh.shape[0], qh.shape[1], qh.shape[2]
    t0 = time.perf_counter()
    ref, _ = oracle.prefill(qh, kh, vh, SCALE, causal=True, nthreads=threads)
    elapsed = time.perf_counter() - t0
    flops = B * Hq * 2 * S * S * (128 + 128) // 2
    m, s, c = _err(_host_u16(t["out"]), ref)
    cpu = dict(value=round(flops / elapsed / 1e12, 5), unit="TFLOP/s", cores=threads, kind="port",
               host_cores=_host_cores(),
               sample=f"the whole config 4 prefill (all {S} rows, {Hq} heads), {elapsed:.2f} s on {threads} "
                      f"OpenMP threads; FLOPs counted as on the GPU (causal-halved)")
    err = dict(max_abs=m, mean_abs=s / c, tol={"max_abs": 2e-2, "mean_abs": 2e-3},
               sample="every row and head, against the C oracle")
    return cpu, err


def bench_prefill(cfg_id, steps, warmup, dev, keep=None):
    import torch

    import cuda_llm_ops_amd as fg
    cfg = PREFILL_CONFIGS[cfg_id]
    B, S, Hq, Hkv = cfg["B"], cfg["S"], cfg["Hq"], cfg["Hkv"]
    q = _normal((B, S, Hq, 128), 4, cfg["sigma"], dev)
    k = _normal((B, S, Hkv, 128), 5, cfg["sigma"], dev)
    v = _normal((B, S, Hkv, 128), 6, cfg["sigma"], dev)
    out = torch.empty_like(q)
    lse = torch.empty((B, Hq, S), dtype=torch.float32, device=dev)

    step = fg.prepare_prefill(q, k, v, SCALE, out=out, lse=lse, causal=True)
    kernel = fg.prefill_kernel_name(q, k, v, causal=True)   # what AUTO launches, as the library reports it

    total_ms, per = _time_calls(step, steps, warmup, min_warm_ms=AUX_WARM_MS)
    # the reference's causal-halved count (test_flash_gqa_kernel.py:282-301)
    flops = B * Hq * 2 * S * S * (128 + 128) // 2
    avg = total_ms / steps
    tflops = flops / (avg * 1e-3) / 1e12
    if keep is not None:
        keep.update(q=q, k=k, v=v, out=out, lse=lse)
    return dict(config=f"causal prefill B={B} S={S} Hq={Hq} Hkv={Hkv} D=128 (BASELINE config {cfg_id})",
                us_avg=round(avg * 1e3, 2), us_median=round(per[len(per) // 2] * 1e3, 2),
                us_min=round(per[0] * 1e3, 2),
                roofline={"bound": "mfma", "achieved": round(tflops, 2), "peak": BF16_PEAK_TFLOPS,
                          "unit": "TFLOP/s", "frac": round(tflops / BF16_PEAK_TFLOPS, 4), **_clock_fields(tflops),
                          "traffic": TRAFFIC_BYTES.get(f"prefill_cfg{cfg_id}"),
                          "kernel": kernel,
                          "algorithmic_flops": flops})


def _host_cores():
    """The host's logical CPUs and those this process may run on (the CPU
    baselines use min(these, 16) OpenMP threads: `cores`)."""
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = os.cpu_count() or 1
    return {"logical": os.cpu_count(), "usable": usable}


def cpu_baseline_decode(res, budget_s=12.0):
    """Time the CPU oracle (OpenMP C restatement of the reference's CPU decode)
    on whole sequences of the same inputs, cycling through the batch until
    ~budget_s of CPU work (or one full pass, whichever is longer)."""
    import numpy as np
    import torch

    import oracle
    cfg = res["cfg"]

    def host(t):
        return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)

    threads = min(os.cpu_count() or 1, 16)
    done_bytes = 0
    elapsed = 0.0
    nb = 0
    B = cfg["B"]
    while nb < B or elapsed < budget_s:
        bi = nb % B
        qh, kh, vh = host(res["q"][bi:bi + 1]), host(res["k"][bi:bi + 1]), host(res["v"][bi:bi + 1])
        sl = None if res["lens"] is None else res["lens"][bi:bi + 1]
        t0 = time.perf_counter()
        oracle.decode(qh, kh, vh, SCALE, seqlens=sl, nthreads=threads, with_lse=False)
        elapsed += time.perf_counter() - t0
        n_tok = cfg["S"] if sl is None else int(sl[0])
        done_bytes += 2 * n_tok * cfg["Hkv"] * 128 * 2
        nb += 1
    return dict(value=round(done_bytes / elapsed / 1e9, 3), unit="GB/s", cores=threads, kind="port",
                host_cores=_host_cores(),
                sample=f"{nb} sequence decodes ({nb / B:.2f} passes over the {B}-sequence workload, all heads, "
                       f"all tokens), {elapsed:.1f} s on {threads} OpenMP threads")


def hbm_copy(steps, warmup, dev, nbytes=1 << 30):
    """Plain device-to-device copy of `nbytes` (torch's copy kernel): the
    calibration point for the HBM byte counters and the practical read+write
    bandwidth of the box."""
    import torch
    src = torch.empty(nbytes // 2, dtype=torch.bfloat16, device=dev).normal_()
    dst = torch.empty_like(src)
    total_ms, per = _time_calls(lambda: dst.copy_(src), steps, warmup, min_warm_ms=AUX_WARM_MS)
    avg = total_ms / steps
    return dict(bytes_read=nbytes, bytes_written=nbytes, us_avg=avg * 1e3,
                read_plus_write_GBs=2 * nbytes / (avg * 1e-3) / 1e9)


def bench_paged(cfg_id, steps, warmup, dev, page_size=16, kv="bf16"):
    """Decode over a paged KV cache (block table, pages in random order) with
    the lengths of a BASELINE decode config; KV bytes count the valid tokens
    in the cache's own dtype (fp8: 1 byte per element)."""
    import numpy as np
    import torch

    import cuda_llm_ops_amd as fg
    cfg = DECODE_CONFIGS[cfg_id]
    B, S, Hq, Hkv = cfg["B"], cfg["S"], cfg["Hq"], cfg["Hkv"]
    q, k, v, sl, lens, _ = _decode_setup(cfg, dev)
    if sl is None:
        sl = torch.full((B,), S, dtype=torch.int32, device=dev)
        lens = np.full(B, S, dtype=np.int32)
    max_pages = S // page_size
    n = B * max_pages
    perm = torch.from_numpy(np.random.default_rng(11).permutation(n).astype(np.int64)).to(dev)
    table = perm.view(B, max_pages).to(torch.int32)
    k_scale = v_scale = 1.0
    if kv == "fp8":
        k_scale, v_scale = 6.0 / 448, 6.0 / 448
        k = (k.float() / k_scale).clamp_(-448, 448).to(torch.float8_e4m3fn)
        v = (v.float() / v_scale).clamp_(-448, 448).to(torch.float8_e4m3fn)
    kc = torch.empty((n, page_size, Hkv, 128), dtype=k.dtype, device=dev)
    vc = torch.empty_like(kc)
    kc[perm] = k.reshape(n, page_size, Hkv, 128)
    vc[perm] = v.reshape(n, page_size, Hkv, 128)
    del k, v
    out = torch.empty_like(q)
    n_ws = fg.paged_decode_workspace_bytes(B, S, Hq, Hkv, page_size)
    ws = torch.empty(max(n_ws, 256), dtype=torch.uint8, device=dev)
    step = fg.prepare_decode_paged(q, kc, vc, table, sl, SCALE, k_scale=k_scale, v_scale=v_scale, out=out,
                                   workspace=ws)
    total_ms, per = _time_calls(step, steps, warmup, min_warm_ms=AUX_WARM_MS)
    elem = 1 if kv == "fp8" else 2
    kv_bytes = 2 * int(lens.sum()) * Hkv * 128 * elem
    avg = total_ms / steps
    gbs = kv_bytes / (avg * 1e-3) / 1e9
    return dict(config=f"paged decode, BASELINE config {cfg_id} lengths, page {page_size}, {kv} KV",
                us_avg=round(avg * 1e3, 2), kv_bytes=kv_bytes, GBs=round(gbs, 1),
                frac_hbm=round(gbs / HBM_PEAK_GBS, 4),
                tokens_per_s=round(float(lens.sum()) / (avg * 1e-3), 0))


def bench_swa(steps, warmup, dev, window=512):
    """Sliding-window (+ sink) prefill at the reference's SWA benchmark shape
    (README: B=1, S=4096, Hq=16, Hkv=1, D=128, window 512)."""
    import torch

    import cuda_llm_ops_amd as fg
    B, S, Hq, Hkv = 1, 4096, 16, 1
    q = _normal((B, S, Hq, 128), 8, 1.0, dev)
    k = _normal((B, S, Hkv, 128), 9, 1.0, dev)
    v = _normal((B, S, Hkv, 128), 10, 1.0, dev)
    sink = torch.rand(Hq, generator=torch.Generator().manual_seed(11)).to(dev) + 1e-6
    out = torch.empty_like(q)
    lse = torch.empty((B, Hq, S), dtype=torch.float32, device=dev)
    step = fg.prepare_prefill(q, k, v, SCALE, out=out, lse=lse, causal=True, window_size=window, sink=sink)
    total_ms, per = _time_calls(step, steps, warmup, min_warm_ms=AUX_WARM_MS)
    # the reference's count (test_flash_swa_kernel.py:318-337)
    flops = B * Hq * 2 * S * window * (128 + 128)
    avg = total_ms / steps
    tflops = flops / (avg * 1e-3) / 1e12
    return dict(config=f"sliding-window prefill with sink, B={B} S={S} Hq={Hq} Hkv={Hkv} D=128 window={window}",
                us_avg=round(avg * 1e3, 2), us_min=round(per[0] * 1e3, 2),
                roofline={"bound": "mfma", "achieved": round(tflops, 2), "peak": BF16_PEAK_TFLOPS,
                          "unit": "TFLOP/s", "frac": round(tflops / BF16_PEAK_TFLOPS, 4), **_clock_fields(tflops),
                          "algorithmic_flops": flops})


def bench_mla(steps, warmup, dev):
    """MLA prefill (Q/K head dim 192, V/O 128, causal) at the reference's MLA
    benchmark shape (README: B=1, S=4096, Hq=Hkv=16)."""
    import math

    import torch

    import cuda_llm_ops_amd as fg
    B, S, Hq, Hkv, Dqk, Dv = 1, 4096, 16, 16, 192, 128
    q = _normal((B, S, Hq, Dqk), 12, 1.0, dev)
    k = _normal((B, S, Hkv, Dqk), 13, 1.0, dev)
    v = _normal((B, S, Hkv, Dv), 14, 1.0, dev)
    out = torch.empty((B, S, Hq, Dv), dtype=torch.bfloat16, device=dev)
    lse = torch.empty((B, Hq, S), dtype=torch.float32, device=dev)
    step = fg.prepare_prefill(q, k, v, 1.0 / math.sqrt(Dqk), out=out, lse=lse, causal=True)
    total_ms, per = _time_calls(step, steps, warmup, min_warm_ms=AUX_WARM_MS)
    # the reference's causal-halved count (test_flash_mla_kernel.py:282-301)
    flops = B * Hq * 2 * S * S * (Dqk + Dv) // 2
    avg = total_ms / steps
    tflops = flops / (avg * 1e-3) / 1e12
    return dict(config=f"MLA causal prefill B={B} S={S} Hq={Hq} Hkv={Hkv} Dqk={Dqk} Dv={Dv}",
                us_avg=round(avg * 1e3, 2), us_median=round(per[len(per) // 2] * 1e3, 2),
                us_min=round(per[0] * 1e3, 2),
                roofline={"bound": "mfma", "achieved": round(tflops, 2), "peak": BF16_PEAK_TFLOPS,
                          "unit": "TFLOP/s", "frac": round(tflops / BF16_PEAK_TFLOPS, 4), **_clock_fields(tflops),
                          "algorithmic_flops": flops})


def _sparse_indices(B, Hkv, S, nsparse, seed, dev, recent=16):
    """Index lists shaped like the reference test's
    (examples/python/Triton/test_flash_sgqa_kernel.py:30-94): row i has
    min(nsparse, i + 1) entries, its `recent` latest causal keys, then keys drawn
    from the older causal range (here with replacement), then -1 padding."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    pos = torch.arange(S, device=dev, dtype=torch.int64)[:, None]
    slot = torch.arange(nsparse, device=dev, dtype=torch.int64)[None, :]
    n_valid = torch.clamp(pos + 1, max=nsparse)
    n_recent = torch.clamp(n_valid, max=recent)
    start = pos - n_recent + 1
    rnd = (torch.rand((B, Hkv, S, nsparse), generator=g, device=dev) * start.clamp(min=1)).long()
    idx = torch.where(slot < n_recent, start + slot, rnd)
    idx = torch.where(slot < n_valid, idx, torch.full_like(idx, -1))
    return idx.to(torch.int32).contiguous()


def bench_sparse(steps, warmup, dev):
    """Sparse-index prefill at the reference's sparse-GQA benchmark shape
    (README: B=1, S=32768, Hq=16, Hkv=1, D=128, 512 entries per row, causal),
    with index lists shaped like the reference test's (recent 16 + random)."""
    import torch

    import cuda_llm_ops_amd as fg
    B, S, Hq, Hkv, n = 1, 32768, 16, 1, 512
    q = _normal((B, S, Hq, 128), 15, 1.0, dev)
    k = _normal((B, S, Hkv, 128), 16, 1.0, dev)
    v = _normal((B, S, Hkv, 128), 17, 1.0, dev)
    idx = _sparse_indices(B, Hkv, S, n, 18, dev)
    out = torch.empty_like(q)
    lse = torch.empty((B, Hq, S), dtype=torch.float32, device=dev)
    step = fg.prepare_sparse_prefill(q, k, v, idx, SCALE, out=out, lse=lse, causal=True)
    total_ms, per = _time_calls(step, steps, warmup, min_warm_ms=AUX_WARM_MS)
    # the reference's count (test_flash_sgqa_kernel.py:488-506)
    flops = 2 * B * Hq * S * n * (128 + 128)
    # K and V rows gathered per launch (one 256-byte K row and V row per list entry,
    # shared by the 16 query heads); served mostly from L2 / MALL
    gathered = B * Hkv * S * n * 2 * 256
    avg = total_ms / steps
    tflops = flops / (avg * 1e-3) / 1e12
    return dict(config=f"sparse-index prefill B={B} S={S} Hq={Hq} Hkv={Hkv} D=128 entries={n} causal",
                us_avg=round(avg * 1e3, 2), us_median=round(per[len(per) // 2] * 1e3, 2),
                us_min=round(per[0] * 1e3, 2),
                gathered_bytes=gathered, gather_GBs=round(gathered / (avg * 1e-3) / 1e9, 1),
                roofline={"bound": "mfma", "achieved": round(tflops, 2), "peak": BF16_PEAK_TFLOPS,
                          "unit": "TFLOP/s", "frac": round(tflops / BF16_PEAK_TFLOPS, 4), **_clock_fields(tflops),
                          "algorithmic_flops": flops})


def bench_backward(cfg_id, steps, warmup, dev):
    """Prefill backward (dQ, dK, dV) of a causal forward at a BASELINE prefill
    shape; one step = every launch of fgqa_prefill_backward_bf16."""
    import torch

    import cuda_llm_ops_amd as fg
    cfg = PREFILL_CONFIGS[cfg_id]
    B, S, Hq, Hkv = cfg["B"], cfg["S"], cfg["Hq"], cfg["Hkv"]
    q = _normal((B, S, Hq, 128), 4, cfg["sigma"], dev)
    k = _normal((B, S, Hkv, 128), 5, cfg["sigma"], dev)
    v = _normal((B, S, Hkv, 128), 6, cfg["sigma"], dev)
    do = _normal((B, S, Hq, 128), 7, 1.0, dev)
    out, lse = fg.flash_gqa_forward_bshd(q, k, v, SCALE, causal=True)
    n_ws = fg.backward_workspace_bytes(B, S, S, Hq, Hkv)
    ws = torch.empty(max(n_ws, 256), dtype=torch.uint8, device=dev)
    step = fg.prepare_backward(q, k, v, out, lse, do, SCALE, causal=True, workspace=ws)

    total_ms, per = _time_calls(step, steps, warmup, min_warm_ms=AUX_WARM_MS)
    # the reference's count, QK + dP + dQ + dK + dV causal-halved
    # (test_flash_gqa_kernel.py:344-363); the kernels execute 7 such GEMMs
    # (S and dP are recomputed by the dQ pass), 7/5 of it
    flops = B * Hq * 2 * S * S * (3 * 128 + 2 * 128) // 2
    avg = total_ms / steps
    tflops = flops / (avg * 1e-3) / 1e12
    return dict(config=f"causal prefill backward B={B} S={S} Hq={Hq} Hkv={Hkv} D=128 (BASELINE config {cfg_id} shape)",
                us_avg=round(avg * 1e3, 2), us_median=round(per[len(per) // 2] * 1e3, 2),
                us_min=round(per[0] * 1e3, 2),
                roofline={"bound": "mfma", "achieved": round(tflops, 2), "peak": BF16_PEAK_TFLOPS,
                          "unit": "TFLOP/s", "frac": round(tflops / BF16_PEAK_TFLOPS, 4), **_clock_fields(tflops),
                          "kernel": "bwd_dq(_split) + bwd_dkdv + bwd_dkdv_reduce (whole step)",
                          "algorithmic_flops": flops, "executed_mfma_flops": flops * 7 // 5})


def bench_swa_backward(steps, warmup, dev, window=512):
    """Sliding-window (+ sink) prefill backward at the reference's SWA benchmark
    shape (README: B=1, S=4096, Hq=16, Hkv=1, D=128, window 512), fed the GPU
    forward's O and sink-adjusted LSE; one step = every launch of
    fgqa_prefill_backward_bf16."""
    import torch

    import cuda_llm_ops_amd as fg
    B, S, Hq, Hkv = 1, 4096, 16, 1
    q = _normal((B, S, Hq, 128), 15, 1.0, dev)
    k = _normal((B, S, Hkv, 128), 16, 1.0, dev)
    v = _normal((B, S, Hkv, 128), 17, 1.0, dev)
    do = _normal((B, S, Hq, 128), 18, 1.0, dev)
    sink = torch.rand(Hq, generator=torch.Generator().manual_seed(19)).to(dev) + 1e-6
    out, lse = fg.flash_gqa_forward_bshd(q, k, v, SCALE, causal=True, window_size=window, sink=sink)
    n_ws = fg.backward_workspace_bytes(B, S, S, Hq, Hkv, window_size=window)
    ws = torch.empty(max(n_ws, 256), dtype=torch.uint8, device=dev)
    step = fg.prepare_backward(q, k, v, out, lse, do, SCALE, causal=True, workspace=ws, window_size=window)
    total_ms, per = _time_calls(step, steps, warmup, min_warm_ms=AUX_WARM_MS)
    # the reference's count, QK + dP + dQ + dK + dV over the window
    # (test_flash_swa_kernel.py:400-420); the kernels execute 7 such GEMMs
    flops = B * Hq * 2 * S * window * (3 * 128 + 2 * 128)
    avg = total_ms / steps
    tflops = flops / (avg * 1e-3) / 1e12
    return dict(config=f"sliding-window prefill backward, B={B} S={S} Hq={Hq} Hkv={Hkv} D=128 window={window}",
                us_avg=round(avg * 1e3, 2), us_median=round(per[len(per) // 2] * 1e3, 2),
                us_min=round(per[0] * 1e3, 2),
                roofline={"bound": "mfma", "achieved": round(tflops, 2), "peak": BF16_PEAK_TFLOPS,
                          "unit": "TFLOP/s", "frac": round(tflops / BF16_PEAK_TFLOPS, 4), **_clock_fields(tflops),
                          "kernel": "bwd_dq(_split) + bwd_dkdv + bwd_dkdv_reduce (whole step)",
                          "algorithmic_flops": flops, "executed_mfma_flops": flops * 7 // 5})


def bench_mla_backward(steps, warmup, dev):
    """MLA prefill backward (Q/K head dim 192, V/O 128, causal) at the
    reference's MLA benchmark shape (README: B=1, S=4096, Hq=Hkv=16), fed the
    GPU MLA forward's O and LSE; one step = every launch of
    fgqa_prefill_backward_bf16."""
    import math

    import torch

    import cuda_llm_ops_amd as fg
    B, S, Hq, Hkv, Dqk, Dv = 1, 4096, 16, 16, 192, 128
    scale = 1.0 / math.sqrt(Dqk)
    q = _normal((B, S, Hq, Dqk), 20, 1.0, dev)
    k = _normal((B, S, Hkv, Dqk), 21, 1.0, dev)
    v = _normal((B, S, Hkv, Dv), 22, 1.0, dev)
    do = _normal((B, S, Hq, Dv), 23, 1.0, dev)
    out, lse = fg.flash_gqa_forward_bshd(q, k, v, scale, causal=True)
    n_ws = fg.backward_workspace_bytes(B, S, S, Hq, Hkv, head_dim=Dqk, head_dim_v=Dv)
    ws = torch.empty(max(n_ws, 256), dtype=torch.uint8, device=dev)
    step = fg.prepare_backward(q, k, v, out, lse, do, scale, causal=True, workspace=ws)
    total_ms, per = _time_calls(step, steps, warmup, min_warm_ms=AUX_WARM_MS)
    # the reference's causal-halved count, QK + dP + dQ + dK + dV
    # (test_flash_mla_kernel.py:344-363); the kernels execute S and dP twice
    flops = B * Hq * 2 * S * S * (3 * Dqk + 2 * Dv) // 2
    avg = total_ms / steps
    tflops = flops / (avg * 1e-3) / 1e12
    return dict(config=f"MLA causal prefill backward, B={B} S={S} Hq={Hq} Hkv={Hkv} Dqk={Dqk} Dv={Dv}",
                us_avg=round(avg * 1e3, 2), us_median=round(per[len(per) // 2] * 1e3, 2),
                us_min=round(per[0] * 1e3, 2),
                roofline={"bound": "mfma", "achieved": round(tflops, 2), "peak": BF16_PEAK_TFLOPS,
                          "unit": "TFLOP/s", "frac": round(tflops / BF16_PEAK_TFLOPS, 4), **_clock_fields(tflops),
                          "kernel": "bwd_dq<192> + bwd_dkdv<192> (whole step)",
                          "algorithmic_flops": flops})


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=150)
    ap.add_argument("--split-tokens", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-backward", action="store_true")
    ap.add_argument("--no-paged", action="store_true")
    ap.add_argument("--no-swa", action="store_true")
    ap.add_argument("--no-swa-backward", action="store_true")
    ap.add_argument("--no-mla-backward", action="store_true")
    ap.add_argument("--no-mla", action="store_true")
    ap.add_argument("--no-sparse", action="store_true")
    ap.add_argument("--page-size", type=int, default=16, help="with --mode paged")
    ap.add_argument("--kv", choices=["bf16", "fp8"], default="bf16", help="with --mode paged")
    ap.add_argument("--no-configs", action="store_true",
                    help="leave out BASELINE configs 1, 3 and 5 (reported by default)")
    ap.add_argument("--no-check", action="store_true", help="leave out the oracle checks (max-abs / mean-abs)")
    ap.add_argument("--mode", choices=["bench", "decode", "paged", "prefill", "swa", "mla", "sparse", "backward",
                                       "swa_backward", "mla_backward", "copy"],
                    default="bench",
                    help="decode/prefill/copy: run only that workload (for profiling) and print its timing")
    ap.add_argument("--config", type=int, default=0,
                    help="with --mode decode/prefill/backward: BASELINE config id")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path (--gpus must be 1)", file=sys.stderr)
        sys.exit(2)

    import torch
    import cuda_llm_ops_amd  # noqa: F401  (fails loudly if libfgqa.so is missing)
    dev = torch.device("cuda:0")

    if args.mode == "copy":
        print(json.dumps({"mode": "copy", **hbm_copy(args.steps, args.warmup, dev)}), flush=True)
        return
    if args.mode == "decode":
        r = bench_decode(args.config or 2, args.steps, args.warmup, args.split_tokens, dev)
        print(json.dumps({"mode": "decode", "config": args.config or 2, "us_avg": r["avg_launch_ms"] * 1e3,
                          "kv_bytes": r["kv_bytes"], "GBs": r["kv_bytes"] / (r["avg_launch_ms"] * 1e-3) / 1e9}),
              flush=True)
        return
    if args.mode == "prefill":
        print(json.dumps({"mode": "prefill", **bench_prefill(args.config or 4, args.steps, args.warmup, dev)}),
              flush=True)
        return
    if args.mode == "paged":
        print(json.dumps({"mode": "paged", **bench_paged(args.config or 3, args.steps, args.warmup, dev,
                                                          args.page_size, args.kv)}), flush=True)
        return
    if args.mode == "sparse":
        print(json.dumps({"mode": "sparse", **bench_sparse(args.steps, args.warmup, dev)}), flush=True)
        return
    if args.mode == "mla":
        print(json.dumps({"mode": "mla", **bench_mla(args.steps, args.warmup, dev)}), flush=True)
        return
    if args.mode == "swa":
        print(json.dumps({"mode": "swa", **bench_swa(args.steps, args.warmup, dev)}), flush=True)
        return
    if args.mode == "backward":
        print(json.dumps({"mode": "backward", **bench_backward(args.config or 4, args.steps, args.warmup, dev)}),
              flush=True)
        return
    if args.mode == "swa_backward":
        print(json.dumps({"mode": "swa_backward", **bench_swa_backward(args.steps, args.warmup, dev)}), flush=True)
        return
    if args.mode == "mla_backward":
        print(json.dumps({"mode": "mla_backward", **bench_mla_backward(args.steps, args.warmup, dev)}), flush=True)
        return

    res = bench_decode(2, args.steps, args.warmup, args.split_tokens, dev)
    gbs = res["kv_bytes"] / (res["ms_step"] * 1e-3) / 1e9
    achieved = res["kv_bytes"] / (res["avg_launch_ms"] * 1e-3) / 1e9
    line = {
        "metric": "decode KV-read GB/s (% HBM peak); prefill TFLOPS (% bf16 MFMA peak)",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["ms_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1) bf16 (seeded torch.randn on the GPU), resident in HBM",
        "config": {"workload": "GQA decode, BASELINE config 2", "batch": 60, "seq_len": 4096,
                   "num_q_heads": 128, "num_kv_heads": 8, "head_dim": 128, "parallelism": "none (1 GPU)",
                   "split_tokens": args.split_tokens or "auto"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": TRAFFIC_BYTES.get("decode_cfg2"),
                     "kernel": res["kernel"], "algorithmic_bytes": res["kv_bytes"],
                     "avg_launch_us": round(res["avg_launch_ms"] * 1e3, 2),
                     "median_launch_us": round(res["median_ms"] * 1e3, 2),
                     "min_launch_us": round(res["min_ms"] * 1e3, 2), "sclk_mhz": res["sclk_mhz"]},
        "decode_all_tensor_GBs": round((res["kv_bytes"] + res["qo_bytes"]) / (res["ms_step"] * 1e-3) / 1e9, 2),
    }
    threads = min(os.cpu_count() or 1, 16)
    if not args.no_check:
        line["error"] = decode_check(res, (0, 29, 59), threads)
    keep4 = {}
    if not args.no_prefill:
        line["prefill"] = bench_prefill(4, args.steps, args.warmup, dev, keep=keep4)
    if not args.no_configs:
        line["decode_cfg1"] = decode_block(1, args.steps, args.warmup, dev, (0, 1), threads)
        line["decode_cfg3"] = decode_block(3, max(5, args.steps // 5), 2, dev, None, threads)
        keep5 = {}
        line["prefill_cfg5"] = bench_prefill(5, max(3, args.steps // 10), 2, dev, keep=keep5)
        if not args.no_check:
            S5, B5 = PREFILL_CONFIGS[5]["S"], PREFILL_CONFIGS[5]["B"]
            import numpy as np
            rng = np.random.default_rng(5)
            blocks = [(0, 0, 128), (0, S5 - 128, S5)]
            for b in range(B5):
                for r0 in sorted(rng.integers(0, S5 // 32, size=2) * 32):
                    blocks.append((b, int(r0), int(r0) + 32))
            line["prefill_cfg5"]["error"] = prefill_check(keep5, blocks, threads)
            line["prefill_cfg5"]["error"]["sample"] = (
                f"rows [0,128) and [{S5 - 128},{S5}) of batch 0 and two random 32-row blocks of every batch "
                f"({sum(r1 - r0 for _, r0, r1 in blocks)} rows x 32 heads), against the C oracle")
        del keep5
    if not args.no_paged:
        line["decode_paged"] = [bench_paged(3, max(5, args.steps // 5), 2, dev, 16, kv)
                                for kv in ("bf16", "fp8")]
    if not args.no_swa:
        line["swa"] = bench_swa(max(5, args.steps // 2), max(2, args.warmup // 2), dev)
    if not args.no_mla:
        line["mla"] = bench_mla(max(5, args.steps // 2), max(2, args.warmup // 2), dev)
    if not args.no_sparse:
        line["sparse"] = bench_sparse(max(5, args.steps // 5), 2, dev)
    if not args.no_backward:
        line["backward"] = bench_backward(4, max(5, args.steps // 2), max(2, args.warmup // 2), dev)
    if not args.no_swa_backward:
        line["swa_backward"] = bench_swa_backward(max(5, args.steps // 2), max(2, args.warmup // 2), dev)
    if not args.no_mla_backward:
        line["mla_backward"] = bench_mla_backward(max(5, args.steps // 5), 2, dev)
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline_decode(res)
        if keep4:
            line["cpu_baseline_prefill"], err4 = cpu_baseline_prefill(keep4, threads)
            if not args.no_check:
                line["prefill"]["error"] = err4
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
