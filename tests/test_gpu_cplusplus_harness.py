"""The C++ bench harness (tests/cplusplus/bench_flash_gqa.cpp) on the GPU: it
drives the C++ drop-in entry points at the BASELINE configurations, checks
them against the CPU oracle (max-abs 2e-2, mean-abs 2e-3, LSE 1e-3) and
reports GPU us / GB/s / TFLOPS, the roofline fraction and the CPU reference
time with its thread count.  The binary is built by __graft_entry__.build()
(make -C tests/cplusplus); a missing binary fails the test."""
import json
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cplusplus", "bin", "bench_flash_gqa")


def _run(configs, iters, timeout):
    assert os.path.isfile(BIN), f"{BIN} is not built (make -C tests/cplusplus)"
    print(f"C++ harness configs {configs}", flush=True)
    r = subprocess.run([BIN, "--configs", configs, "--iters", str(iters), "--warmup", "3", "--threads", "16"],
                       capture_output=True, text=True, timeout=timeout)
    print(r.stdout, r.stderr, flush=True)
    rows = [json.loads(line) for line in r.stdout.splitlines() if line.startswith("{")]
    return r.returncode, rows


def test_harness_decode_and_prefill_configs():
    rc, rows = _run("1,2,4", 10, 240)
    assert rc == 0
    assert [row["config"] for row in rows] == [1, 2, 4]
    for row in rows:
        assert row["pass"] is True
        assert row["roofline"]["frac"] > 0 and row["cpu_s"] > 0 and row["cpu_threads"] == 16
        assert row["max_abs"] <= 2e-2 and row["mean_abs"] <= 2e-3
    assert rows[0]["kv_bytes"] == 2 * 2 * 512 * 2 * 128 * 2
    assert rows[1]["kv_bytes"] == 1006632960
    assert rows[2]["flops"] == 68719476736 and rows[2]["lse_max_abs"] <= 1e-3


def test_harness_ragged_and_long_prefill_configs():
    rc, rows = _run("3,5", 5, 600)
    assert rc == 0
    assert [row["config"] for row in rows] == [3, 5]
    for row in rows:
        assert row["pass"] is True
    assert rows[1]["cpu_sample"].startswith("batch 0")
