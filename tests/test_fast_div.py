"""The magic-number division of cuda_llm_ops_amd/csrc/hip/fgqa_device.h
(make_fast_div on the host, fast_div on host and device), which the prefill
kernels use to map a work rank to its (query block, head group, kv head,
batch).  A host program built with hipcc against the header divides, for
every divisor 1..2048 and a spread of larger ones, numerators at the edges
of each quotient step and up to 2^31 - 1 by the fast path and by `/`, and
prints every disagreement; there must be none.  A magic number one too
small (planted in the test program) is shown to disagree, so the check can
fail."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

SRC = r'''
#include <cstdio>
#include <cstdint>
#include "fgqa_device.h"
using fgqa::FastDiv;
static long long bad = 0, checked = 0;
static void check(int d, int x, bool planted) {
    FastDiv f = fgqa::make_fast_div(d);
    if (planted) f.mul -= 1;
    const int q = fgqa::fast_div(x, f);
    ++checked;
    if (q != x / d) { if (bad < 5) std::printf("MISMATCH d=%d x=%d q=%d\n", d, x, q); ++bad; }
}
static void sweep(int d, bool planted) {
    const int top = 2147483647;
    int xs[] = {0, 1, d - 1, d, d + 1, 2 * d - 1, 2 * d, top, top - 1, top - d, top / d * d, top / d * d - 1,
                1 << 30, (1 << 30) - 1, 123456789, 987654321, 65535, 65536};
    for (int x : xs) if (x >= 0) check(d, x, planted);
    // numerators around the multiples of d spread over the whole range
    for (int k = 1; k < 64; ++k) {
        const long long base = (long long)top / 64 * k / d * d;
        for (int e = -1; e <= 1; ++e) if (base + e >= 0 && base + e <= top) check(d, (int)(base + e), planted);
    }
}
int main() {
    for (int d = 1; d <= 2048; ++d) sweep(d, false);
    const int big[] = {4095, 4097, 65535, 65537, 1000003, (1 << 20) + 7, (1 << 30) - 1, 1 << 30, (1 << 30) + 1,
                       2147483646, 2147483647};
    for (int d : big) sweep(d, false);
    std::printf("checked %lld bad %lld\n", checked, bad);
    long long before = bad;
    for (int d = 3; d <= 2048; ++d) sweep(d, true);
    std::printf("planted bad %lld\n", bad - before);
    return 0;
}
'''


@pytest.fixture(scope="module")
def fast_div_run(tmp_path_factory):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not available")
    d = tmp_path_factory.mktemp("fastdiv")
    (d / "t.hip").write_text(SRC)
    exe = d / "t"
    subprocess.run([HIPCC, "-O2", "-std=c++17", "--offload-arch=gfx950",
                    "-I", os.path.join(ROOT, "cuda_llm_ops_amd", "csrc", "hip"), str(d / "t.hip"), "-o", str(exe)],
                   check=True, capture_output=True)
    return subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout


def test_fast_div_matches_division(fast_div_run):
    lines = fast_div_run.strip().split("\n")
    summary = [l for l in lines if l.startswith("checked")][0].split()
    assert int(summary[1]) > 100000
    assert int(summary[3]) == 0, fast_div_run


def test_planted_bad_magic_is_caught(fast_div_run):
    planted = [l for l in fast_div_run.strip().split("\n") if l.startswith("planted")][0].split()
    assert int(planted[2]) > 0
