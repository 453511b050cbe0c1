"""The 64-bit index helpers of include/cplusplus/Utils/utils.h (the
reference's include/cplusplus/Utils/utils.cuh:14-44 computes them in `int`).

A small C++ program built with g++ against the header evaluates them at
indices that cross 2^31 elements -- a [128, 32768, 8, 128] KV cache, twice
BASELINE config 3's batch, and the byte offsets of config 3's own
[64, 32768, 8, 128] cache -- and the results are checked against exact
integer arithmetic.  The same indices evaluated with 32-bit wrap-around (the
reference's `int` formula) are shown to differ, so the test fails if the
header ever narrows back to 32 bits."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# (i1, i2, i3, i4) in a [*, D2, D3, D4] tensor
CASES_4D = [
    ((63, 32767, 7, 127), (32768, 8, 128)),      # config 3: the last element (2^31 - 1)
    ((64, 0, 0, 0), (32768, 8, 128)),            # batch 64 of a 128-sequence cache: exactly 2^31
    ((127, 32767, 7, 127), (32768, 8, 128)),     # its last element, 2^32 - 1
    ((100, 12345, 3, 77), (32768, 8, 128)),
    ((3, 16383, 31, 127), (16384, 32, 128)),     # config 5's Q/O [4, 16384, 32, 128]
]
CASES_3D = [
    ((63, 63, 127), (64, 128)),                  # config 3's Q [64, 64, 128]
    ((70000, 12, 100), (32768, 128)),            # 2.9e11
]
CASES_CEIL = [((1 << 33) + 1, 128), ((1 << 31) + 5, 4096), (127, 128), (0, 7)]


def _wrap32(x):
    x &= 0xFFFFFFFF
    return x - (1 << 32) if x >= (1 << 31) else x


def _ref32_4d(i, d):
    # the reference's int formula: i1*D2*D3*D4 + i2*D3*D4 + i3*D4 + i4, each step wrapping
    i1, i2, i3, i4 = i
    D2, D3, D4 = d
    return _wrap32(_wrap32(_wrap32(_wrap32(i1 * D2 * D3 * D4) + _wrap32(i2 * D3 * D4)) + i3 * D4) + i4)


@pytest.fixture(scope="module")
def helper_values(tmp_path_factory):
    lines = []
    for i, d in CASES_4D:
        lines.append(f'printf("%lld\\n", (long long)GET_1D_INDEX_FROM_4D({i[0]}, {i[1]}, {i[2]}, {i[3]}, '
                     f'{d[0]}, {d[1]}, {d[2]}));')
    for i, d in CASES_3D:
        lines.append(f'printf("%lld\\n", (long long)GET_1D_INDEX_FROM_3D({i[0]}, {i[1]}, {i[2]}, {d[0]}, {d[1]}));')
    for a, b in CASES_CEIL:
        lines.append(f'printf("%lld\\n", (long long)CEIL_DIV({a}LL, {b}));')
    src = ('#include <cstdio>\n#include "Utils/utils.h"\n'
           # constexpr evaluation at a 2^31-crossing index (config 3's byte offset of its last element)
           'static_assert(GET_1D_INDEX_FROM_4D(63, 32767, 7, 127, 32768, 8, 128) * 2 == 4294967294LL, "bytes");\n'
           'int main() {\n' + "\n".join(lines) + '\nreturn 0;\n}\n')
    d = tmp_path_factory.mktemp("utils")
    (d / "t.cpp").write_text(src)
    exe = d / "t"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", f"-I{ROOT}/include/cplusplus",
                    str(d / "t.cpp"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()
    return [int(x) for x in out]


def test_index_helpers_exact_past_2_31(helper_values):
    it = iter(helper_values)
    for (i1, i2, i3, i4), (D2, D3, D4) in CASES_4D:
        assert next(it) == ((i1 * D2 + i2) * D3 + i3) * D4 + i4
    for (i1, i2, i3), (D2, D3) in CASES_3D:
        assert next(it) == (i1 * D2 + i2) * D3 + i3
    for a, b in CASES_CEIL:
        assert next(it) == -(-a // b)


def test_index_helpers_differ_from_32_bit_arithmetic(helper_values):
    """The cases past 2^31 are exactly those the reference's int formula gets wrong."""
    for (i, d), got in zip(CASES_4D, helper_values):
        exact = ((i[0] * d[0] + i[1]) * d[1] + i[2]) * d[2] + i[3]
        assert got == exact
        assert (_ref32_4d(i, d) == exact) == (exact < (1 << 31))
