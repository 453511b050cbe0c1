"""The library's host code built with g++ under AddressSanitizer and
UndefinedBehaviorSanitizer, no recovery:
  - the argument validation and launch planning every C-ABI entry runs before
    it touches the device (cuda_llm_ops_amd/csrc/host/fgqa_plan.cpp), driven by
    tests/host/test_plan.cpp: the benchmark shapes against plans worked out by
    hand, each rejection rule at its boundary, sizes up to INT_MAX / INT64_MAX,
    and 200 000 fuzzed argument sets per entry point;
  - the C++ operator layer (src/cplusplus/FlashGQA/flash_gqa.cpp) over a
    recording stand-in of the C ABI (tests/host/test_operator_layer.cpp).
A signed overflow, out-of-bounds access or other undefined behaviour ends the
program with a sanitizer report.  CPU only: no GPU, no HIP."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HOST = os.path.join(ROOT, "cuda_llm_ops_amd", "csrc", "host")


SAN_FLAGS = ["-std=c++17", "-O1", "-g", "-Wall", "-Wextra", "-Werror", "-fsanitize=address,undefined",
             "-fno-sanitize-recover=all", "-fno-omit-frame-pointer"]


def _build_and_run(tmp_path, name, sources):
    exe = tmp_path / name
    subprocess.run(["g++", *SAN_FLAGS, "-I" + os.path.join(ROOT, "include"),
                    "-I" + os.path.join(ROOT, "include", "cplusplus"), "-I" + HOST, *sources, "-o", str(exe)],
                   check=True, timeout=300)
    env = dict(os.environ)
    # (verify_asan_link_order=0: a library the environment preloads may come first)
    env["ASAN_OPTIONS"] = "detect_leaks=1:abort_on_error=1:verify_asan_link_order=0"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1:halt_on_error=1"
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-4000:]
    assert "0 failed" in r.stdout
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_plan_under_asan_and_ubsan(tmp_path):
    _build_and_run(tmp_path, "test_plan",
                   [os.path.join(HOST, "fgqa_plan.cpp"), os.path.join(ROOT, "tests", "host", "test_plan.cpp")])


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_operator_layer_under_asan_and_ubsan(tmp_path):
    """src/cplusplus/FlashGQA/flash_gqa.cpp over a recording stand-in of the C
    ABI that validates with the planner above (tests/host/test_operator_layer.cpp)."""
    _build_and_run(tmp_path, "test_operator_layer",
                   [os.path.join(ROOT, "src", "cplusplus", "FlashGQA", "flash_gqa.cpp"),
                    os.path.join(HOST, "fgqa_plan.cpp"),
                    os.path.join(ROOT, "tests", "host", "test_operator_layer.cpp")])


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_sanitizer_build_catches_a_planted_overflow(tmp_path):
    """The same flags on a program with a signed overflow: the run must fail
    with a UBSan report, so a clean run above means something."""
    src = tmp_path / "planted.cpp"
    src.write_text("#include <climits>\nint main(int argc, char**) { int x = INT_MAX - 1; x += argc + 1; "
                   "return x == 0; }\n")
    exe = tmp_path / "planted"
    subprocess.run(["g++", "-std=c++17", "-O1", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                    str(src), "-o", str(exe)], check=True, timeout=300)
    env = dict(os.environ)
    env["ASAN_OPTIONS"] = "verify_asan_link_order=0"
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60, env=env)
    assert r.returncode != 0 and "runtime error" in r.stderr
