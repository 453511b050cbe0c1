"""The CPU oracle's own tests (tests/test_oracle.py) against the oracle built
with AddressSanitizer and UndefinedBehaviorSanitizer (oracle/Makefile target
liboracle_san.so, gcc, host code only), in a subprocess that preloads the
sanitizer runtimes.  Any out-of-bounds access, use of freed memory, signed
overflow, misaligned access or other undefined behaviour in the oracle aborts
that run.  Leak checking is off: the Python interpreter itself keeps
allocations until exit."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _runtime(name):
    return subprocess.run(["gcc", f"-print-file-name={name}"], check=True, capture_output=True,
                          text=True).stdout.strip()


def test_oracle_tests_pass_under_asan_and_ubsan():
    subprocess.run(["make", "-C", os.path.join(ROOT, "oracle"), "-B", "liboracle_san.so"], check=True,
                   stdout=subprocess.DEVNULL)
    env = dict(os.environ)
    # the sanitizer runtimes first, then whatever the environment preloads already
    env["LD_PRELOAD"] = " ".join(x for x in (_runtime("libasan.so"), _runtime("libubsan.so"),
                                             os.environ.get("LD_PRELOAD", "")) if x)
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=1"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1:halt_on_error=1"
    env["FGQA_ORACLE_LIB"] = os.path.join(ROOT, "oracle", "liboracle_san.so")
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider",
                        os.path.join(ROOT, "tests", "test_oracle.py")],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-4000:]
    assert "passed" in r.stdout and "AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr
