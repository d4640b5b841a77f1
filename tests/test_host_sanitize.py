"""Host code under AddressSanitizer + UndefinedBehaviorSanitizer, on the CPU.

* The oracle: `make -C oracle sanitize` builds oracle.c with
  oracle/sanitize_main.c, which runs every oracle function on small ragged
  shapes with exactly sized heap buffers (plus cross-checks between the
  restatements); the binary must print "ok" with no sanitizer report.
* The library's host code: `make -C simplang_amd/runtime sanitize` builds
  libsimp_hip_san.so with the host side instrumented (device code unchanged).
  The CPU tests that drive it -- every entry point's descriptor checks and
  error paths, the checkpoint header, tokenizer and sampler -- run again in a
  child process that loads it (SIMP_HIP_LIB) with the compiler's ASan runtime
  preloaded; any report aborts that process.
"""
import glob
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN_ENV = {"ASAN_OPTIONS": "halt_on_error=1:abort_on_error=0",
           "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1"}


def test_oracle_under_sanitizers():
    if shutil.which("gcc") is None and shutil.which("cc") is None:
        pytest.skip("no C compiler")
    subprocess.run(["make", "-C", os.path.join(ROOT, "oracle"), "sanitize"], check=True,
                   capture_output=True)
    env = dict(os.environ, OMP_NUM_THREADS="4", **SAN_ENV)
    env["ASAN_OPTIONS"] += ":detect_leaks=1"
    r = subprocess.run([os.path.join(ROOT, "oracle", "_build", "oracle_san")], env=env,
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-4000:]
    assert r.stdout.strip() == "ok", r.stdout
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr, r.stderr[-4000:]


def test_library_host_code_under_sanitizers():
    san = os.path.join(ROOT, "simplang_amd", "libsimp_hip_san.so")
    if not os.path.exists(san):
        pytest.skip("libsimp_hip_san.so not built (make -C simplang_amd/runtime sanitize)")
    rt = sorted(glob.glob("/opt/rocm/lib/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not rt:
        pytest.skip("the compiler's ASan runtime is not installed")
    env = dict(os.environ, SIMP_HIP_LIB=san, LD_PRELOAD=rt[-1], **SAN_ENV)
    env["ASAN_OPTIONS"] += ":detect_leaks=0"   # the interpreter itself is not leak-clean
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-m", "not gpu",
                        "-p", "no:cacheprovider",
                        os.path.join(ROOT, "tests", "test_abi.py"),
                        os.path.join(ROOT, "tests", "test_model_io.py")],
                       env=env, cwd=ROOT, capture_output=True, text=True, timeout=600)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert " passed" in r.stdout and "AddressSanitizer" not in out and "runtime error" not in out
