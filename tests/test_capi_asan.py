"""The C-ABI validation tests (test_capi_cpu.py) under AddressSanitizer, on the CPU.

The library is rebuilt with its host code instrumented (build.py --asan: ``-Xarch_host -fsanitize=address``;
the device code is unchanged and never runs here) and loaded in a child process through SAGEATTN_MI355X_LIB,
with clang's ASan runtime preloaded.  Every validation path of the entry points -- the argument checks, the
stride and 32-bit limit arithmetic, the split planner, the error-message formatting -- then runs with
out-of-bounds and use-after-free detection on; any report aborts the child and fails this test.
"""
import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(REPO, "sageattention-rdna3_amd"))
import build as sage_build  # noqa: E402


def _stale(lib):
    if not os.path.exists(lib):
        return True
    t = os.path.getmtime(lib)
    srcs = [os.path.join(sage_build.CSRC, f) for f in os.listdir(sage_build.CSRC)]
    srcs += [os.path.join(sage_build.INCLUDE, f) for f in os.listdir(sage_build.INCLUDE)]
    return any(os.path.getmtime(f) > t for f in srcs)


@pytest.fixture(scope="module")
def asan_env():
    try:
        runtime = sage_build.asan_runtime()
    except RuntimeError as e:
        pytest.skip(str(e))
    if _stale(sage_build.ASAN_LIB):
        sage_build.build_asan()
    env = dict(os.environ)
    env.update(LD_PRELOAD=runtime, SAGEATTN_MI355X_LIB=sage_build.ASAN_LIB,
               ASAN_OPTIONS="detect_leaks=0:alloc_dealloc_mismatch=0:halt_on_error=1:abort_on_error=1")
    return env


def test_library_is_instrumented(asan_env):
    out = subprocess.run(["nm", "-D", "--undefined-only", sage_build.ASAN_LIB], capture_output=True, text=True,
                         check=True).stdout
    assert "__asan_report_load" in out and "__asan_report_store" in out
    probe = ("import ctypes, os; ctypes.CDLL(os.environ['SAGEATTN_MI355X_LIB']); "
             "print(sum('libclang_rt.asan' in ln for ln in open('/proc/self/maps')))")
    r = subprocess.run([sys.executable, "-c", probe], env=asan_env, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    assert int(r.stdout.strip().splitlines()[-1]) > 0, "ASan runtime not mapped"


def test_capi_validation_under_asan(asan_env):
    r = subprocess.run([sys.executable, "-m", "pytest", os.path.join(REPO, "tests", "test_capi_cpu.py"), "-q",
                        "-p", "no:cacheprovider", "-m", "not gpu"],
                       cwd=REPO, env=asan_env, capture_output=True, text=True, timeout=900)
    tail = (r.stdout + r.stderr)[-4000:]
    assert r.returncode == 0, tail
    assert "ERROR: AddressSanitizer" not in r.stderr, tail
    assert " passed" in r.stdout, tail
