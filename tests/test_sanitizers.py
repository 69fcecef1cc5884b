"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer (CPU).

The reference has no sanitizer runs at all; this build checks its own host C
and C++ code with them.  The host half of ``libfa2.so`` is parameter
validation, plan making and workspace sizing: every ``fa2_*`` entry point
runs it before any HIP call.  The oracle is plain C.  Both are built
a second time with ASan + UBSan on the host code:

* ``python triton-kernels_amd/build.py --sanitize`` writes
  ``triton-kernels_amd/_san/libfa2.so`` (``__graft_entry__.build()`` does it too);
* ``make -C oracle sanitize`` writes ``oracle/_san/liboracle.so``.

The test runs the CPU suites that drive those two libraries (C-ABI checks,
oracle vs golden fixtures, closed forms and planted mistakes) in a child
Python process with the clang ASan runtime preloaded and the libraries
selected by ``FA2_LIBRARY`` / ``FA2_ORACLE_LIBRARY``.  Any sanitizer report
fails it: UBSan is built not to recover, and ASan halts on its first error.
Leak checking is off: the Python interpreter and torch keep allocations
alive until exit by design.
"""

from __future__ import annotations

import glob
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN_FA2 = os.path.join(ROOT, "triton-kernels_amd", "_san", "libfa2.so")
SAN_ORACLE = os.path.join(ROOT, "oracle", "_san", "liboracle.so")
SUITES = ["tests/test_abi.py", "tests/test_oracle.py", "tests/test_oracle_decode.py"]


def _asan_runtime():
    found = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    return found[-1] if found else None


def _instrumented(path: str) -> bool:
    """The library imports the sanitizer runtime's entry points (it was
    really built with both sanitizers, not just copied under _san/)."""
    r = subprocess.run(["nm", "-D", "--undefined-only", path], capture_output=True, text=True)
    return "__asan_init" in r.stdout and "__ubsan_handle_" in r.stdout


def _missing():
    if _asan_runtime() is None:
        return "clang ASan runtime not found under /opt/rocm/llvm"
    if not os.path.exists(SAN_FA2):
        return "sanitized libfa2.so not built (python triton-kernels_amd/build.py --sanitize)"
    if not os.path.exists(SAN_ORACLE):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "sanitize"], check=True)
    return None


@pytest.mark.timeout(900)
def test_host_code_under_asan_and_ubsan():
    why = _missing()
    if why:
        pytest.skip(why)
    assert _instrumented(SAN_FA2), SAN_FA2
    assert _instrumented(SAN_ORACLE), SAN_ORACLE
    # ASan's runtime must come first among the preloaded libraries; any the
    # environment already preloads stay after it.  Every GPU is hidden: the
    # sanitized child must not start the HIP runtime, and its plans then use
    # the fixed CU-count fallback on any host.
    pre = os.environ.get("LD_PRELOAD", "")
    env = dict(os.environ,
               LD_PRELOAD=_asan_runtime() + (":" + pre if pre else ""),
               HIP_VISIBLE_DEVICES="-1",
               CUDA_VISIBLE_DEVICES="-1",
               ROCR_VISIBLE_DEVICES="-1",
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1",
               FA2_LIBRARY=SAN_FA2,
               FA2_ORACLE_LIBRARY=SAN_ORACLE)
    # the child reports which libraries it actually loaded, then runs the suites
    probe = ("import sys, os; sys.path[:0] = [%r, %r]; "
             "from kernels import _fa2; import oracle; "
             "L = _fa2.lib(); oracle.round_scalar(1.0, 'f16'); "
             "maps = open('/proc/self/maps').read(); "
             "print('LOADED', %r in maps, %r in maps)"
             % (ROOT, os.path.join(ROOT, "triton-kernels_amd"), SAN_FA2, SAN_ORACLE))
    r = subprocess.run([sys.executable, "-c", probe], cwd=ROOT, env=env, capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 0 and "LOADED True True" in r.stdout, (r.stdout + r.stderr)[-4000:]
    r = subprocess.run([sys.executable, "-m", "pytest", *SUITES, "-m", "not gpu", "-q", "-x",
                        "-p", "no:cacheprovider", "-p", "no:xdist"],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=880)
    out = r.stdout + r.stderr
    assert "ERROR: AddressSanitizer" not in out, out[-6000:]
    assert "runtime error:" not in out, out[-6000:]
    assert r.returncode == 0, out[-6000:]
    assert " passed" in out, out[-2000:]
