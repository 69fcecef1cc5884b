"""Build ``kernels/libfa2.so`` (hipcc, gfx950) and the PyTorch-ROCm launch
extension ``kernels/fa2_torch*.so`` in-tree.

Usage: ``python triton-kernels_amd/build.py`` (or ``build()`` from Python).
libfa2.so is a plain C ABI (include/fa2.h); fa2_torch is the launch half of
flash_attention_v2 in C++ (csrc/fa2_torch.cpp), linked against libfa2.so.
"""

from __future__ import annotations

import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")
SOURCES = [os.path.join(HERE, "csrc", "fa2_fwd.hip")]  # includes every csrc/*.h
OUT_DIR = os.path.join(HERE, "kernels")
OUT = os.path.join(OUT_DIR, "libfa2.so")
EXT_NAME = "fa2_torch"

FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Wl,-soname,libfa2.so",
    "-I" + os.path.join(ROOT, "include"),
    # packed fp32 VALU ops are kept out of all device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd, verbose, what):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (r.stderr or "").splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"{what} failed ({r.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def ext_path() -> str:
    return os.path.join(OUT_DIR, EXT_NAME + sysconfig.get_config_var("EXT_SUFFIX"))


def build_ext(verbose: bool = False) -> str:
    """g++ against torch's headers and libraries (no JIT cache), rpath to
    libfa2.so next to it."""
    import torch
    import torch.utils.cpp_extension as ce

    inc = ce.include_paths(device_type="cuda") + [sysconfig.get_paths()["include"],
                                                  os.path.join(ROOT, "include")]
    libdirs = ce.library_paths(device_type="cuda")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    out = ext_path()
    tmp = out + ".tmp"
    cmd = ([CXX, "-O2", "-std=c++17", "-shared", "-fPIC", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
            f"-DTORCH_EXTENSION_NAME={EXT_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H",
            "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1"]
           + ["-I" + d for d in inc]
           + [os.path.join(HERE, "csrc", "fa2_torch.cpp"), "-o", tmp]
           + ["-L" + d for d in libdirs] + ["-L" + OUT_DIR]
           + ["-lfa2", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
              "-ltorch_python", "-Wl,-rpath,$ORIGIN"]
           + ["-Wl,-rpath," + d for d in libdirs])
    _run(cmd, verbose, "g++ (fa2_torch)")
    os.replace(tmp, out)
    return out


# Host-sanitized build of the same library (AddressSanitizer + UBSan on the
# host code only: parameter checks, plans, workspace sizing).  Its device code
# is the regular build's; it is for CPU tests that call the host half of the C
# ABI under the clang ASan runtime (tests/test_sanitizers.py), never for GPU runs.
SAN_DIR = os.path.join(HERE, "_san")
SAN_OUT = os.path.join(SAN_DIR, "libfa2.so")
SAN_HOST_FLAGS = [
    "-Xarch_host", "-fsanitize=address",
    "-Xarch_host", "-fsanitize=undefined",
    "-Xarch_host", "-fno-sanitize-recover=undefined",
    "-Xarch_host", "-fno-omit-frame-pointer",
    "-Xarch_host", "-g",
    "-Xarch_host", "-O1",
]


def build(verbose: bool = False, sanitize: bool = False) -> str:
    """Compile libfa2.so and the launch extension; with ``sanitize`` also the
    host-sanitized libfa2.so (in parallel with the regular one)."""
    tmp = OUT + ".tmp"
    san = None
    if sanitize:
        os.makedirs(SAN_DIR, exist_ok=True)
        san_cmd = [HIPCC] + FLAGS + SAN_HOST_FLAGS + SOURCES + ["-o", SAN_OUT + ".tmp"]
        if verbose:
            print(" ".join(san_cmd), flush=True)
        san = subprocess.Popen(san_cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    try:
        _run([HIPCC] + FLAGS + SOURCES + ["-o", tmp], verbose, "hipcc")
        os.replace(tmp, OUT)
    finally:
        log = san.communicate()[0] if san is not None else ""
    # Neither of these is needed at run time (the wrapper falls back to the C
    # ABI through ctypes; the sanitizer test skips without its library), so a
    # failure is reported and the build goes on.
    try:
        build_ext(verbose)
    except Exception as e:  # noqa: BLE001 - missing torch headers, compiler errors
        print(f"warning: launch extension not built: {e}", file=sys.stderr, flush=True)
    if san is not None:
        if san.returncode != 0:
            print(f"warning: sanitized host build failed ({san.returncode}):\n{log}",
                  file=sys.stderr, flush=True)
        else:
            os.replace(SAN_OUT + ".tmp", SAN_OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True, sanitize="--sanitize" in sys.argv[1:]))
