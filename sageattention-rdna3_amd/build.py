"""Build the gfx950 C-ABI library ``sageattention/libsage_mi355x.so`` and the compiled host layer of
``sageattn`` (``sageattention/_sage_host.so``, linked against it) in-tree.

Usage: ``python sageattention-rdna3_amd/build.py [-v] [--asan | --stamps]``.
Cross-compiles for gfx950 with hipcc; no GPU is needed.  Every call recompiles.
``--asan`` builds the host-AddressSanitizer variant of the library instead
(``_build_asan/``, for the C-ABI tests on the CPU); ``--stamps`` the variant
whose attention kernels record per-wave cycle stamps (``_build_stamps/``, read
through ``sage_stamps_read``).

Flags:
  * ``-Xclang -target-feature -Xclang -packed-fp32-ops`` on every device
    compile: no packed fp32 VALU instructions are generated;
  * ``-ffp-contract=off`` on the prologue (its quantiser is bit-exact IEEE
    fp32 and must not fuse multiply-adds); no ``-ffast-math`` anywhere;
  * ``-mllvm -amdgpu-mfma-vgpr-form`` on the attention kernel (MFMA
    accumulators in arch VGPRs, no per-tile AGPR copies).
"""
from __future__ import annotations

import os
import shlex
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(REPO, "include")
OUT_DIR = os.path.join(HERE, "sageattention")
LIB_NAME = "libsage_mi355x.so"
LIB_PATH = os.path.join(OUT_DIR, LIB_NAME)
BUILD_DIR = os.path.join(HERE, "_build")
ARCH = os.environ.get("SAGE_OFFLOAD_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
GXX = os.environ.get("CXX", "g++")
# the compiled host layer of sageattn (a Python extension module over the library's C ABI)
HOST_MODULE = "_sage_host"
HOST_SRC = "host_ops.cpp"
HOST_PATH = os.path.join(OUT_DIR, HOST_MODULE + ".so")

COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]

SOURCES = [
    ("capi.cpp", []),
    ("prologue.hip", ["-ffp-contract=off"]),
    # MFMA results in arch VGPRs: the softmax reads every S element and the
    # rare O rescale touches O; AGPR residency costs v_accvgpr copies per tile
    ("attn.hip", ["-mllvm", "-amdgpu-mfma-vgpr-form"]),
]


def _finish(cmd, proc, verbose):
    out, _ = proc.communicate()
    # hipcc's host pass does not know the device-only feature; that warning is expected
    lines = [ln for ln in (out or "").splitlines() if "packed-fp32-ops" not in ln]
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n" + "\n".join(lines))
    if verbose and lines:
        print("\n".join(lines), flush=True)


def _start(cmd, verbose):
    if verbose:
        print(" ".join(shlex.quote(c) for c in cmd), flush=True)
    return subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)


def _run(cmd, verbose):
    _finish(cmd, _start(cmd, verbose), verbose)


def _host_flags():
    """g++ flags of the compiled host layer: torch's headers and libraries (the module uses the torch
    C++ API for tensors and pybind11 for the Python call; no HIP code)."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension

    inc = cpp_extension.include_paths() + [sysconfig.get_paths()["include"], INCLUDE]
    libdir = cpp_extension.library_paths()[0]
    compile_flags = ["-O2", "-std=c++17", "-fPIC", "-Wall", f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
                     f"-DTORCH_EXTENSION_NAME={HOST_MODULE}", *[f"-I{i}" for i in inc]]
    link_flags = [f"-L{libdir}", "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python", f"-Wl,-rpath,{libdir}",
                  f"-L{OUT_DIR}", "-l:" + LIB_NAME, "-Wl,-rpath,$ORIGIN"]
    return compile_flags, link_flags


def build(verbose: bool = False) -> str:
    """Compile every source (the gfx950 library and the host module, in parallel), link the shared
    library, then the host module against it; returns the library's path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    jobs, objs = [], []
    for src, extra in SOURCES:
        obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
        cmd = [HIPCC, *COMMON, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
        if src.endswith(".cpp"):
            cmd[1:1] = ["-x", "hip"]
        jobs.append((cmd, _start(cmd, verbose)))
        objs.append(obj)
    host_cflags, host_lflags = _host_flags()
    host_obj = os.path.join(BUILD_DIR, HOST_SRC.replace(".cpp", ".o"))
    cmd = [GXX, *host_cflags, "-c", os.path.join(CSRC, HOST_SRC), "-o", host_obj]
    jobs.append((cmd, _start(cmd, verbose)))
    for cmd, proc in jobs:
        _finish(cmd, proc, verbose)
    tmp = LIB_PATH + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", f"-Wl,-soname,{LIB_NAME}", *objs, "-o", tmp], verbose)
    os.replace(tmp, LIB_PATH)
    tmp = HOST_PATH + ".tmp"
    _run([GXX, "-shared", host_obj, "-o", tmp, *host_lflags], verbose)
    os.replace(tmp, HOST_PATH)
    return LIB_PATH


# Host-side AddressSanitizer build of the C-ABI library: the same sources, with the host pass of every
# compile instrumented (the device code is built as usual), for running the C-ABI validation tests under
# ASan on the CPU.  Loaded through SAGEATTN_MI355X_LIB with the clang ASan runtime preloaded.
ASAN_DIR = os.path.join(HERE, "_build_asan")
ASAN_LIB = os.path.join(ASAN_DIR, "libsage_mi355x_asan.so")
ASAN_HOST = ["-O1", "-g", "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer"]


def asan_runtime() -> str:
    """The clang ASan runtime that the instrumented library links against."""
    out = subprocess.run([HIPCC, "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True)
    path = out.stdout.strip()
    if not os.path.isabs(path) or not os.path.exists(path):
        raise RuntimeError("clang ASan runtime (libclang_rt.asan-x86_64.so) not found")
    return path


def build_asan(verbose: bool = False) -> str:
    """Build ASAN_LIB (host code instrumented); returns its path."""
    os.makedirs(ASAN_DIR, exist_ok=True)
    jobs, objs = [], []
    common = [c for c in COMMON if c != "-O3"] + ASAN_HOST
    for src, extra in SOURCES:
        obj = os.path.join(ASAN_DIR, os.path.splitext(src)[0] + ".o")
        cmd = [HIPCC, *common, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
        if src.endswith(".cpp"):
            cmd[1:1] = ["-x", "hip"]
        jobs.append((cmd, _start(cmd, verbose)))
        objs.append(obj)
    for cmd, proc in jobs:
        _finish(cmd, proc, verbose)
    tmp = ASAN_LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Xarch_host", "-fsanitize=address", "-shared-libsan",
          *objs, "-o", tmp], verbose)
    os.replace(tmp, ASAN_LIB)
    return ASAN_LIB


# Cycle-stamps build of the library: the attention kernels compiled with SAGE_STAMPS=1 (per-wave s_memtime
# counts of item phases and key-loop steps, csrc/attn_body.inc) plus sage_stamps_read / sage_stamps_clear.
# Loaded through SAGEATTN_MI355X_LIB by a measurement script; never the product library.
STAMPS_DIR = os.path.join(HERE, "_build_stamps")
STAMPS_LIB = os.path.join(STAMPS_DIR, "libsage_mi355x_stamps.so")


def build_stamps(verbose: bool = False) -> str:
    """Build STAMPS_LIB; returns its path."""
    os.makedirs(STAMPS_DIR, exist_ok=True)
    jobs, objs = [], []
    for src, extra in SOURCES:
        obj = os.path.join(STAMPS_DIR, os.path.splitext(src)[0] + ".o")
        cmd = [HIPCC, *COMMON, *extra, "-DSAGE_STAMPS=1", "-c", os.path.join(CSRC, src), "-o", obj]
        if src.endswith(".cpp"):
            cmd[1:1] = ["-x", "hip"]
        jobs.append((cmd, _start(cmd, verbose)))
        objs.append(obj)
    for cmd, proc in jobs:
        _finish(cmd, proc, verbose)
    tmp = STAMPS_LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp], verbose)
    os.replace(tmp, STAMPS_LIB)
    return STAMPS_LIB


if __name__ == "__main__":
    if "--asan" in sys.argv:
        print(build_asan(verbose="-v" in sys.argv))
    elif "--stamps" in sys.argv:
        print(build_stamps(verbose="-v" in sys.argv))
    else:
        print(build(verbose="-v" in sys.argv))
