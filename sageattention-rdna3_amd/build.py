"""Build the gfx950 C-ABI library ``sageattention/libsage_mi355x.so`` in-tree.

Usage: ``python sageattention-rdna3_amd/build.py [-v]``.  Cross-compiles for
gfx950 with hipcc; no GPU is needed.  Every call recompiles.

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


def _run(cmd, verbose):
    if verbose:
        print(" ".join(shlex.quote(c) for c in cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = (res.stdout or "") + (res.stderr or "")
    # hipcc's host pass does not know the device-only feature; that warning is expected
    lines = [ln for ln in out.splitlines() if "packed-fp32-ops" not in ln]
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n" + "\n".join(lines))
    if verbose and lines:
        print("\n".join(lines), flush=True)


def build(verbose: bool = False) -> str:
    """Compile every source for gfx950 and link the shared library; returns its path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    objs = []
    for src, extra in SOURCES:
        obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
        cmd = [HIPCC, *COMMON, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
        if src.endswith(".cpp"):
            cmd[1:1] = ["-x", "hip"]
        _run(cmd, verbose)
        objs.append(obj)
    tmp = LIB_PATH + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp], verbose)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
