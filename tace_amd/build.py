"""Build libtace_hip.so (gfx950) in-tree.

``python -m tace_amd.build`` (or ``__graft_entry__.build()``) regenerates the
tensor-product kernels from ``csrc/codegen.py`` and compiles
``csrc/tace_hip.hip`` with hipcc into ``tace_amd/_lib/libtace_hip.so``.
Packed-FP32 VALU instructions are disabled for every HIP translation unit.
"""

from __future__ import annotations

import os
import subprocess
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "_lib")
LIB = os.path.join(LIBDIR, "libtace_hip.so")
ROOT = os.path.dirname(HERE)

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics", "-Wno-unused-variable", "-Wno-unused-parameter",
]


def generate() -> str:
    sys.path.insert(0, ROOT)
    from tace_amd.csrc import codegen

    dst = os.path.join(CSRC, "gen", "tp_kernels.inc")
    os.makedirs(os.path.dirname(dst), exist_ok=True)
    codegen.emit_all(dst)
    return dst


def build(verbose: bool = True) -> str:
    t0 = time.time()
    generate()
    os.makedirs(LIBDIR, exist_ok=True)
    tmp = LIB + ".tmp"
    cmd = [HIPCC, *HIP_FLAGS, os.path.join(CSRC, "tace_hip.hip"), "-o", tmp]
    if verbose:
        print("[tace_amd.build]", " ".join(cmd), flush=True)
    subprocess.check_call(cmd, cwd=CSRC)
    os.replace(tmp, LIB)
    if verbose:
        print(f"[tace_amd.build] {LIB} in {time.time() - t0:.1f}s", flush=True)
    return LIB


if __name__ == "__main__":
    build()
