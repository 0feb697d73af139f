"""Build libtace_hip.so (gfx950) in-tree.

``python -m tace_amd.build`` (or ``__graft_entry__.build()``) regenerates the
tensor-product kernels from ``csrc/codegen.py`` (one translation unit per
variant), compiles every translation unit with hipcc in parallel and links
``tace_amd/_lib/libtace_hip.so``.  Packed-FP32 VALU instructions are disabled
for every HIP translation unit.  Objects whose source and headers are older
than the object are reused unless ``force=True``.
"""

from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
GEN = os.path.join(CSRC, "gen")
OBJ = os.path.join(CSRC, "_obj")
LIBDIR = os.path.join(HERE, "_lib")
LIB = os.path.join(LIBDIR, "libtace_hip.so")
ROOT = os.path.dirname(HERE)

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics", "-Wno-unused-variable", "-Wno-unused-parameter",
]


def generate():
    sys.path.insert(0, ROOT)
    from tace_amd.csrc import codegen

    return codegen.emit_all(GEN)


def _compile(src: str, force: bool) -> str:
    obj = os.path.join(OBJ, os.path.splitext(os.path.basename(src))[0] + ".o")
    deps = [src, os.path.join(CSRC, "common.h"), os.path.join(CSRC, "bf16x3.h"), os.path.join(CSRC, "tece_common.h"),
            os.path.join(ROOT, "include", "tace_hip.h")]
    deps += glob.glob(os.path.join(GEN, "*.inc"))
    if not force and os.path.exists(obj) and os.path.getmtime(obj) >= max(os.path.getmtime(d) for d in deps):
        return obj
    tmp = obj + ".tmp.o"
    subprocess.run([HIPCC, *HIP_FLAGS, "-c", src, "-o", tmp], cwd=CSRC, check=True, stdout=subprocess.PIPE,
                   stderr=subprocess.STDOUT)
    os.replace(tmp, obj)
    return obj


def build(verbose: bool = True, force: bool = True, jobs: int = 0) -> str:
    t0 = time.time()
    # the longest translation units first
    srcs = [os.path.join(CSRC, n) for n in ("tece_rotin.hip", "tece_rotout.hip", "tece_ace.hip", "linear.hip",
                                            "tace_hip.hip", "tece_score.hip", "tece_wigner.hip", "mlp.hip",
                                            "so2_gemm.hip")] + generate()
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    jobs = jobs or min(16, os.cpu_count() or 4)
    if verbose:
        print(f"[tace_amd.build] {len(srcs)} translation units, {jobs} jobs: {HIPCC} {' '.join(HIP_FLAGS)}", flush=True)
    with cf.ThreadPoolExecutor(jobs) as ex:
        futs = {ex.submit(_compile, s, force): s for s in srcs}
        objs = []
        for f in cf.as_completed(futs):
            try:
                objs.append(f.result())
            except subprocess.CalledProcessError as e:
                sys.stderr.write(e.stdout.decode(errors="replace"))
                raise
    objs.sort()
    tmp = LIB + ".tmp"
    subprocess.check_call([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp])
    os.replace(tmp, LIB)
    if verbose:
        print(f"[tace_amd.build] {LIB} in {time.time() - t0:.1f}s", flush=True)
    return LIB


if __name__ == "__main__":
    build(force="--incremental" not in sys.argv)
