"""Compile libfmxq.so (the HIP kernels and the C ABI) in-tree for gfx950.

``python -m fastmlx_amd.build`` or ``fastmlx_amd.build.build()``.  Objects go to
``fastmlx_amd/_build/``; the shared library lands next to this file so it
travels with the source tree.  ``--diag`` (``build_diag()``) also builds the
time-line diagnostic program ``diag/qmv1_timeline``.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libfmxq.so")
ARCH = os.environ.get("FMXQ_ARCH", "gfx950")

# -packed-fp32-ops keeps the compiler from emitting packed fp32 VALU ops.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(HERE, "..", "include"),
]


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; libfmxq.so cannot be built")


def _compile(src: str, obj: str, flags=None) -> None:
    cmd = [_hipcc(), *(flags or HIP_FLAGS), "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    # hipcc's host pass warns that it does not know the packed-fp32 feature; drop that.
    noise = "is not a recognized feature for this target"
    msgs = [ln for ln in r.stderr.splitlines() if noise not in ln and ln.strip()]
    if msgs:
        print("\n".join(msgs), file=sys.stderr)


DIAG = os.path.join(HERE, "diag")
TIMELINE = os.path.join(DIAG, "qmv1_timeline")


def build_diag(verbose: bool = True) -> str:
    """The time-line diagnostic (diag/qmv1_timeline.hip): a program, not part of the
    library, linked with its own build of fmxq_qmv.hip under FMXQ_QMV1_TIMELINE."""
    os.makedirs(OUT_DIR, exist_ok=True)
    flags = [*HIP_FLAGS, "-I", CSRC, "-DFMXQ_QMV1_TIMELINE"]
    objs = []
    for src in (os.path.join(DIAG, "qmv1_timeline.hip"), os.path.join(CSRC, "fmxq_qmv.hip")):
        obj = os.path.join(OUT_DIR, "timeline_" + os.path.basename(src) + ".o")
        _compile(src, obj, flags)
        objs.append(obj)
    r = subprocess.run([_hipcc(), f"--offload-arch={ARCH}", "-o", TIMELINE, *objs],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {TIMELINE}\n{r.stdout}\n{r.stderr}")
    if verbose:
        print(f"built {TIMELINE}")
    return TIMELINE


def build(verbose: bool = True) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))
    objs = [os.path.join(OUT_DIR, os.path.basename(s) + ".o") for s in srcs]
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        list(ex.map(_compile, srcs, objs))
    tmp = LIB + ".tmp"
    rocm_lib = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "lib")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs,
           f"-L{rocm_lib}", f"-Wl,-rpath,{rocm_lib}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()
    if "--diag" in sys.argv[1:]:
        build_diag()
