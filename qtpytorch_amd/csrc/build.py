"""Build libmxk.so (the gfx950 HIP kernels + C ABI) in-tree with hipcc.

    python qtpytorch_amd/csrc/build.py [--jobs N]

Each .hip source compiles to an object in parallel, then one shared
library is linked next to the package (qtpytorch_amd/libmxk.so).  Flags:
  --offload-arch=gfx950             CDNA4 only, no other targets
  -ffp-contract=off                 no implicit FMA contraction: every
                                    rounding step of the reference is kept
  -target-feature -packed-fp32-ops  no packed FP32 instructions
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
OUT = os.path.join(PKG, "libmxk.so")
SOURCES = ["mxk_quant.hip", "mxk_gemm.hip", "mxk_linear.hip", "mxk_linear_mfma.hip", "mxk_kv.hip", "mxk_elem.hip", "mxk_dyn.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libmxk.so)")


def _compile(src: str, obj: str) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", os.path.join(HERE, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr[-6000:]}")


def _check_waits(src: str) -> None:
    import importlib.util

    spec = importlib.util.spec_from_file_location("mxk_check_lgkm", os.path.join(HERE, "check_lgkm.py"))
    check_lgkm = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(check_lgkm)
    n, problems = check_lgkm.check_source(src, hipcc(), HIPCC_FLAGS)
    if problems:
        raise RuntimeError(f"LDS wait check failed for {os.path.basename(src)} ({n} kernels):\n" + "\n".join(problems))


def build(jobs: int = 4, verbose: bool = True) -> str:
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    srcs = [s for s in SOURCES if os.path.exists(os.path.join(HERE, s))]
    objs = [os.path.join(objdir, s.replace(".hip", ".o")) for s in srcs]
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        futs = [ex.submit(_compile, s, o) for s, o in zip(srcs, objs)]
        # the GEMM's hand-counted LDS waits, checked on its assembly (check_lgkm.py)
        chk = ex.submit(_check_waits, os.path.join(HERE, "mxk_gemm.hip"))
        for f in futs:
            f.result()
        chk.result()
    tmp = OUT + ".tmp"
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-4000:]}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT} from {', '.join(srcs)}")
    return OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=4)
    a = ap.parse_args()
    try:
        build(a.jobs)
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
