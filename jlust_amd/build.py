"""In-tree build of the native parts of jlust_amd.

- ``libjlust_hip.so``: the HIP kernels and the C ABI (``include/jlust_hip.h``),
  compiled by hipcc for gfx950 only.
- ``libjlust_workloads.so``: the host-side synthetic input generator.

Run ``python -m jlust_amd.build`` (or ``__graft_entry__.build()``).  Sources are
compiled in parallel into ``jlust_amd/_build/`` and linked next to this file.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
HIP_LIB = os.path.join(HERE, "libjlust_hip.so")
WL_LIB = os.path.join(HERE, "libjlust_workloads.so")

HIP_SOURCES = ["capi.hip", "scan.hip", "spmv.hip", "coo_spmv.hip", "spmm.hip", "sddmm.hip",
               "bsr_spmm.hip", "convert.hip", "assemble.hip", "fn.hip", "dcsr.hip", "coo_plan.hip",
               "periodic.hip", "spmv_binned.hip", "coo_csc.hip"]

ARCH = os.environ.get("JLUST_HIP_ARCH", "gfx950")

# Packed-FP32 instructions are disabled (-packed-fp32-ops): the compiler would
# otherwise form v_pk_{add,mul,fma}_f32 from ordinary float code.
HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-mcode-object-version=5", "-munsafe-fp-atomics",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-result",
    f"-I{os.path.join(ROOT, 'include')}",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP library cannot be built")


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("build step failed:\n  " + " ".join(cmd) + "\n" + r.stdout + r.stderr)
    return r


def build_hip(jobs: int = 8, verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    hipcc = _hipcc()
    objs = []
    cmds = []
    for src in HIP_SOURCES:
        obj = os.path.join(BUILD, src.replace(".hip", ".o"))
        objs.append(obj)
        cmds.append([hipcc, *HIPCC_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        for cmd, fut in zip(cmds, [ex.submit(_run, c) for c in cmds]):
            fut.result()
            if verbose:
                print(" ".join(cmd), flush=True)
    tmp = HIP_LIB + ".tmp"
    _run([hipcc, "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", tmp, *objs])
    os.replace(tmp, HIP_LIB)
    return HIP_LIB


def build_workloads() -> str:
    tmp = WL_LIB + ".tmp"
    _run(["gcc", "-O3", "-fPIC", "-fopenmp", "-shared", "-std=gnu11", "-Wall",
          os.path.join(CSRC, "workloads.c"), "-o", tmp, "-lm"])
    os.replace(tmp, WL_LIB)
    return WL_LIB


def build(jobs: int = 8, verbose: bool = False):
    with cf.ThreadPoolExecutor(max_workers=2) as ex:
        f1 = ex.submit(build_hip, jobs, verbose)
        f2 = ex.submit(build_workloads)
        return f1.result(), f2.result()


if __name__ == "__main__":
    out = build(verbose="-v" in sys.argv)
    print("\n".join(out))
