"""Build libmiqmm.so (the HIP kernels + C ABI) for gfx950 with hipcc, in-tree.

    python sen-mlx_amd/build.py [--jobs N]

Objects go to sen-mlx_amd/_build/, the library to sen-mlx_amd/miqmm/libmiqmm.so.
Every HIP file is compiled with packed-fp32 instructions disabled.
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "miqmm", "libmiqmm.so")
SOURCES = ["qmv.hip", "checkpoint.cpp", "qmv_mfma.hip", "qmvx.hip", "qmm.hip", "qmvs.hip", "aux.hip", "api.cpp"]
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function",
    # leading scalar kernel arguments arrive in SGPRs at wave launch (no scalar
    # memory round trip before a kernel's first load)
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


# per-file flags: the small-M MFMA GEMV keeps its few accumulators in VGPRs,
# where the dequant's fused multiply-adds read them directly (in AGPRs every
# read is a copy)
FILE_FLAGS = {"qmv_mfma.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *FLAGS, *FILE_FLAGS.get(src, []), "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def build(jobs: int = 4) -> str:
    os.makedirs(BUILD, exist_ok=True)
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


def _usage(src: str) -> dict:
    """Register use of every kernel instantiation of one source (device pass only)."""
    os.makedirs(BUILD, exist_ok=True)
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".usage.o")
    cmd = [hipcc(), *FLAGS, *FILE_FLAGS.get(src, []), "--offload-device-only",
           "-Rpass-analysis=kernel-resource-usage", "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stderr}")
    os.remove(obj)
    out = {"kernels": 0, "vgpr_spill": 0, "scratch": 0, "sgpr_spill": 0}
    for line in r.stderr.splitlines():
        if "Function Name:" in line:
            out["kernels"] += 1
        for key, tag in (("vgpr_spill", "VGPRs Spill:"), ("sgpr_spill", "SGPRs Spill:"),
                         ("scratch", "ScratchSize [bytes/lane]:")):
            if tag in line and int(line.split(tag)[1].split()[0]) > 0:
                out[key] += 1
    return out


def resource_usage(jobs: int = 4) -> bool:
    """Prints, per HIP source, how many kernel instantiations spill VGPRs, use
    scratch memory or spill SGPRs (SGPR spills go to VGPR lanes, not memory);
    False if any instantiation spills VGPRs or uses scratch."""
    srcs = [s for s in SOURCES if s.endswith(".hip")]
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        res = list(ex.map(_usage, srcs))
    ok = True
    for src, u in zip(srcs, res):
        print(f"{src}: {u['kernels']} kernels, VGPR spills {u['vgpr_spill']}, scratch {u['scratch']}, "
              f"SGPR spills (to VGPR lanes) {u['sgpr_spill']}")
        ok = ok and u["vgpr_spill"] == 0 and u["scratch"] == 0
    return ok


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=4)
    ap.add_argument("--resource-usage", action="store_true",
                    help="report spills and scratch of every kernel instantiation instead of building")
    args = ap.parse_args()
    if args.resource_usage:
        sys.exit(0 if resource_usage(args.jobs) else 1)
    print(build(args.jobs))
