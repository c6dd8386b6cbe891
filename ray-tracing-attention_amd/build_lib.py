"""Builds librta.so (the gfx950 detector path) in-tree with hipcc.

The library is the product; it is compiled for gfx950 only.  Every call compiles
from source (no cache), so a stale library can never mask an edit.
"""
import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
SOURCES = ["csrc/rta_gemv.hip", "csrc/rta_attention.hip", "csrc/rta_step.hip", "csrc/rta_model.hip",
           "csrc/rta_asset.cpp"]
LIB = HERE / "lib" / "librta.so"
# the resident worker (stdin/stdout protocol of the reference's rt_optical_resident)
WORKER_SRC = "worker/rt_optical_resident.cpp"
WORKER = HERE / "lib" / "rt_optical_resident"
# measurement support for the benchmark (the HBM read ceiling), not part of the path
CEILING_SRC = "csrc/rta_ceiling.hip"
CEILING = HERE / "lib" / "librta_ceiling.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-fgpu-rdc",
    # keep the compiler from forming v_pk_{add,mul,fma}_f32
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # the first 16 dwords of every kernel's arguments arrive preloaded in SGPRs, so a
    # kernel's first loads need not wait on a scalar load of its arguments (a kernel
    # starts with cold caches; batch-32 decode step 4.24 -> 4.19 ms)
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wall", "-Wno-unused-function",
]


def build(verbose=False):
    LIB.parent.mkdir(parents=True, exist_ok=True)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, *FLAGS, "-shared", "--hip-link", *[str(HERE / s) for s in SOURCES], "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (res.stdout + res.stderr).splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{out}")
    if out.strip() and verbose:
        print(out, file=sys.stderr)
    os.replace(tmp, LIB)
    wtmp = WORKER.with_suffix(".tmp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-O2", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "-Wall", str(HERE / WORKER_SRC), "-L", str(LIB.parent), "-lrta",
           "-Wl,-rpath,$ORIGIN", "-o", str(wtmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (res.stdout + res.stderr).splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on the worker ({res.returncode}):\n{out}")
    os.replace(wtmp, WORKER)
    ctmp = CEILING.with_suffix(".so.tmp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared", "-Xclang", "-target-feature",
           "-Xclang", "-packed-fp32-ops", "-Wall", str(HERE / CEILING_SRC), "-o", str(ctmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on the ceiling probe ({res.returncode}):\n{res.stdout + res.stderr}")
    os.replace(ctmp, CEILING)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
