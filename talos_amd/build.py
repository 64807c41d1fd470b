"""Build the MI355X decode backend (gfx950) into talos_amd/libtalos_hip.so.

Compiles every HIP source with hipcc --offload-arch=gfx950 (cross-compiles
on a machine without a GPU) and the host C++ with g++, then links one shared
library exporting the C ABI of include/talos_hip.h and include/talos_host.h.

    python -m talos_amd.build          # or talos_amd.build.build()
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libtalos_hip.so")

ARCH = "gfx950"
HIP_SOURCES = ["talos_hip.hip", "mega_inst_q4_mfma.hip", "mega_inst_q4_q6k.hip", "mega_inst_q4_q4.hip",
               "mega_inst_q8_wide.hip", "mega_inst_q8_small.hip", "mega_inst_f32.hip"]
HOST_SOURCES = ["host/gguf.cpp", "host/synth.cpp", "host/model.cpp", "host/host_capi.cpp"]

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Keep the compiler from forming packed-FP32 instructions.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-pthread"]


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build talos_amd)")


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")


def build(verbose: bool = False) -> str:
    """Compile and link the library; returns its path."""
    os.makedirs(BUILD, exist_ok=True)
    hipcc = _hipcc()
    cxx = shutil.which("g++") or "g++"
    jobs = []
    objs = []
    for src in HIP_SOURCES:
        obj = os.path.join(BUILD, os.path.basename(src) + ".o")
        jobs.append([hipcc, *HIPCC_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
        objs.append(obj)
    for src in HOST_SOURCES:
        obj = os.path.join(BUILD, os.path.basename(src) + ".o")
        jobs.append([cxx, *CXX_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
        objs.append(obj)
    with ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
        for cmd, fut in [(c, ex.submit(_run, c)) for c in jobs]:
            if verbose:
                print(" ".join(cmd))
            fut.result()
    tmp = LIB + ".tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-o", tmp, *objs, "-pthread"])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
