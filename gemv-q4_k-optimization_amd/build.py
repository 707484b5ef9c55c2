"""Builds libq4k_gemv.so in-tree: the gfx950 kernels + C ABI (hipcc), the host
Q4_K/Q6_K quantisers and the GGUF reader (g++), linked into one shared
library."""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libq4k_gemv.so")
ARCH = "gfx950"


def _hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found")


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout)
        raise RuntimeError(f"build step failed: {' '.join(cmd)}")
    return r.stdout


def build(verbose: bool = False, save_temps: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    hipcc = _hipcc()
    host_obj = os.path.join(BUILD, "q4k_quantize_host.o")
    # the device sources compile in parallel (each instantiates many kernels)
    dev_objs, procs = [], []
    for src in ("q4k_gemv.hip", "q6k_gemv.hip", "q4k_sums.hip", "q6k_sums.hip", "q4k_short.hip", "q6k_short.hip",
                "q4k_probe.hip"):
        obj = os.path.join(BUILD, src.replace(".hip", ".o"))
        cmd = [hipcc, f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
               # no packed-FP32 instructions in device code
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               "-Wall", "-Wno-unused-function",
               "-c", os.path.join(CSRC, src), "-o", obj]
        if save_temps:
            cmd.insert(1, "--save-temps=obj")
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
        dev_objs.append(obj)
    for cmd, pr in procs:
        out, _ = pr.communicate()
        if pr.returncode != 0:
            sys.stderr.write(out)
            raise RuntimeError(f"build step failed: {' '.join(cmd)}")
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-ffp-contract=off", "-fno-fast-math", "-Wall",
          "-c", os.path.join(CSRC, "q4k_quantize_host.cpp"), "-o", host_obj], verbose)
    gguf_obj = os.path.join(BUILD, "gguf_reader.o")
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra",
          "-c", os.path.join(CSRC, "gguf_reader.cpp"), "-o", gguf_obj], verbose)
    tmp = LIB + ".tmp"
    _run([hipcc, "-shared", "-fPIC", "-o", tmp, *dev_objs, host_obj, gguf_obj, "-lpthread"], verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True, save_temps="--save-temps" in sys.argv))
