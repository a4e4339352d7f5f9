"""Builds the native libraries in-tree: ``python -m silvic_amd.build``.

- ``_lib/libsilvic_rocm.so``: the HIP backend (include/silvic_rocm.h) for gfx950;
- ``_lib/libsilvic_synth.so``: the synthetic-workload generator (host code).

HIP code is compiled with ``-ffp-contract=off`` (no implicit fused multiply-adds: quantization and split gains
must round exactly as silvic's CPU path does) and with packed FP32 instructions disabled.
"""

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "_lib")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-shared", "-pthread", "-Wall"]


def _run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(line for line in proc.stdout.splitlines() if "packed-fp32-ops" not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{out}")
    return out


def build_rocm():
    os.makedirs(LIB, exist_ok=True)
    out = os.path.join(LIB, "libsilvic_rocm.so")
    tmp = out + ".tmp"
    _run([HIPCC, *HIP_FLAGS, "-o", tmp, os.path.join(CSRC, "backend.hip")])
    os.replace(tmp, out)
    return out


def build_synth():
    os.makedirs(LIB, exist_ok=True)
    out = os.path.join(LIB, "libsilvic_synth.so")
    tmp = out + ".tmp"
    _run(["g++", *CXX_FLAGS, "-o", tmp, os.path.join(CSRC, "synth.cpp")])
    os.replace(tmp, out)
    return out


def build_all():
    return [build_synth(), build_rocm()]


if __name__ == "__main__":
    for path in build_all():
        print(path)
    sys.exit(0)
