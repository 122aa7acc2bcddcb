"""Builds the gfx950 attention path in-tree: the kernels' code object and the C-ABI host library.

    python ghost-infer_amd/gi_build.py

Outputs (beside this file): gi_attn_gfx950.hsaco (hipcc --genco, loaded at run time with hipModuleLoad),
gi_probes_gfx950.hsaco (bench.py's peak probes),
libgi_attn.so (the C ABI of include/gi_attn.h) and gi_layer_harness (a C++ caller of that ABI playing one
layer's attention, harness/gi_layer_harness.cpp). hipcc cross-compiles for gfx950, so this runs on a
machine without a GPU.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
HSACO = os.path.join(HERE, "gi_attn_gfx950.hsaco")
LIB = os.path.join(HERE, "libgi_attn.so")
HARNESS = os.path.join(HERE, "gi_layer_harness")
PROBES = os.path.join(HERE, "gi_probes_gfx950.hsaco")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# packed f32 VALU ops are disabled for all device code (see the project's design notes on gfx950 boxes)
DEVICE_FLAGS = ["--offload-arch=gfx950", "-O3", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def run(cmd):
    print("+", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def build_kernels():
    run([HIPCC, *DEVICE_FLAGS, "--genco", os.path.join(CSRC, "gi_attn_kernels.hip"), "-o", HSACO])
    # the bench's peak probes (MFMA rate, HBM read stream): their own code object, not part of the path
    run([HIPCC, *DEVICE_FLAGS, "--genco", os.path.join(CSRC, "gi_probes.hip"), "-o", PROBES])


def build_host():
    run([HIPCC, "--offload-arch=gfx950", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-I", os.path.join(ROOT, "include"),
         os.path.join(CSRC, "gi_attn_host.cpp"), "-o", LIB, "-ldl"])


def build_harness():
    run([HIPCC, "--offload-arch=gfx950", "-O2", "-std=c++17", "-Wall", "-I", os.path.join(ROOT, "include"),
         os.path.join(HERE, "harness", "gi_layer_harness.cpp"), "-o", HARNESS, "-L", HERE, "-lgi_attn",
         "-Wl,-rpath,$ORIGIN"])


def build():
    build_kernels()
    build_host()
    build_harness()


if __name__ == "__main__":
    build()
    sys.exit(0)
