"""Builds, in-tree next to the Python package that loads them:
- libpkv.so: HIP kernels for gfx950 + the C-ABI + the host KV manager;
- pkv_kernels.hsaco: the same kernel bodies under the reference engine's
  kernel names and signatures (a code object for hipModuleLoadData)."""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "pkv", "libpkv.so")
HSACO = os.path.join(HERE, "pkv", "pkv_kernels.hsaco")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# Packed FP32 instructions are kept out of every code object.
COMMON = [
    "--offload-arch=gfx950", "-O3", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]
FLAGS = COMMON + ["-fPIC", "-shared"]
SOURCES = ["pkv_capi.hip", "pkv_host.cpp"]


def _run(cmd, what, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"{what} build failed")


def build(verbose=False):
    _run([HIPCC] + FLAGS + [os.path.join(CSRC, s) for s in SOURCES] + ["-o", OUT], "libpkv.so", verbose)
    _run([HIPCC, "--genco"] + COMMON + [os.path.join(CSRC, "pkv_refabi.hip"), "-o", HSACO], "pkv_kernels.hsaco",
         verbose)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
