"""Build the gfx950 HIP library in-tree: zeninfer_amd/lib/libzq_hip.so.

hipcc cross-compiles for gfx950 without a GPU, so this runs on any host with
ROCm.  Flags: -O3, IEEE-correct fp32 divide/sqrt (the activation quantiser
must reproduce the CPU's amax/127 and 1/d bit for bit), and packed-fp32
instructions disabled.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "csrc")
LIB_DIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIB_DIR, "libzq_hip.so")
SOURCES = ["zq_backend.hip", "zq_gemv.hip", "zq_gemm.hip", "zq_misc.hip", "zq_gguf.cpp", "zq_layer.hip", "zq_model.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]


def build(verbose=False):
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = LIB + ".tmp"
    cmd = [HIPCC, *FLAGS, "-o", tmp, *[os.path.join(SRC, s) for s in SOURCES]]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (res.stdout + res.stderr).splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
