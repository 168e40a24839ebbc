"""Builds libovfq.so (the HIP library behind include/ovfq.h) in-tree with hipcc for gfx950."""
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libovfq.so")
SOURCES = ["quant.hip", "project.hip", "gemv.hip", "mfma.hip", "moe.hip", "heads.hip", "noalloc.hip", "api.cpp"]

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    # Per-operation IEEE fp32: the reference's C# never contracts a*b+c into an FMA.
    "-ffp-contract=off",
    # No packed-fp32 instructions (v_pk_{add,mul,fma}_f32) in any kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]

# Per-file additions. The MFMA kernels accumulate in VGPRs instead of AGPRs: with AGPR accumulators the expert-stream
# and small-M kernels copy every result out (v_accvgpr_read, 12 per super-block step) before the fp32 tail.
FILE_FLAGS = {"mfma.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=true"]}


def build(verbose: bool = False) -> str:
    objs = []
    for src in SOURCES:
        obj = os.path.join(CSRC, src + ".o")
        cmd = [HIPCC, *FLAGS, *FILE_FLAGS.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True)
        objs.append(obj)
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    for obj in objs:
        os.remove(obj)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
