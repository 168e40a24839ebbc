"""Build recipe for the oracle (test infrastructure only).

Compiles the C restatement of the reference's CPU arithmetic (ovfq_oracle.c, plain x86-64 code) and the
AVX2 + thread-pool CPU baseline (cpu_baseline.c) into oracle/libovfq_oracle.so with gcc.

The reference itself (C# / .NET 10) cannot be built in this image (no dotnet toolchain), so there is no
oracle/_ref build; see the oracle's header for how each function is pinned instead.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libovfq_oracle.so")

# Per-operation IEEE binary32, no contraction: the reference's C# never fuses a*b+c.
COMMON = ["-O2", "-fPIC", "-std=c11", "-ffp-contract=off", "-fno-fast-math", "-Wall", "-Wextra",
          "-Wno-unused-parameter"]


def build(verbose: bool = False) -> str:
    objs = []
    cpub_flags = [*COMMON, "-mavx2", "-mfma"]
    steps = [
        ("ovfq_oracle.c", []),
        ("cpu_baseline.c", ["-mavx2", "-mfma", '-DCPUB_FLAGS="%s"' % " ".join(cpub_flags)]),
    ]
    for src, extra in steps:
        obj = os.path.join(HERE, src.replace(".c", ".o"))
        cmd = ["gcc", *COMMON, *extra, "-c", os.path.join(HERE, src), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True)
        objs.append(obj)
    tmp = LIB + ".tmp"
    cmd = ["gcc", "-shared", "-o", tmp, *objs, "-lpthread", "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    for obj in objs:
        os.remove(obj)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
