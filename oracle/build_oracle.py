"""Build recipe for the CPU oracle (test infrastructure only).

Compiles oracle/jules_oracle.c into oracle/liboracle.so with gcc.  The hot
loops carry target_clones, so the .so built here also runs (and uses AVX-512
where present) on the GPU box's host CPU.

The reference's own kernels (include/jules/Kernel/*.h) cannot be compiled in
this image: FusedKernels.h:31 and FlashAttention.h:26 include <cblas.h>, which
the image does not ship, so there is no oracle/_ref build.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "jules_oracle.c")
OUT = os.path.join(HERE, "liboracle.so")

CFLAGS = ["-O3", "-std=c11", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off",
          "-fno-math-errno", "-Wall", "-Wextra", "-Wno-unused-parameter"]


def build(verbose: bool = False) -> str:
    tmp = OUT + ".tmp"
    cmd = ["gcc", *CFLAGS, SRC, "-o", tmp, "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
