"""Build recipe for the CPU oracle shared library (test infrastructure only).

Compiles oracle/*.c with gcc into oracle/liboracle.so.  The floating-point
flags are part of the oracle's contract: -ffp-contract=off keeps every f32
operation separately rounded (Go on amd64 does not fuse multiply-add), and
no -ffast-math keeps the sequential reduction order and IEEE semantics.
"""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
SOURCES = ["numeric.c", "norm.c", "rope.c", "activation.c", "page.c", "attention.c", "matmul.c", "quant.c"]
LIBRARY = os.path.join(HERE, "liboracle.so")

CFLAGS = [
    "-O3", "-march=x86-64-v3", "-std=c11", "-D_GNU_SOURCE", "-fPIC", "-shared", "-fopenmp",
    "-ffp-contract=off", "-fno-fast-math", "-fno-finite-math-only",
    "-Wall", "-Wno-unknown-pragmas",
]


def build(verbose: bool = False) -> str:
    cmd = ["gcc", *CFLAGS, *[os.path.join(HERE, s) for s in SOURCES], "-o", LIBRARY + ".tmp", "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(LIBRARY + ".tmp", LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose=True))
