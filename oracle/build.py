"""Build recipe for the CPU oracle (test infrastructure only).

Compiles oracle/gguf_oracle.c into oracle/liboracle.so with gcc.
-ffp-contract=off keeps every f32 multiply and add separately rounded, as the
reference's Rust code is (Rust never contracts a*b+c into an FMA).

The reference itself (asqrzk/CombsEngine) is Rust; this image has no
cargo/rustc, so there is no oracle/_ref build of it.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "gguf_oracle.c")
OUT = os.path.join(HERE, "liboracle.so")


def build(verbose: bool = False) -> str:
    cmd = ["gcc", "-O2", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off",
           "-fno-fast-math", "-std=c11", "-Wall", "-o", OUT, SRC, "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    return OUT


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
