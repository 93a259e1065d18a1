"""Build the C part of the CPU oracle (test infrastructure, never shipped).

    python oracle/build.py        # -> oracle/libks_oracle.so

gcc only; -ffp-contract=off keeps every fp32 operation separately rounded unless
the source asks for fmaf() explicitly.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "ks_oracle.c")
LIB = os.path.join(HERE, "libks_oracle.so")


def build(verbose: bool = False) -> str:
    tmp = LIB + ".tmp"
    cmd = ["gcc", "-O2", "-std=c11", "-fopenmp", "-ffp-contract=off", "-fno-fast-math",
           "-Wall", "-shared", "-fPIC", SRC, "-o", tmp, "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
