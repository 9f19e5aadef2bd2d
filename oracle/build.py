"""Builds the CPU oracle (test infrastructure only): oracle/build/libmkv_oracle.so from mkv_oracle.c and
flint_oracle.c.

gcc -O3 -fopenmp -ffp-contract=off: every product and sum is rounded to f32 in source order (no FMA contraction),
the convention the restatement fixes for the reference's WGSL arithmetic.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "build", "libmkv_oracle.so")


def build(verbose=False):
    os.makedirs(os.path.dirname(OUT), exist_ok=True)
    cmd = ["gcc", "-O3", "-fopenmp", "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-shared", "-std=c11",
           "-Wall", "-Wno-unknown-pragmas", "-o", OUT, os.path.join(HERE, "mkv_oracle.c"), os.path.join(HERE, "flint_oracle.c"), "-lm"]
    if verbose:
        print(" ".join(cmd))
    subprocess.run(cmd, check=True)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
