"""Build recipe for the CPU oracle (test infrastructure only).

Compiles oracle/kqref.c (fp64 restatement of the reference CPU paths),
oracle/vqquant.c (the VQ quantiser as specified for the GPU) and
oracle/cpu_fast.c (x86 restatement of the reference's CPU int4 GEMV, the timed
baseline) into oracle/_build/libkqref.so with gcc; cpu_fast.c goes through
ROCm's clang when it is there, since the neon16 restatement needs the
AVX-512-FP16 intrinsics that gcc 11 lacks (with gcc it builds without that
path). No -ffast-math: the oracle relies on IEEE fp64 semantics.

The reference's own CPU code cannot be compiled here (its CPU references sit in
Objective-C++ translation units that import Metal/Foundation, and its fast
CPU path needs arm_neon.h and Accelerate), so there is no oracle/_ref build.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(OUT_DIR, "libkqref.so")


CLANG = "/opt/rocm/llvm/bin/clang"
FLAGS = ["-O2", "-std=c11", "-fPIC", "-pthread", "-Wall", "-Wextra", "-Wno-unused-parameter"]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def build(verbose: bool = False) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    fast_cc = CLANG if os.path.exists(CLANG) else "gcc"
    fast_o = os.path.join(OUT_DIR, "cpu_fast.o")
    _run([fast_cc] + FLAGS + ["-c", "-o", fast_o, os.path.join(HERE, "cpu_fast.c")], verbose)
    srcs = [os.path.join(HERE, "kqref.c"), os.path.join(HERE, "vqquant.c")]
    tmp = LIB + ".tmp"
    _run(["gcc"] + FLAGS + ["-shared", "-o", tmp] + srcs + [fast_o, "-lm"], verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
