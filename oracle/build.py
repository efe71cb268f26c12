"""Build recipe for the CPU oracle (test infrastructure only).

Compiles oracle/srq_oracle.c with gcc into oracle/_build/libsrq_oracle.so.
-ffp-contract=off keeps every multiply and add separately rounded, and no
-ffast-math flag is given, so the reference's reduction orders survive.

The reference itself is Go (cmd/monolith/monolith.go) and no Go toolchain
exists here, so there is no oracle/_ref build: the restatement is pinned by
the checks listed in srq_oracle.h instead.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(OUT_DIR, "libsrq_oracle.so")
SRC = os.path.join(HERE, "srq_oracle.c")


def build(force=True):
    """Compile the oracle; always recompiles when force is true."""
    if not force and os.path.exists(LIB) and os.path.getmtime(LIB) >= os.path.getmtime(SRC):
        return LIB
    os.makedirs(OUT_DIR, exist_ok=True)
    tmp = LIB + ".tmp%d" % os.getpid()
    cmd = ["gcc", "-std=c11", "-D_GNU_SOURCE", "-O3", "-march=x86-64-v2", "-ffp-contract=off",
           "-fno-fast-math", "-fPIC", "-shared", "-pthread", "-Wall", "-o", tmp, SRC, "-lm"]
    subprocess.check_call(cmd)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(force=True))
    sys.exit(0)
