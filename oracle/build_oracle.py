"""Build the oracle (test infrastructure): ``oracle/liboracle.so`` from ``oracle/oracle.cpp``.

The oracle is compiled with the flags that keep its f32 arithmetic in the reference's order:
no FMA contraction, AVX2 + FMA intrinsics where the reference uses them, glibc libm.

The reference itself is a Rust crate (Cargo.toml, no build.rs, crates.io dependencies not
vendored) and this image has no rustc/cargo, so no ``oracle/_ref`` build exists.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")


def build() -> str:
    tmp = LIB + ".tmp"
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-mavx2", "-mfma", "-mpopcnt",
           "-ffp-contract=off", "-fno-fast-math", os.path.join(HERE, "oracle.cpp"), "-o", tmp,
           "-lpthread", "-lm"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("oracle build failed")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
