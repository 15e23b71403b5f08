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
# -O3 for the AVX2 / FMA / BMI2 level of x86-64 (x86-64-v3), tuned for Zen 3: the reference builds
# with target-cpu=native on a Zen 3 laptop (.cargo/config.toml:1-8). The library runs on other
# hosts than the one that builds it, so the ISA is named, not `native`. No FMA contraction and
# no fast math keep every f32 result in the reference's order (the dots use explicit FMAs).
FLAGS = ["-O3", "-march=x86-64-v3", "-mtune=znver3", "-std=c++17", "-fPIC", "-shared",
         "-ffp-contract=off", "-fno-fast-math"]


def build() -> str:
    tmp = LIB + ".tmp"
    cmd = ["g++", *FLAGS, os.path.join(HERE, "oracle.cpp"), "-o", tmp, "-lpthread", "-lm"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("oracle build failed")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
