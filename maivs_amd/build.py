"""Build the in-tree native parts of maivs_amd.

* ``libmaivs_gpu.so`` - the HIP kernels and the C ABI (``include/maivs_gpu.h``), hipcc for gfx950.
* ``_maivs*.so``      - the host index (build path) and the Python binding, g++ + pybind11.

Both land next to this file, so the package loads them from the source tree without
installation. Run ``python -m maivs_amd.build``.
"""
from __future__ import annotations

import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
HOST_SRC = [os.path.join(HERE, "csrc", "host", f) for f in ("bind.cpp", "index.cpp", "tree.cpp", "persist.cpp")]
GPU_SRC = [os.path.join(HERE, "csrc", "gpu", f) for f in ("maivs_gpu.hip", "build.hip", "store.hip")]
GPU_LIB = os.path.join(HERE, "libmaivs_gpu.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# Device code: no FMA contraction (bit-exact parity with the reference's f32 arithmetic), no
# fast math, correctly rounded f32 division/sqrt, and no packed-FP32 instruction selection.
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off", "-fno-fast-math", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def host_ext_path() -> str:
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    return os.path.join(HERE, "_maivs" + suffix)


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("build step failed: " + " ".join(cmd[:3]) + " ...")


def build_gpu() -> str:
    out = GPU_LIB
    tmp = out + ".tmp"
    _run([HIPCC, *HIP_FLAGS, "-I", os.path.join(ROOT, "include"), *GPU_SRC, "-o", tmp])
    os.replace(tmp, out)
    return out


def build_host() -> str:
    import pybind11

    out = host_ext_path()
    tmp = out + ".tmp"
    py_inc = sysconfig.get_paths()["include"]
    cmd = [
        "g++", "-O3", "-std=c++17", "-fPIC", "-shared", "-mavx2", "-mfma", "-mpopcnt",
        "-ffp-contract=off", "-fno-fast-math", "-fvisibility=hidden",
        "-I", py_inc, "-I", pybind11.get_include(), "-I", os.path.join(ROOT, "include"),
        *HOST_SRC, "-o", tmp, "-ldl", "-lpthread",
    ]
    _run(cmd)
    os.replace(tmp, out)
    return out


def build_all() -> None:
    build_host()
    build_gpu()


if __name__ == "__main__":
    which = sys.argv[1:] or ["host", "gpu"]
    if "host" in which:
        print(build_host())
    if "gpu" in which:
        print(build_gpu())
