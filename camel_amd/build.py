"""Builds the native libraries in-tree.

* ``camel_amd/lib/libcamel_hip.so`` -- the HIP kernels and the C-ABI shim
  (``include/camel_hip.h``), compiled for gfx950 only.
* ``camel_amd/lib/libcamel_tensor.so`` -- the C++ operator layer (the
  ``tensor:*`` operators, ``TensorObject`` with device residency) linked
  against libcamel_hip.so.

``python -m camel_amd.build`` or ``__graft_entry__.build()`` runs it; every call
recompiles.  Objects go to ``_build/`` (git-ignored).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "camel_amd")
HIP_SRC = os.path.join(PKG, "csrc", "hip")
MOD_SRC = os.path.join(PKG, "csrc", "module")
INCLUDE = os.path.join(ROOT, "include")
LIB_DIR = os.path.join(PKG, "lib")
BUILD_DIR = os.path.join(ROOT, "_build")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# -ffp-contract=off: one rounding per reference operation (no FMA contraction
# outside the MFMA accumulators).  Packed fp32 instructions are disabled.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", f"-I{INCLUDE}",
]
CXX_FLAGS = ["-O3", "-fPIC", "-std=c++20", "-Wall", "-Wextra", "-Wno-unused-parameter",
             "-ffp-contract=off", f"-I{INCLUDE}", f"-I{MOD_SRC}"]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        msg = "\n".join(
            line for line in (proc.stdout + proc.stderr).splitlines()
            if "packed-fp32-ops" not in line)
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{msg}")


def _compile_hip(src: str) -> str:
    obj = os.path.join(BUILD_DIR, os.path.basename(src) + ".o")
    _run([HIPCC, *HIP_FLAGS, "-c", src, "-o", obj])
    return obj


def _compile_cxx(src: str) -> str:
    obj = os.path.join(BUILD_DIR, "mod_" + os.path.basename(src) + ".o")
    _run(["g++", *CXX_FLAGS, "-c", src, "-o", obj])
    return obj


def build_hip(jobs: int = 8) -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    srcs = sorted(os.path.join(HIP_SRC, f) for f in os.listdir(HIP_SRC) if f.endswith(".hip"))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile_hip, srcs))
    out = os.path.join(LIB_DIR, "libcamel_hip.so")
    tmp = out + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, out)
    return out


def build_module(jobs: int = 8) -> str | None:
    if not os.path.isdir(MOD_SRC):
        return None
    srcs = sorted(os.path.join(MOD_SRC, f) for f in os.listdir(MOD_SRC) if f.endswith(".cpp"))
    if not srcs:
        return None
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile_cxx, srcs))
    out = os.path.join(LIB_DIR, "libcamel_tensor.so")
    tmp = out + ".tmp"
    _run(["g++", "-shared", "-fPIC", "-o", tmp, *objs, f"-L{LIB_DIR}", "-lcamel_hip",
          "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, out)
    return out


def build_oracle() -> str:
    """Compiles the CPU oracle (test infrastructure, never linked by the product)."""
    _run(["make", "-s", "-B", "-C", os.path.join(ROOT, "oracle")])
    return os.path.join(ROOT, "oracle", "liboracle.so")


def build_all(jobs: int = 8) -> list[str]:
    if shutil.which(HIPCC) is None and not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    built = [build_hip(jobs)]
    mod = build_module(jobs)
    if mod:
        built.append(mod)
    built.append(build_oracle())
    return built


if __name__ == "__main__":
    for path in build_all():
        print(path)
    sys.exit(0)
