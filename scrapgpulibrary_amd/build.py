"""Builds scrapgpulibrary_amd/libscrapgpu_hip.so: the scrapgpu_ C API core and the gfx950 `hip`
backend, compiled in-tree with hipcc (host C++17 + device code for gfx950 only).

    python -m scrapgpulibrary_amd.build        # or __graft_entry__.build()
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
OBJ = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libscrapgpu_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON = ["-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden", "-Wall", "-Wno-unused-function",
          "-I", os.path.join(ROOT, "include"), "-I", CSRC]
# device flags: gfx950 only; packed-fp32 instruction selection disabled (some packed fp32 forms
# have given wrong results on these machines)
DEVICE = ["--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-munsafe-fp-atomics"]

SOURCES = [
    ("core/status.cpp", []),
    ("core/registry.cpp", []),
    ("core/op.cpp", []),
    ("core/tensor.cpp", []),
    ("hip/backend.cpp", ["-x", "hip"] + DEVICE),
    ("hip/matvec.hip", DEVICE),
    ("hip/matvec_float.hip", DEVICE),
    ("hip/matmul.hip", DEVICE),
    # bit-exact conversions: one IEEE operation per source operation
    ("hip/quant.hip", DEVICE + ["-ffp-contract=off"]),
]


def _compile(src: str, extra: list[str]) -> str:
    out = os.path.join(OBJ, src.replace("/", "_") + ".o")
    cmd = [HIPCC] + COMMON + extra + ["-c", os.path.join(CSRC, src), "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return out


C_CALLER_SRC = os.path.join(ROOT, "tests", "c", "standalone_matmul.c")
C_CALLER = os.path.join(ROOT, "tests", "c", "standalone_matmul")


def build_c_caller() -> str:
    """The C99 test caller of the public API (tests/c/standalone_matmul.c), linked against the
    library in-tree (rpath to the package directory)."""
    cmd = ["gcc", "-std=c99", "-O2", "-Wall", "-Wextra", "-Werror", "-I", os.path.join(ROOT, "include"), C_CALLER_SRC,
           "-L", PKG, "-lscrapgpu_hip", "-Wl,-rpath,$ORIGIN/../../scrapgpulibrary_amd", "-o", C_CALLER]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"C caller build failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return C_CALLER


def build(verbose: bool = True) -> str:
    os.makedirs(OBJ, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        objs = list(ex.map(lambda s: _compile(*s), SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "-shared", "--offload-arch=gfx950", "-fPIC", "-o", tmp] + objs + ["-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    build_c_caller()
    if verbose:
        print("built", LIB)
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
