"""Build script for the gfx950 IQ2_XXS library (libcmk_iq2.so) and its C++ host layer.

Run `python candelora-metal-kernels_amd/build.py` (or __graft_entry__.build()).
Every HIP source is compiled with hipcc for gfx950 only; objects go to
candelora-metal-kernels_amd/_build/, the shared libraries next to this file.

  libcmk_iq2.so        C ABI (include/cmk_iq2.h): kernels + dispatch + runtime wrappers
  libcandelora_iq2.so  C++ host layer with the reference's API (host/), linked to libcmk_iq2
  libcmk_probe.so      bench.py's plain HBM read (the floor the decode GEMV is set beside)
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
HOST = os.path.join(PKG, "host")
OBJ = os.path.join(PKG, "_build")
INCLUDE = os.path.join(REPO, "include")

LIB = os.path.join(PKG, "libcmk_iq2.so")
HOST_LIB = os.path.join(PKG, "libcandelora_iq2.so")
PROBE_LIB = os.path.join(PKG, "libcmk_probe.so")

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# Packed FP32 instructions are disabled for every device compile.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]

HIP_SOURCES = [
    "iq2xxs_dequant.hip",
    "iq2xxs_gemv.hip",
    "iq2xxs_gemv_rows.hip",
    "iq2xxs_gemm.hip",
    "iq2xxs_simple.hip",
    "iq_variants.hip",
    "mlp_ops.hip",
    "cmk_iq2.cpp",
]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns about the device-only target feature; keep other output.
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        sys.stderr.write(err + "\n")
        raise RuntimeError("command failed: " + " ".join(cmd))
    if err.strip():
        sys.stderr.write(err + "\n")


def _compile(src: str) -> str:
    obj = os.path.join(OBJ, os.path.splitext(os.path.basename(src))[0] + ".o")
    lang = ["-x", "hip"] if src.endswith(".cpp") else []
    _run([HIPCC, *HIP_FLAGS, *lang, "-c", src, "-o", obj])
    return obj


def build_lib() -> str:
    os.makedirs(OBJ, exist_ok=True)
    srcs = [os.path.join(CSRC, s) for s in HIP_SOURCES]
    with ThreadPoolExecutor(max_workers=4) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIB)
    return LIB


def build_probe() -> str:
    """bench.py's plain-read kernel (bench_read_floor.hip beside it), a library of its own."""
    obj = _compile(os.path.join(REPO, "bench_read_floor.hip"))
    tmp = PROBE_LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, obj])
    os.replace(tmp, PROBE_LIB)
    return PROBE_LIB


def build_host() -> str:
    """C++ host layer with the reference API (host code only, over the C ABI)."""
    host_src = os.path.join(HOST, "iq2_matmul.cpp")
    if not os.path.exists(host_src):
        return ""
    rocm_inc = "/opt/rocm/include"
    cxx = ["g++", "-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", f"-I{INCLUDE}", f"-I{HOST}",
           f"-I{rocm_inc}"]
    tmp = HOST_LIB + ".tmp"
    _run([*cxx, "-shared", "-o", tmp, host_src, f"-L{PKG}", "-lcmk_iq2", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, HOST_LIB)
    return HOST_LIB


def build() -> str:
    if not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    lib = build_lib()
    build_host()
    build_probe()
    return lib


def clean() -> None:
    shutil.rmtree(OBJ, ignore_errors=True)
    for p in (LIB, HOST_LIB, PROBE_LIB):
        if os.path.exists(p):
            os.remove(p)


if __name__ == "__main__":
    print(build())
