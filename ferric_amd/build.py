"""Builds libferric_hip.so (gfx950) in-tree with hipcc.

Every translation unit under ferric_amd/csrc is compiled for gfx950 only, with
FP contraction off (the reference's scalar arithmetic rounds every product
and sum separately; kernels that want FMA ask for it explicitly) and with
packed-FP32 instruction selection disabled. The shared library lands next to
this file so that it travels with the source tree.
"""

from __future__ import annotations

import concurrent.futures
import os
import subprocess
import sys
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_DIR = PACKAGE_DIR.parent
CSRC = PACKAGE_DIR / "csrc"
BUILD_DIR = PACKAGE_DIR / "_build"
LIBRARY = PACKAGE_DIR / "libferric_hip.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    "-Wno-unused-value",
    "-Wno-unused-result",
]


def _compile(src: Path) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, "-I", str(REPO_DIR / "include"), "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(verbose: bool = True) -> Path:
    """Compiles every csrc/*.hip for gfx950 and links libferric_hip.so."""
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    workers = min(len(sources), max(1, (os.cpu_count() or 4)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        objects = list(pool.map(_compile, sources))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY.relative_to(REPO_DIR)} from {len(sources)} sources", file=sys.stderr)
    build_c_host(verbose)
    build_hip_checks(verbose)
    return LIBRARY


C_HOST_SRC = REPO_DIR / "tests" / "c" / "abi_decode.c"
C_HOST_BIN = REPO_DIR / "tests" / "c" / "abi_decode"


def build_c_host(verbose: bool = True) -> Path:
    """Compiles the plain-C host of the ABI (tests/c/abi_decode.c) with gcc
    against the in-tree library (found at run time through its rpath)."""
    rocm_lib = Path(HIPCC).resolve().parent.parent / "lib"
    cmd = ["gcc", "-O2", "-std=c99", "-Wall", "-Wextra", "-I", str(REPO_DIR / "include"), str(C_HOST_SRC),
           "-L", str(LIBRARY.parent), "-lferric_hip", f"-Wl,-rpath-link,{rocm_lib}",
           "-Wl,-rpath,$ORIGIN/../../ferric_amd", "-o", str(C_HOST_BIN)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"gcc failed for {C_HOST_SRC.name}:\n{proc.stdout}\n{proc.stderr}")
    if verbose:
        print(f"built {C_HOST_BIN.relative_to(REPO_DIR)}", file=sys.stderr)
    return C_HOST_BIN


HIP_CHECKS = [REPO_DIR / "tests" / "hip" / "sqrt_rn_check.hip"]


def build_hip_checks(verbose: bool = True) -> list:
    """Compiles the standalone HIP check programs under tests/hip (each one
    exercises a device helper directly; the GPU tests run them)."""
    out = []
    for src in HIP_CHECKS:
        binary = src.with_suffix("")
        cmd = [HIPCC, *[f for f in COMMON_FLAGS if f != "-fPIC"], "-o", str(binary), str(src)]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stdout}\n{proc.stderr}")
        if verbose:
            print(f"built {binary.relative_to(REPO_DIR)}", file=sys.stderr)
        out.append(binary)
    return out


if __name__ == "__main__":
    build()
