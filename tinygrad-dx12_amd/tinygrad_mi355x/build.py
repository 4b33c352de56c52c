"""Build ``libtgm_mi355x.so`` from ``csrc/*.hip`` for gfx950 with hipcc.

Run as ``python -m tinygrad_mi355x.build``.  Objects are compiled in parallel into
``_build/`` and linked into ``tinygrad_mi355x/_lib/``.  Every HIP translation unit
is compiled with packed-FP32 instruction selection disabled.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
CSRC = ROOT / "csrc"
INCLUDE = ROOT.parent / "include"
BUILD = ROOT / "_build"
LIB = PACKAGE / "_lib" / "libtgm_mi355x.so"
ARCH = os.environ.get("MI355X_OFFLOAD_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
FLAGS = [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", f"-I{CSRC}", f"-I{INCLUDE}"]


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [HIPCC, *FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr}")
    return obj


VENDOR_SRC = ROOT / "vendor_bar" / "ck_mx_gemm_bar.cpp"
VENDOR_BIN = PACKAGE / "_lib" / "ck_mx_gemm_bar"
CK_INSTANCES = Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "lib" / "libdevice_gemm_operations.a"


def build_vendor_bar(verbose: bool = False) -> Path | None:
    """The benchmark's vendor comparison for the FP4 GEMM (Composable Kernel's prebuilt MXFP4
    instances, timed beside tgm_gemm_mx in one process); skipped where ROCm ships no instances."""
    if not CK_INSTANCES.exists():
        if verbose:
            print(f"skipped {VENDOR_BIN.name}: no {CK_INSTANCES}")
        return None
    VENDOR_BIN.parent.mkdir(exist_ok=True)
    tmp = VENDOR_BIN.with_name(VENDOR_BIN.name + ".tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-O2", "-std=c++17", "-w", str(VENDOR_SRC), "-o", str(tmp),
           f"-L{CK_INSTANCES.parent}", "-ldevice_gemm_operations", "-ldl"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {VENDOR_SRC.name}:\n{proc.stderr}")
    os.replace(tmp, VENDOR_BIN)
    if verbose:
        print(f"built {VENDOR_BIN}")
    return VENDOR_BIN


def build_library(verbose: bool = False) -> Path:
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    BUILD.mkdir(exist_ok=True)
    LIB.parent.mkdir(exist_ok=True)
    workers = min(len(sources), max(1, (os.cpu_count() or 2) // 2), 8)
    with concurrent.futures.ThreadPoolExecutor(workers + 1) as pool:
        vendor = pool.submit(build_vendor_bar, verbose)
        objects = list(pool.map(_compile, sources))
        vendor.result()
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build_library(verbose=True)
    sys.exit(0)
