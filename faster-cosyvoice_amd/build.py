"""Build libfcvdit.so (gfx950 HIP kernels + C ABI) in-tree with hipcc.

Usage: ``python faster-cosyvoice_amd/build.py`` or ``build_library()`` from Python.
The shared library lands next to this file so that it travels with the source tree.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
INCLUDE = PKG_DIR.parent / "include"
LIB_NAME = "libfcvdit.so"
ARCH = "gfx950"

SOURCES = ["gemm.hip", "gemv.hip", "attention.hip", "conv.hip", "elementwise.hip", "frontend.hip",
           "hift.hip", "hift_capi.hip", "capi.hip"]

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-result",
    # packed fp32 VALU forms are kept out of the generated code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build libfcvdit.so")
    return path


def library_path() -> Path:
    return PKG_DIR / LIB_NAME


# The DiT sources compile without floating-point contraction: every fused multiply-add there is
# an explicit fmaf.  With contraction allowed the compiler fuses a product and its fp16
# conversion into v_fma_mix (one rounding instead of two) in some template instantiations and
# not in others, so an element's fp16 bits would depend on the GEMM tile shape, and with it on
# the batch a document is packed with.
EXACT_SOURCES = {"gemm.hip", "gemv.hip", "attention.hip", "conv.hip", "elementwise.hip", "capi.hip"}
EXACT_FLAGS = ["-ffp-contract=off"]


def _compile(src: Path, obj: Path) -> None:
    extra = EXACT_FLAGS if src.name in EXACT_SOURCES else []
    cmd = [hipcc(), *HIPCC_FLAGS, *extra, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o",
           str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr}")
    noise = [ln for ln in res.stderr.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
    if noise:
        sys.stderr.write(f"[{src.name}]\n" + "\n".join(noise) + "\n")


def build_library(verbose: bool = False) -> Path:
    """Compile every kernel source for gfx950 and link libfcvdit.so (always rebuilds)."""
    build_dir = PKG_DIR / "_build"
    build_dir.mkdir(exist_ok=True)
    objs = [build_dir / (Path(s).stem + ".o") for s in SOURCES]
    jobs = min(len(SOURCES), max(1, int(os.environ.get("MAX_JOBS", "8"))))
    with ThreadPoolExecutor(jobs) as pool:
        list(pool.map(lambda so: _compile(CSRC / so[0], so[1]), zip(SOURCES, objs)))
    out = library_path()
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    build_library(verbose=True)
