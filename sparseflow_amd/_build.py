"""Build libsparseflow_hip.so in-tree with hipcc for gfx950.

The library is the C-ABI kernel library declared in include/sparseflow.h.
It is written next to this file so it travels with the source tree; it is
never installed into site-packages.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import tempfile
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO_DIR / "include"
LIB_NAME = "libsparseflow_hip.so"
LIB_PATH = PKG_DIR / LIB_NAME
SOURCES = ("sf_prescan.hip", "sf_conv.hip", "sf_rows.hip", "sf_flat.hip", "sf_px3.hip", "sf_lif.hip", "sf_bmm.hip", "sf_attn.hip", "sf_linmfma.hip", "sf_mfma_conv.hip", "sf_band.hip", "sf_rows_fused.hip", "sf_dense_mfma.hip", "sf_capi.hip")

ARCH = "gfx950"
# Packed-FP32 VALU ops are disabled on purpose: the library's float math is
# kept in scalar form on this target.
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build SparseFlow-AMD")
    return path


def _compile(src: Path, obj: Path) -> None:
    cmd = [hipcc(), *COMMON_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    # The host pass does not know the packed-fp32 feature name; that warning is
    # expected and filtered out of the log.
    noise = "is not a recognized feature for this target"
    errlines = [ln for ln in (res.stderr or "").splitlines() if noise not in ln]
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n" + "\n".join(errlines))
    if errlines:
        print("\n".join(errlines))


def build_library(verbose: bool = False) -> Path:
    """Compile every HIP source and link LIB_PATH.  Always rebuilds."""
    with tempfile.TemporaryDirectory(prefix="sf_build_") as tmp:
        objs = []
        jobs = []
        with cf.ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
            for name in SOURCES:
                src = CSRC / name
                obj = Path(tmp) / (name + ".o")
                objs.append(obj)
                jobs.append(ex.submit(_compile, src, obj))
            for j in jobs:
                j.result()
        tmp_lib = Path(tmp) / LIB_NAME
        cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp_lib)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError("link failed:\n" + res.stderr)
        # Atomic replace so a concurrently loaded copy is never half-written.
        staged = LIB_PATH.with_suffix(".so.tmp")
        shutil.copyfile(tmp_lib, staged)
        os.replace(staged, LIB_PATH)
    if verbose:
        print(f"[sparseflow_amd] built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build_library(verbose=True)
