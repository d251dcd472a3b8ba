"""Build libgollek_hip.so (the C-ABI library of the gfx950 kernels) in-tree.

The library is compiled with hipcc for gfx950 only.  Packed-FP32 instruction
selection is disabled for every HIP translation unit.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_DIR = PACKAGE_DIR.parent
CSRC_DIR = PACKAGE_DIR / "csrc"
INCLUDE_DIR = REPO_DIR / "include"
LIB_PATH = PACKAGE_DIR / "libgollek_hip.so"
# Measurement kernels of bench.py --ceilings (not part of the product library).
CEILING_LIB_PATH = PACKAGE_DIR / "libgollek_ceiling.so"
CEILING_SOURCES = ("hbm_ceiling.hip",)
OBJ_DIR = PACKAGE_DIR / "_build"

HIP_SOURCES = (
    "gguf_capi.hip",
    "gguf_dequant.hip",
    "gguf_file.hip",
    "gguf_gemv.hip",
    "gguf_k56.hip",
    "gguf_gemv_mfma.hip",
    "gguf_gemv_q6k_mfma.hip",
    "gguf_gemv_ring.hip",
    "gguf_gemm.hip",
    "gguf_gemm_tile.hip",
    "gguf_moe.hip",
    "gguf_moe_mfma.hip",
    "gguf_moe_router.hip",
)

ARCH = "gfx950"


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the gfx950 library cannot be built")


def compile_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-Wall",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        f"-I{INCLUDE_DIR}",
        f"-I{CSRC_DIR}",
    ]


def _compile_one(hipcc: str, src: Path, obj: Path) -> tuple[Path, str]:
    cmd = [hipcc, *compile_flags(), "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    log = "\n".join(l for l in (proc.stdout + proc.stderr).splitlines()
                    if "packed-fp32-ops" not in l and l.strip())
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{log}")
    return obj, log


def build_library(verbose: bool = False) -> Path:
    """Compile every HIP source and link libgollek_hip.so (and the measurement
    library libgollek_ceiling.so); returns the product library's path."""
    _link(CEILING_SOURCES, CEILING_LIB_PATH, verbose)
    return _link(HIP_SOURCES, LIB_PATH, verbose)


def _link(names, lib_path: Path, verbose: bool) -> Path:
    hipcc = _hipcc()
    OBJ_DIR.mkdir(exist_ok=True)
    sources = [CSRC_DIR / s for s in names if (CSRC_DIR / s).exists()]
    jobs = min(len(sources), max(1, min(16, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        results = list(pool.map(
            lambda s: _compile_one(hipcc, s, OBJ_DIR / (s.stem + ".o")), sources))
    for obj, log in results:
        if verbose and log:
            print(f"[{obj.name}] {log}", file=sys.stderr)
    tmp = lib_path.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC",
           *[str(o) for o, _ in results], "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}{proc.stderr}")
    os.replace(tmp, lib_path)
    return lib_path


if __name__ == "__main__":
    print(build_library(verbose=True))
