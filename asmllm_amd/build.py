"""Builds libasmllm.so (HIP, gfx950) in-tree with hipcc.

The library replaces the reference's build/libasmllm.so (build_kernel.py:39-139,
export list :85-104).  Every translation unit is compiled for gfx950 only,
with packed-fp32 instructions disabled, then linked into one shared object
under asmllm_amd/lib/.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = REPO / "include"
OBJ_DIR = PKG / "_obj"
LIB_DIR = PKG / "lib"
LIB_PATH = LIB_DIR / "libasmllm.so"

SOURCES = [
    "matvec.hip",
    "matvec_mfma.hip",
    "measure.hip",
    "decode_ops.hip",
    "quant.hip",
    "gemm.hip",
    "capi.hip",
]

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-mllvm",
    "-amdgpu-mfma-vgpr-form",
    # the first 16 dwords of every kernel's arguments arrive in SGPRs at wave
    # launch instead of through a scalar load (gfx950 firmware preloads them;
    # the compiler keeps a loading prologue for firmware that does not)
    "-mllvm",
    "-amdgpu-kernarg-preload-count=16",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: install ROCm or set HIPCC")


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(
        line for line in (res.stdout + res.stderr).splitlines()
        # The host pass of hipcc does not know the device feature flag.
        if "packed-fp32-ops' is not a recognized feature" not in line
    )
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def build_library(jobs: int | None = None) -> Path:
    hipcc = _hipcc()
    OBJ_DIR.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    objs = [OBJ_DIR / (Path(s).stem + ".o") for s in SOURCES]

    def compile_one(src_obj):
        src, obj = src_obj
        _run([hipcc, *HIPCC_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])

    with cf.ThreadPoolExecutor(max_workers=jobs or min(8, len(SOURCES))) as ex:
        list(ex.map(compile_one, zip(SOURCES, objs)))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


REFERENCE = Path("/root/reference")


def build_oracle() -> Path:
    """Compiles the CPU oracle (test infrastructure) with its Makefile, and,
    where the reference tree is present, the reference's own GGUF loader into
    oracle/_ref/ (the checker of the GGUF reader)."""
    oracle_dir = REPO / "oracle"
    _run(["make", "-s", "-C", str(oracle_dir), "-B", "liboracle.so"])
    if (REFERENCE / "src" / "loader" / "gguf_loader.c").exists():
        _run(["make", "-s", "-C", str(oracle_dir), "-B", f"REF={REFERENCE}", "_ref/libgguf_ref.so"])
    return oracle_dir / "liboracle.so"


def main() -> None:
    print(f"built {build_library()}")
    print(f"built {build_oracle()}")


if __name__ == "__main__":
    main()
