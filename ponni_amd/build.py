"""Build libponni_hip.so (gfx950) in-tree with hipcc.

Every HIP source is compiled for gfx950 only, with packed-fp32 VALU ops
disabled (the compiler otherwise fuses scalar fp32 pairs into v_pk_* forms),
and linked into ponni_amd/libponni_hip.so next to this file.
"""
from __future__ import annotations

import concurrent.futures
import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OBJ = HERE / "_build"
LIB = HERE / "libponni_hip.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = [
    "plan.cpp",
    "file_abi.cpp",
    "kernels_generic.hip",
    "kernels_narrow.hip",
    "kernels_mfma_dispatch.cpp",
    "kernels_mfma_f32_mt2.hip",
    "kernels_mfma_f32_mt4.hip",
    "kernels_mfma_f32_mt8.hip",
    "kernels_fill.hip",
]

COMMON = [
    "-O3",
    "-std=c++20",
    "-fPIC",
    "--offload-arch=gfx950",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-result",
]


def _compile(src: Path, obj: Path) -> None:
    cmd = [HIPCC, *COMMON, "-c", str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd[1:1] = ["-x", "hip"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr[-6000:]}")


def build_library(jobs: int | None = None, verbose: bool = True) -> Path:
    OBJ.mkdir(exist_ok=True)
    jobs = jobs or min(8, os.cpu_count() or 4)
    objs = []
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        futs = []
        for name in SOURCES:
            src = CSRC / name
            obj = OBJ / (name + ".o")
            objs.append(obj)
            futs.append(pool.submit(_compile, src, obj))
        for f in futs:
            f.result()
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "-shared", "-fPIC", "--offload-arch=gfx950", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr[-6000:]}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build_library()
