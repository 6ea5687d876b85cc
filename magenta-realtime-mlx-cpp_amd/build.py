"""Build ``libmrt_df.so`` (HIP kernels for gfx950 + host orchestration + C ABI).

Usage: python build.py [--jobs N]
The library is written next to this file; objects go to ``_build/``.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import pathlib
import shutil
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
LIB = HERE / "libmrt_df.so"

SOURCES = [
    "decode_kernels.hip",
    "sample_kernels.hip",
    "encoder_kernels.hip",
    "persist_kernels.hip",
    "stream_kernels.hip",
    "batch_kernels.hip",
    "spec_kernels.hip",
    "codec_kernels.hip",
    "coca_kernels.hip",
    "probe_kernels.hip",
    "safetensors.cpp",
    "model.cpp",
    "stream.cpp",
    "batch.cpp",
    "codec.cpp",
    "coca.cpp",
    "api.cpp",
]

ARCH = os.environ.get("MRT_OFFLOAD_ARCH", "gfx950")
COMMON = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Wall", "-Wno-unused-result"]
# Packed fp32 VALU ops are disabled for every HIP translation unit.
DEVICE = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and pathlib.Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found")


def compile_one(src: str) -> pathlib.Path:
    obj = BUILD / (src + ".o")
    cmd = [hipcc(), *COMMON, "-c", str(CSRC / src), "-o", str(obj)]
    if src.endswith(".hip"):
        cmd[1:1] = ["-x", "hip"]
        cmd += DEVICE
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                    if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {src}\n{' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)
    return obj


def build(jobs: int = 6) -> pathlib.Path:
    BUILD.mkdir(exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), "-shared", f"--offload-arch={ARCH}", "-o", str(tmp), *map(str, objs),
           "-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed\n{' '.join(cmd)}\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=6)
    a = ap.parse_args()
    print(build(a.jobs))


if __name__ == "__main__":
    main()
