"""Build recipe of the pjrtx ROCm plugin (libpjrtx_rocm_plugin.so), in-tree.

Compiles every C++/HIP source under pjrtx_amd/csrc with hipcc for gfx950 and
links one shared library exporting GetPjrtApi (include/pjrt_c_api.h) and the
pjrtx_hip_* C ABI (include/pjrtx_hip.h). The device helper header used by the
generated fusion kernels is embedded as a string so the library is
self-contained on the GPU box.

Usage: python -m pjrtx_amd.build  [--jobs N] [--debug]
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import pathlib
import shutil
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libpjrtx_rocm_plugin.so"
ARCH = os.environ.get("PJRTX_OFFLOAD_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

# Packed f32 instructions stay disabled in every HIP translation unit.
COMMON = [
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    "-Wno-unused-but-set-variable",
    "-fvisibility=hidden",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", str(CSRC),
    "-I", str(BUILD),
    "-I", str(ROOT / "include"),
]


def sources() -> list[pathlib.Path]:
    out = sorted(CSRC.glob("*.cc")) + sorted(CSRC.glob("kernels/*.hip"))
    return out


def embed_device_header() -> pathlib.Path:
    """Writes fusion_device_inc.h holding kernels/fusion_device.h as a string."""
    text = (CSRC / "kernels" / "fusion_device.h").read_text()
    delim = "PJRTXDEV"
    assert f"){delim}\"" not in text
    BUILD.mkdir(exist_ok=True)
    out = BUILD / "fusion_device_inc.h"
    body = (
        "// Generated from kernels/fusion_device.h by pjrtx_amd/build.py.\n#pragma once\n"
        f"static const char kFusionDeviceHeader[] = R\"{delim}(\n{text}\n){delim}\";\n"
    )
    if not out.exists() or out.read_text() != body:
        out.write_text(body)
    return out


def compile_one(src: pathlib.Path, debug: bool) -> pathlib.Path:
    obj = BUILD / (src.name + ".o")
    opt = ["-O0", "-g"] if debug else ["-O3"]
    lang = ["-x", "hip"] if src.suffix == ".hip" else []
    cmd = [HIPCC, *COMMON, *opt, *lang, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {src.name}\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def build(jobs: int | None = None, debug: bool = False, verbose: bool = True) -> pathlib.Path:
    embed_device_header()
    srcs = sources()
    jobs = jobs or min(8, os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: compile_one(s, debug), srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "-shared", f"--offload-arch={ARCH}", "-fPIC", *map(str, objs), "-o", str(tmp),
           "-lhiprtc", "-lhipblaslt", "-Wl,--no-undefined", "-Wl,-rpath,/opt/rocm/lib"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB.relative_to(ROOT)} ({LIB.stat().st_size // 1024} KiB, {len(srcs)} sources, arch {ARCH})")
    return LIB


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--debug", action="store_true")
    a = ap.parse_args()
    build(a.jobs, a.debug)
    return 0


if __name__ == "__main__":
    sys.exit(main())
