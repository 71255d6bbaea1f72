#!/usr/bin/env python3
"""Builds the MI355X (gfx950) artefacts in-tree.

  build/libgyro_native.so   the gd_* C ABI (csrc/runtime/gyro_native.cpp)
  build/libgyro_moe.so      the C++ host engine above the ABI (host/*.cpp)
  build/kernels/<name>.co   one code object per pipeline (csrc/kernels/<name>.hip)

Every HIP compile disables packed fp32 instructions (-packed-fp32-ops).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
BUILD = HERE / "build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
NO_PACKED = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
KERNEL_DIR = HERE / "csrc" / "kernels"


def kernel_sources():
    return sorted(KERNEL_DIR.glob("*.hip"))


def compile_kernel(src: Path) -> str:
    out = BUILD / "kernels" / (src.stem + ".co")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-O3", "--genco", "-std=c++17", "-ffp-contract=fast",
           *NO_PACKED, "-I", str(KERNEL_DIR), "-o", str(out), str(src)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{src.name}:\n{r.stderr}")
    return out.name


def compile_runtime() -> str:
    out = BUILD / "libgyro_native.so"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-O2", "-fPIC", "-shared", "-std=c++17", *NO_PACKED,
           "-Wno-unused-result", "-Wno-unused-value", "-I", str(ROOT / "include"),
           "-o", str(out), str(HERE / "csrc" / "runtime" / "gyro_native.cpp")]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"runtime:\n{r.stderr}")
    return out.name


# Host sources compiled as HIP: engine.cpp defines the device scratch array of the
# no-allocation entry point (its only device code). The others are plain C++.
HIP_HOST_SOURCES = {"engine.cpp"}


def compile_host() -> str:
    out = BUILD / "libgyro_moe.so"
    srcs = sorted((HERE / "host").glob("*.cpp"))
    if not srcs:
        return "(no host sources)"
    objdir = BUILD / "host_obj"
    objdir.mkdir(parents=True, exist_ok=True)
    inc = ["-I", str(ROOT / "include"), "-I", str(HERE / "host")]
    objs = []
    for src in srcs:
        obj = objdir / (src.stem + ".o")
        if src.name in HIP_HOST_SOURCES:
            cmd = [HIPCC, f"--offload-arch={ARCH}", "-x", "hip", "-O2", "-fPIC", "-std=c++17", "-Wall",
                   "-Wno-unused-parameter", *NO_PACKED, *inc, "-c", "-o", str(obj), str(src)]
        else:
            cmd = ["g++", "-O2", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-parameter", *inc, "-c", "-o", str(obj),
                   str(src)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"host {src.name}:\n{r.stderr}")
        objs.append(str(obj))
    cmd = [HIPCC, "-shared", "-fPIC", "-o", str(out), *objs, f"-L{BUILD}", "-lgyro_native", "-Wl,-rpath,$ORIGIN"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"host link:\n{r.stderr}")
    return out.name


def build(verbose: bool = True) -> None:
    (BUILD / "kernels").mkdir(parents=True, exist_ok=True)
    jobs = min(8, os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(jobs) as ex:
        futs = [ex.submit(compile_kernel, s) for s in kernel_sources()]
        rt = ex.submit(compile_runtime)
        names = [f.result() for f in futs]
        names.append(rt.result())
    names.append(compile_host())
    if verbose:
        print("built:", " ".join(names))


if __name__ == "__main__":
    try:
        build()
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
