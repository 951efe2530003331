#!/usr/bin/env python3
"""Build the two native libraries of the astc_kv package in place:

* astc_kv/libakv_astc.so   CPU ASTC codec behind the akv_* bridge (g++)
* astc_kv/libastckv_hip.so gfx950 decode-attention kernels + C-ABI (hipcc)

Run `python astc-kv_amd/build.py` (both) or with --cpu-only / --hip-only.
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
PKG = HERE / "astc_kv"
CODEC = HERE / "csrc" / "codec"
HIP = HERE / "csrc" / "hip"
INCLUDE = ROOT / "include"

CODEC_SOURCES = ["astc_format.cpp", "astc_decode.cpp", "astc_encode.cpp", "bridge.cpp"]
HIP_SOURCES = [HIP / "decode_attention.hip", HIP / "paged_attention.hip", CODEC / "astc_format.cpp"]
ARCH = os.environ.get("PYTORCH_ROCM_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libastckv_hip.so)")


def run(cmd):
    print("+", " ".join(str(c) for c in cmd), flush=True)
    subprocess.run([str(c) for c in cmd], check=True)


def build_cpu():
    out = PKG / "libakv_astc.so"
    run(["g++", "-O3", "-std=c++17", "-Wall", "-Wextra", "-fPIC", "-shared", "-ffp-contract=off",
         f"-I{INCLUDE}", f"-I{CODEC}", *[CODEC / s for s in CODEC_SOURCES], "-o", out])
    return out


def build_hip():
    """Each source compiled to an object in parallel (the kernel translation
    units take a minute or more each), then linked."""
    from concurrent.futures import ThreadPoolExecutor

    out = PKG / "libastckv_hip.so"
    tmp = out.with_suffix(".so.tmp")
    objdir = HERE / "_build"
    objdir.mkdir(exist_ok=True)
    flags = [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
             # Packed FP32 instructions are kept out of every kernel.
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             f"-I{INCLUDE}", f"-I{CODEC}", f"-I{HIP}"]
    objs = [objdir / (src.stem + ".o") for src in HIP_SOURCES]
    with ThreadPoolExecutor(max_workers=len(HIP_SOURCES)) as pool:
        for f in [pool.submit(run, [hipcc(), *flags, "-c", src, "-o", obj]) for src, obj in zip(HIP_SOURCES, objs)]:
            f.result()
    run([hipcc(), f"--offload-arch={ARCH}", "-fPIC", "-shared", *objs, "-o", tmp])
    tmp.replace(out)
    return out


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--cpu-only", action="store_true")
    ap.add_argument("--hip-only", action="store_true")
    args = ap.parse_args(argv)
    if not args.hip_only:
        build_cpu()
    if not args.cpu_only:
        build_hip()


if __name__ == "__main__":
    sys.exit(main())
