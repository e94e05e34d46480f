"""Builds libnuq.so (the HIP kernels + C-ABI shim) for gfx950, in-tree.

hipcc cross-compiles without a GPU. Flags:
  -Xclang -target-feature -Xclang -packed-fp32-ops  no packed-FP32 VALU ops
  -fno-gpu-flush-denormals-to-zero                  IEEE denormals (F16 scales)
  -ffp-contract=fast is the hipcc default; the exact decoders switch
  contraction off locally with `#pragma clang fp contract(off)`.
"""
from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libnuq.so"
SOURCES = ["api.hip", "gemv.hip", "gemv_int.hip", "gemm.hip", "sampling.hip", "quantize.cpp", "gguf.cpp"]
ARCH = "gfx950"


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    return path


def build(verbose: bool = False) -> Path:
    build_dir = PKG / "_build"
    build_dir.mkdir(exist_ok=True)
    common = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function", "-I", str(PKG.parent / "include")]
    objects = []
    procs = []
    for src in SOURCES:
        obj = build_dir / (Path(src).stem + ".o")
        if src.endswith(".hip"):
            cmd = [hipcc(), "-x", "hip", f"--offload-arch={ARCH}", *common,
                   "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                   "-fno-gpu-flush-denormals-to-zero", "-munsafe-fp-atomics",
                   "-c", str(CSRC / src), "-o", str(obj)]
        else:
            cmd = [hipcc(), *common, "-pthread", "-c", str(CSRC / src), "-o", str(obj)]
        objects.append(obj)
        procs.append((src, cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
    failed = []
    for src, cmd, p in procs:
        out, _ = p.communicate()
        if verbose or p.returncode != 0:
            print(f"[nuq build] {src}:\n{out}")
        if p.returncode != 0:
            failed.append(src)
    if failed:
        raise RuntimeError(f"hipcc failed for {failed}")
    tmp = LIB.with_suffix(".so.tmp")
    link = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-pthread", *map(str, objects), "-o", str(tmp)]
    subprocess.run(link, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
