"""Builds the HIP library libferro_gpu.so in-tree for gfx950 with hipcc.

Run as `python -m ferrolm_amd.build` (or through __graft_entry__.build()).
It compiles every time it is called. `--stamps` builds the same sources with
the in-kernel timeline (-DFERRO_STAMPS) into libferro_gpu_stamps.so instead, a
measurement aid loaded when FERRO_STAMPS=1 (ferrolm_amd.stamps). Packed FP32 instructions are disabled
(-packed-fp32-ops) for every device compilation, and floating-point
contraction is off (-ffp-contract=off): a fused multiply-add happens only
where the source writes fmaf, as in the reference's mul_add. Besides matching
the reference's operation order, this keeps lanes that combine values across
the wave (shuffle sums) bit-identical, which the activation pieces rely on.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "libferro_gpu.so"
SOURCES = ["kernels.hip", "sampling.hip", "quant.hip", "api.hip"]
HOST_SOURCES = ["host.cpp"]  # plain C++ (g++), no contraction: exact load-time arithmetic
ARCH = os.environ.get("FERRO_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and Path(c).exists():
            return c
    raise RuntimeError("hipcc not found")


def flags() -> list[str]:
    return [f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function",
            "-ffp-contract=off", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            f"-I{ROOT / 'include'}", f"-I{CSRC}"]


def build(verbose: bool = False, stamps: bool = False) -> Path:
    obj = OBJ.with_name(OBJ.name + "_stamps") if stamps else OBJ
    lib_path = LIB.with_name("libferro_gpu_stamps.so") if stamps else LIB
    extra = ["-DFERRO_STAMPS"] if stamps else []
    obj.mkdir(exist_ok=True)
    cc = hipcc()

    def compile_one(src: str) -> Path:
        out = obj / (Path(src).stem + ".o")
        cmd = [cc, *flags(), *extra, "-c", str(CSRC / src), "-o", str(out)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr}")
        if verbose and r.stderr.strip():
            print(r.stderr, file=sys.stderr)
        return out

    def compile_host(src: str) -> Path:
        out = obj / (Path(src).stem + ".o")
        cmd = ["g++", "-O2", "-fPIC", "-std=c++17", "-ffp-contract=off", "-pthread", "-Wall",
               f"-I{ROOT / 'include'}", "-c", str(CSRC / src), "-o", str(out)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"g++ failed on {src}:\n{r.stderr}")
        return out

    with ThreadPoolExecutor(max_workers=len(SOURCES) + len(HOST_SOURCES)) as ex:
        futs = [ex.submit(compile_one, s) for s in SOURCES] + [ex.submit(compile_host, s) for s in HOST_SOURCES]
        objs = [f.result() for f in futs]
    tmp = lib_path.with_suffix(".so.tmp")
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-pthread", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, lib_path)
    return lib_path


if __name__ == "__main__":
    print(build(verbose=True, stamps="--stamps" in sys.argv[1:]))
