"""Ahead-of-time build of the gfx950 C-ABI library ``libkotflash_amd.so``.

Each ``csrc/*.hip`` / ``csrc/*.cpp`` file is compiled by ``hipcc`` for
``--offload-arch=gfx950`` into ``_build/`` and linked into
``kotflash_amd/libkotflash_amd.so`` next to this file. There is no JIT step:
the reference builds its CUDA append op lazily with
``torch.utils.cpp_extension.load`` (reference kotflash/_cuda_append.py:9-28);
here the library is built once, in-tree, and loaded with ctypes.

Usage: ``python -m kotflash_amd.build`` (or ``build()`` from Python).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_NAME = "libkotflash_amd.so"
LIB_PATH = PKG_DIR / LIB_NAME
ARCH = "gfx950"

# -packed-fp32-ops: keep the compiler from forming packed fp32 VALU ops.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# Per-file additions: the VGPR form of the MFMA builtins. LLVM chooses the
# accumulator register class of MFMAs per function; where a kernel also needs
# accumulation registers (AGPRs) it otherwise writes every MFMA result there,
# and the softmax then reads S (and dP) back with one v_accvgpr_read per
# element. With the VGPR form those results land in VGPRs. bwd.hip keeps the
# dK/dV accumulators in AGPRs through inline-assembly MFMAs (dkdv_mfma_acc).
# Measured on MI355X, outputs bit-identical: dK/dV -1.4% (config 3) to -4.3%
# (config 4, D = 72); the split forms of dQ -4 to -7% and of the forward -5%
# (config 1) to -8%; the D = 96 / 128 decodes -2 to -3%. Kernels that used no
# AGPRs compile as before.
FILE_FLAGS = {
    "bwd.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "fwd.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "decode.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; set HIPCC or install ROCm")


def sources() -> list[Path]:
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


def _compile(src: Path, verbose: bool) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc(), *HIP_FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass reports the device-only feature flag as unknown; that
    # line is expected and carries no information.
    noise = "is not a recognized feature for this target"
    msgs = [ln for ln in (res.stdout + res.stderr).splitlines() if noise not in ln]
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n" + "\n".join(msgs))
    if verbose and msgs:
        print("\n".join(msgs), flush=True)
    return obj


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every source and link ``libkotflash_amd.so``; returns its path."""
    BUILD_DIR.mkdir(exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no sources under {CSRC}")
    jobs = jobs or min(len(srcs), max(1, min(16, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(lambda s: _compile(s, verbose), srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("link failed:\n" + res.stdout + res.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
