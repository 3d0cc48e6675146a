"""Builds libdgg_hip.so (the gfx950 kernels + C ABI of include/dgg.h) in-tree with hipcc.

    python -m deepgengraph_amd.build            # compile every csrc/*.hip, link the shared library

Objects go to deepgengraph_amd/_build/, the library to deepgengraph_amd/libdgg_hip.so. hipcc
cross-compiles for gfx950 without a GPU present.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_NAME = "libdgg_hip.so"
LIB_PATH = PKG_DIR / LIB_NAME
ARCH = os.environ.get("DGG_OFFLOAD_ARCH", "gfx950")

# Packed-fp32 VALU ops (v_pk_{add,mul,fma}_f32) are disabled for all device code: some of their forms
# have produced silently wrong results on the target machines. The host pass warns that it does not
# know the feature; that warning is harmless.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


# Per-source extra flags. The attention kernels are long unrolled MFMA / LDS-read sequences; LLVM's
# iterative ILP machine scheduler issues the LDS fragment reads further ahead of the MFMAs that consume them
# than the default occupancy-driven scheduler (measured on MI355X: +3% prefill at head_dim 128, +10% at 256).
EXTRA_FLAGS = {
    # -amdgpu-mfma-vgpr-form: at one wave per SIMD (head_dim 256) LLVM otherwise writes MFMA results to AGPRs and
    # copies them out for the softmax; with it the head_dim-256 forward runs 0.98 instead of 1.09 ms (config 3)
    "attention.hip": ["-mllvm", "-amdgpu-sched-strategy=iterative-ilp", "-mllvm", "-amdgpu-mfma-vgpr-form"],
    "attention_d256.hip": ["-mllvm", "-amdgpu-sched-strategy=iterative-ilp", "-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found: the ROCm toolchain is required to build libdgg_hip.so")
    return exe


def _compile(src: Path, verbose: bool) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [_hipcc(), *HIPCC_FLAGS, *EXTRA_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")
    return obj


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compiles every csrc/*.hip for gfx950 and links deepgengraph_amd/libdgg_hip.so. Always rebuilds."""
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
