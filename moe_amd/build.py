"""Build libmoe_hip.so (and the bench's probes, libmoe_diag.so) in-tree for gfx950.

    python -m moe_amd.build            # compile every source, link the library

Each HIP source is compiled separately (in parallel) and linked into
``moe_amd/libmoe_hip.so``.  The routing and combine kernels are compiled with
``-ffp-contract=off``: they reproduce the reference's rounding step by step, so
no multiply and add may be fused behind their back.  Every device compile
disables packed fp32 ops (hipcc emits them on its own from plain float code).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libmoe_hip.so"
# The bench's measurement probes, a library of their own (not the layer ABI).
DIAG_SRC = PKG / "diag" / "diag.hip"
DIAG_LIB = PKG / "libmoe_diag.so"
ARCH = os.environ.get("MOE_OFFLOAD_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
# Sources whose arithmetic must follow the reference operation by operation.
EXACT = {"route.hip", "combine.hip", "expert_gemv.hip", "expert_decode.hip"}
# Per-source code-generation options.  expert_stream.hip keeps its MFMA
# accumulators in VGPRs: with the accumulators in AGPRs the register
# allocator rotates them between registers every loop iteration (dozens of
# v_accvgpr moves per step), in VGPRs the loop has none.
EXTRA = {"expert_stream.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}

SOURCES = ["route.hip", "expert_gemv.hip", "expert_decode.hip", "expert_batch.hip", "expert_mfma.hip",
           "expert_stream.hip", "combine.hip",
           "model_ops.hip", "moe_abi.hip"]
HOST_SOURCES = ["host_util.cpp", "container.cpp"]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"build step failed: {' '.join(cmd)}")


def _compile_hip(src: str) -> Path:
    obj = BUILD / (src + ".o")
    flags = list(HIP_FLAGS)
    if src in EXACT:
        flags.append("-ffp-contract=off")
    flags += EXTRA.get(src, [])
    _run([HIPCC, *flags, "-c", str(CSRC / src), "-o", str(obj)])
    return obj


def _compile_host(src: str) -> Path:
    obj = BUILD / (src + ".o")
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-pthread", "-ffp-contract=off", "-Wall",
          "-c", str(CSRC / src), "-o", str(obj)])
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every source and link ``libmoe_hip.so``; returns its path."""
    BUILD.mkdir(exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as pool:
        futs = [pool.submit(_compile_hip, s) for s in SOURCES]
        futs += [pool.submit(_compile_host, s) for s in HOST_SOURCES]
        objs = [f.result() for f in futs]
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-pthread", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, LIB)
    dtmp = DIAG_LIB.with_suffix(".so.tmp")
    _run([HIPCC, *HIP_FLAGS, "-shared", str(DIAG_SRC), "-o", str(dtmp)])
    os.replace(dtmp, DIAG_LIB)
    if verbose:
        print(f"built {LIB} and {DIAG_LIB.name}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
