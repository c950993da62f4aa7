"""Build libtpr_attn.so in-tree with hipcc for gfx950 (no JIT, no torch extension).

``python -m bridge_amd._build`` or ``bridge_amd._build.build()`` compiles every
source under ``bridge_amd/csrc`` and links ``bridge_amd/libtpr_attn.so``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_PATH = os.path.join(PKG_DIR, "libtpr_attn.so")
ARCH = os.environ.get("TPR_OFFLOAD_ARCH", "gfx950")

# (source, object, extra flags). The 16x16x32 family is compiled per head size
# and kernel group (TPR_M16_GROUP bits: 1 = forward and delta, 2 = dK/dV and
# its reduction, 4 = dQ). -amdgpu-mfma-vgpr-form builds the MFMAs with their
# accumulators in VGPRs; the default form puts them in AGPRs, and a kernel then
# copies each score tile out for its softmax. Measured per group (forward /
# dK/dV / dQ ms, default -> VGPR form): head_dim 64 at prefix 4096 + 4 x 4096,
# GQA 32/8, every group gains; head_dim 256 at the Qwen3.5 shape, forward 1.08
# -> 0.96 and dK/dV 2.39 -> 2.03 gain, dQ 1.28 -> 1.39 loses and keeps the
# default form.
_VGPR_FORM = ["-mllvm", "-amdgpu-mfma-vgpr-form"]
HIP_UNITS = [
    ("tpr_abi.hip", "tpr_abi", []),
    ("tpr_simt.hip", "tpr_simt", []),
    ("tpr_mfma.hip", "tpr_mfma", []),
    ("tpr_mfma16.hip", "tpr_mfma16_d64", ["-DTPR_M16_HEAD_DIM=64", "-DTPR_M16_GROUP=7", *_VGPR_FORM]),
    ("tpr_mfma16.hip", "tpr_mfma16_d256_fwd", ["-DTPR_M16_HEAD_DIM=256", "-DTPR_M16_GROUP=1", *_VGPR_FORM]),
    ("tpr_mfma16.hip", "tpr_mfma16_d256_dkdv", ["-DTPR_M16_HEAD_DIM=256", "-DTPR_M16_GROUP=2", *_VGPR_FORM]),
    ("tpr_mfma16.hip", "tpr_mfma16_d256_dq", ["-DTPR_M16_HEAD_DIM=256", "-DTPR_M16_GROUP=4"]),
]
CXX_SOURCES = ["tpr_plan.cpp"]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; set HIPCC or install ROCm")


def _hip_flags():
    return [
        f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
        "-Wno-unused-function", "-Wno-unused-variable",
        # packed fp32 VALU forms are kept out of every kernel
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", os.path.join(PKG_DIR, "..", "include"),
    ]


def _run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    lines = [ln for ln in proc.stdout.splitlines() if "packed-fp32-ops" not in ln]
    return proc.returncode, "\n".join(lines)


def build(verbose: bool = False, extra_flags=()) -> str:
    """Compile all sources and link the shared library; returns its path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    hipcc = _hipcc()
    jobs = []
    for src, name, unit_flags in HIP_UNITS:
        obj = os.path.join(BUILD_DIR, name + ".o")
        jobs.append((obj, [hipcc, *_hip_flags(), *unit_flags, *extra_flags, "-c", os.path.join(CSRC, src), "-o", obj]))
    for src in CXX_SOURCES:
        obj = os.path.join(BUILD_DIR, src.rsplit(".", 1)[0] + ".o")
        jobs.append((obj, ["g++", "-O2", "-std=c++17", "-fPIC", "-Wall", "-I",
                           os.path.join(PKG_DIR, "..", "include"), "-c", os.path.join(CSRC, src), "-o", obj]))
    with ThreadPoolExecutor(max_workers=min(8, len(jobs))) as pool:
        results = list(pool.map(lambda job: _run(job[1]), jobs))
    for (obj, cmd), (rc, out) in zip(jobs, results):
        if verbose and out:
            print(out)
        if rc != 0:
            raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{out}")
    tmp = LIB_PATH + ".tmp"
    rc, out = _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp,
                    *[obj for obj, _ in jobs]])
    if rc != 0:
        raise RuntimeError(f"link failed:\n{out}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
