"""Build libomhip.so (gfx950) and the C++ HIPBackend test program in-tree.

    python -m omnimatchdeeplearningtool_amd.build

Compiles every .hip / .cpp source under csrc/ with hipcc for gfx950 into
_build/, links omnimatchdeeplearningtool_amd/libomhip.so, and builds
_build/test_hip_backend from tests/cpp/test_hip_backend.cpp (the C++23 HAL
caller used by the GPU tests). Sources compile in parallel.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libomhip.so")
ARCH = os.environ.get("OMHIP_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
# Packed-fp32 VALU forms are disabled for all device code.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON = ["-O3", "-std=c++20", "-fPIC", "-Wall", "-Wno-unused-function", "-Wno-unused-variable"]

SOURCES = ["runtime.cpp", "eltwise.hip", "gemm_f32.hip", "conv.hip", "conv_stem.hip", "conv_wgrad.hip", "gemm_half.hip", "gemm_half_heads.hip", "train.hip",
           "pool.hip", "attention.hip", "infer.hip", "loss.hip", "mha.hip", "heads.hip"]
# conv tiles keep at most 128 accumulators per lane: forcing the VGPR form of
# the MFMA operands stops the register allocator from copying every
# accumulator between AGPRs and VGPRs on each trip of the mainloop (and, in
# the fused attention, every score back to VGPRs for the softmax).
EXTRA_FLAGS = {"conv.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"], "conv_stem.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"], "conv_wgrad.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
               "attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass warns about the device-only feature flag; drop that noise
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    return out


def _compile(src: str) -> str:
    path = os.path.join(CSRC, src)
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    if src.endswith(".hip"):
        cmd = [HIPCC, f"--offload-arch={ARCH}", *COMMON, *DEVICE_FLAGS, *EXTRA_FLAGS.get(src, []), "-c", path, "-o",
               obj]
    else:
        cmd = [HIPCC, *COMMON, "-c", path, "-o", obj]
    _run(cmd)
    return obj


def build(verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIB)
    if verbose:
        print(f"[omhip] built {LIB}")
    # C++ HAL caller (HIPBackend) test program, linked against libomhip.so
    test_src = os.path.join(ROOT, "tests", "cpp", "test_hip_backend.cpp")
    if os.path.exists(test_src):
        exe = os.path.join(BUILD, "test_hip_backend")
        _run([HIPCC, "-O2", "-std=c++23", f"-I{os.path.join(ROOT, 'include')}", test_src, "-o", exe,
              f"-L{PKG}", "-lomhip", "-Wl,-rpath,$ORIGIN/.."])
        if verbose:
            print(f"[omhip] built {exe}")
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
