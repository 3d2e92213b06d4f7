"""Build libw4h.so (HIP for gfx950 + host runtime) in-tree.

Usage: python -m whisper4j_amd.build   (or whisper4j_amd.build.build()).
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libw4h.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# Packed FP32 (v_pk_*_f32) is disabled for all device code.
DEVICE_FLAGS = ["--offload-arch=" + ARCH, "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
                "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
CLANG = os.environ.get("W4H_HOST_CXX", "/opt/rocm/lib/llvm/bin/clang++")
# Host-only translation units: plain C++ against the HIP runtime API (no device code).
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include"]
# Step-kernel instances (rows x weight type x register rounds; "_s": sampled runs), one translation unit each so they
# compile in parallel; the shared device code is w4h_kernels.h.
STEP_VARIANTS = ["1_f16_r2", "1_f16_r3", "1_q8_r2", "8_f16_r2", "8_f16_r3", "8_q8_r2", "1_f16_r2_s", "1_f16_r3_s",
                 "1_q8_r2_s"]
SOURCES = ([("w4h_device.hip", HIPCC, DEVICE_FLAGS), ("w4h_wide.hip", HIPCC, DEVICE_FLAGS),
            ("w4h_xkv.hip", HIPCC, DEVICE_FLAGS), ("w4h_sample.hip", HIPCC, DEVICE_FLAGS), ("w4h_encoder.hip", HIPCC, DEVICE_FLAGS)] + [(f"w4h_step_{v}.hip", HIPCC, DEVICE_FLAGS) for v in STEP_VARIANTS] +
           [("w4h_api.cpp", CLANG, HOST_FLAGS), ("w4h_ggml.cpp", CLANG, HOST_FLAGS), ("w4h_decode.cpp", CLANG, HOST_FLAGS), ("w4h_encoder_api.cpp", CLANG, HOST_FLAGS)])


def _compile(src, cxx, flags):
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [cxx, *flags, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(ln for ln in (r.stdout + r.stderr).splitlines() if noise not in ln)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{err}")
    return obj, err


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4)) as ex:
        results = list(ex.map(lambda s: _compile(*s), SOURCES))
    if verbose:
        for _, msg in results:
            if msg.strip():
                print(msg, file=sys.stderr)
    objs = [o for o, _ in results]
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=" + ARCH, "-shared", "-fPIC", *objs, "-o", tmp, "-lz"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
