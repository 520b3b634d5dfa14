"""Builds the native library in-tree.

Three artefacts, all written next to this file:

* ``moearc_attn_gfx950.co`` -- the device code object (every kernel, one translation unit), built
  by ``hipcc --genco`` for gfx950 only and loaded at context creation with ``hipModuleLoad``;
* ``libmoearc_attn.so`` -- the host runtime behind the C ABI in ``include/moearc_attn.h`` and the
  KV page pool of ``include/moearc_kv.h``, built by the host compiler against the HIP runtime API
  (no device code in it);
* ``launch_overhead`` -- the submission-cost measurement of the reference's
  ``examples/launch_overhead.rs``, a C++ program over the C ABI (run by ``bench.py``).

Run ``python -m moearc_amd.build`` (or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

CODE_OBJECT = os.path.join(HERE, "moearc_attn_gfx950.co")
LIBRARY = os.path.join(HERE, "libmoearc_attn.so")
LAUNCH_OVERHEAD = os.path.join(HERE, "launch_overhead")

# Packed-FP32 instructions stay disabled (v_pk_fma_f32 and friends are not emitted).
# -fno-honor-nans: no kernel tests for NaN (the f16 codec classifies NaNs by their bits), and
# without it every fmaxf is preceded by a NaN-quieting v_max x,x.
# MFMA accumulators stay in VGPRs: with the AGPR form the compiler copies every accumulator to
# VGPRs and back around each rescale branch of the prefill loop.
HIPCC_FLAGS = [
    "--offload-arch=gfx950", "--genco", "--no-gpu-bundle-output", "-O3", "-std=c++17",
    "-fno-honor-nans", "-mllvm", "-amdgpu-mfma-vgpr-form=1", "-mllvm", "-amdgpu-kernarg-preload-count=14",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}")
    return res


def build(verbose: bool = False) -> None:
    hipcc = shutil.which("hipcc") or os.path.join(ROCM, "bin", "hipcc")
    tmp_co = CODE_OBJECT + ".tmp"
    _run([hipcc, *HIPCC_FLAGS, "-I", CSRC, os.path.join(CSRC, "moearc_kernels.hip"), "-o", tmp_co],
         verbose)
    os.replace(tmp_co, CODE_OBJECT)
    cxx = os.environ.get("CXX", "g++")
    tmp_so = LIBRARY + ".tmp"
    _run([cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra",
          "-D__HIP_PLATFORM_AMD__", "-I", INCLUDE, "-I", CSRC, "-I", os.path.join(ROCM, "include"),
          os.path.join(CSRC, "runtime.cpp"), os.path.join(CSRC, "kv_cache.cpp"), "-o", tmp_so,
          "-L", os.path.join(ROCM, "lib"), "-lamdhip64", "-ldl",
          "-Wl,-rpath," + os.path.join(ROCM, "lib")], verbose)
    os.replace(tmp_so, LIBRARY)
    tmp_exe = LAUNCH_OVERHEAD + ".tmp"
    _run([cxx, "-O2", "-std=c++17", "-Wall", "-Wextra", "-I", INCLUDE,
          os.path.join(CSRC, "launch_overhead.cpp"), "-o", tmp_exe, "-L", HERE, "-lmoearc_attn",
          "-Wl,-rpath,$ORIGIN"], verbose)
    os.replace(tmp_exe, LAUNCH_OVERHEAD)


if __name__ == "__main__":
    build(verbose=True)
