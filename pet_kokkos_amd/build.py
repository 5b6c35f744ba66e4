"""Builds the gfx950 HIP library in-tree: pet_kokkos_amd/libpet_attn.so.

    python -m pet_kokkos_amd.build

hipcc cross-compiles for gfx950 without a GPU. Packed-FP32 instruction
selection is switched off for the device code (``-packed-fp32-ops``); the host
pass warns that it does not know that feature, which is harmless.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libpet_attn.so")
SOURCES = ["attention.hip", "ops.hip", "rows.hip", "forces.hip", "model.hip", "gemm.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-result",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP library cannot be built")


CPP_TEST_SRC = os.path.join(ROOT, "tests", "cpp", "attention_api_test.cpp")
CPP_TEST = os.path.join(ROOT, "tests", "cpp", "attention_api_test")
CPP_TEST2_SRC = os.path.join(ROOT, "tests", "cpp", "layer_forces_test.cpp")
CPP_TEST2 = os.path.join(ROOT, "tests", "cpp", "layer_forces_test")
CPP_TEST3_SRC = os.path.join(ROOT, "tests", "cpp", "model_test.cpp")
CPP_TEST3 = os.path.join(ROOT, "tests", "cpp", "model_test")


def build_cpp_test(verbose: bool = False) -> str:
    """The C++ callers of include/pet/attention.hpp, include/pet/forces.hpp and
    include/pet/model.hpp that tests/test_gpu_cpp_api.py runs."""
    for src, exe in ((CPP_TEST_SRC, CPP_TEST), (CPP_TEST2_SRC, CPP_TEST2), (CPP_TEST3_SRC, CPP_TEST3)):
        cmd = [hipcc(), "--offload-arch=gfx950", "-O2", "-std=c++17", "-I", os.path.join(ROOT, "include"),
               "-o", exe, src, "-L", HERE, "-lpet_attn", "-Wl,-rpath,$ORIGIN/../../pet_kokkos_amd"]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            sys.stderr.write(res.stdout + res.stderr)
            raise RuntimeError(f"hipcc failed ({res.returncode}) building {exe}")
    return CPP_TEST


def build(verbose: bool = False) -> str:
    """Compile every HIP source into LIB (always recompiles) and return its path."""
    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    tmp = LIB + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, "-I", os.path.join(ROOT, "include"), "-o", tmp, *srcs,
           "-L/opt/rocm/lib", "-lrocblas", "-Wl,-rpath,/opt/rocm/lib"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed ({res.returncode}) building {LIB}")
    os.replace(tmp, LIB)
    build_cpp_test(verbose)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
