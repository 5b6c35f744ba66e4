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
SOURCES = ["attention.hip", "attention_pair.hip", "attention_stream.hip", "ops.hip", "rows.hip", "forces.hip", "model.hip", "gemm.hip", "probe.hip"]

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


def _run(cmd, what: str, verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed ({res.returncode}) building {what}")


def build(verbose: bool = False) -> str:
    """Compile every HIP source into LIB (always recompiles; one hipcc per
    source, in parallel, then one link) and return its path."""
    from concurrent.futures import ThreadPoolExecutor
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    cflags = [f for f in HIPCC_FLAGS if f != "-shared"]
    jobs = []
    for s in SOURCES:
        obj = os.path.join(objdir, s.replace(".hip", ".o"))
        jobs.append((obj, [hipcc(), *cflags, "-c", "-I", os.path.join(ROOT, "include"), "-o", obj,
                           os.path.join(CSRC, s)]))
    workers = max(1, min(len(jobs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))
    with ThreadPoolExecutor(workers) as pool:
        for f in [pool.submit(_run, cmd, obj, verbose) for obj, cmd in jobs]:
            f.result()
    tmp = LIB + ".tmp"
    _run([hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *[o for o, _ in jobs],
          "-L/opt/rocm/lib", "-lrocblas", "-Wl,-rpath,/opt/rocm/lib"], LIB, verbose)
    os.replace(tmp, LIB)
    build_cpp_test(verbose)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
