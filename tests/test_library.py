"""The C-ABI library without a GPU: it loads, exports every function
include/pet_attn.h declares, and rejects bad arguments before touching the
device."""
from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest

import oracle
from pet_kokkos_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "pet_attn.h")


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"PET_ATTN_API\s+[\w\s\*]+?\b(pet_\w+)\s*\(", text)))


def test_header_declares_the_abi():
    assert declared() == sorted(_lib.EXPORTS)


def test_library_loads_and_exports_every_symbol():
    lib = _lib.load()
    for name in declared():
        assert hasattr(lib, name), name
    nm = os.popen(f"nm -D --defined-only {_lib.LIB_PATH}").read()
    for name in declared():
        assert re.search(rf"\bT {name}\b", nm), name


def test_scale_matches_reference_rounding():
    lib = _lib.load()
    for hd in (16, 32, 48, 64, 80, 128):
        for t in (1.0, 0.7, 2.5):
            assert lib.pet_attn_scale(hd, t) == oracle.scale(hd, t)


def test_error_codes_without_device():
    lib = _lib.load()
    sh = _lib.Shape(4, 20, 8, 2, 24, 0, 0.2)  # head_dim 24: not held
    assert lib.pet_attn_fwd(ctypes.byref(sh), 16, 96, 16, 16, 8, 16, 48, None, None) == _lib.EHEADDIM
    sh = _lib.Shape(4, 20, 300, 2, 32, 0, 0.2)  # too many slots
    assert lib.pet_attn_fwd(ctypes.byref(sh), 16, 192, 16, 16, 300, 16, 64, None, None) == _lib.ESLOTS
    sh = _lib.Shape(4, 20, 8, 2, 32, 0, 0.2)
    assert lib.pet_attn_fwd(ctypes.byref(sh), None, 192, 16, 16, 8, 16, 64, None, None) == _lib.EINVAL
    assert lib.pet_attn_fwd(ctypes.byref(sh), 16, 100, 16, 16, 8, 16, 64, None, None) == _lib.EINVAL  # ldq < 3D
    assert lib.pet_attn_fwd(ctypes.byref(sh), 20, 192, 16, 16, 8, 16, 64, None, None) == _lib.EALIGN
    assert lib.pet_attn_fwd(None, 16, 192, 16, 16, 8, 16, 64, None, None) == _lib.EINVAL
    sh = _lib.Shape(4, 20, 8, 2, 32, 0, 0.2)
    assert lib.pet_attention_bwd_workspace(ctypes.byref(sh)) >= 4 * (20 * 64 + 20 * 192 + 4 * 8 * 2)
    for code in range(9):
        assert _lib.strerror(code)


def test_error_raises():
    with pytest.raises(_lib.PetAttnError):
        _lib.check(_lib.EHEADDIM, "x")
    assert issubclass(_lib.PetAttnError, RuntimeError)
    _ = np
