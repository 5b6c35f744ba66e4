"""The C-ABI library without a GPU: it loads, exports every function
include/pet_attn.h and include/pet_model.h declare, and rejects bad arguments before touching the
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
HEADERS = [os.path.join(ROOT, "include", h) for h in ("pet_attn.h", "pet_model.h")]


def declared():
    text = "".join(open(h).read() for h in HEADERS)
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
    for hd in (0, 129):  # head_dim outside 1..128 (the reference's kMaxHeadDim)
        sh = _lib.Shape(4, 20, 8, 2, hd, 0, 0.2)
        assert lib.pet_attn_fwd(ctypes.byref(sh), 16, 6 * max(hd, 1), 16, 16, 8, 16, 48, None, None) == _lib.EHEADDIM
    sh = _lib.Shape(4, 20, 8, 2, 24, 0, 0.2)  # head_dim 24 (the streaming kernels): its own checks apply
    assert lib.pet_attn_fwd(ctypes.byref(sh), 16, 100, 16, 16, 8, 16, 48, None, None) == _lib.EINVAL  # ldq < 3D
    sh = _lib.Shape(4, 20, 8, 2, 10, 0, 0.2)  # head_dim 10: 4-byte alignment suffices, 2 bytes does not
    assert lib.pet_attn_fwd(ctypes.byref(sh), 18, 60, 16, 16, 8, 16, 20, None, None) == _lib.EALIGN
    sh = _lib.Shape(4, 20, 8, 2, 32, 0, 0.2)
    assert lib.pet_attn_fwd(ctypes.byref(sh), None, 192, 16, 16, 8, 16, 64, None, None) == _lib.EINVAL
    assert lib.pet_attn_fwd(ctypes.byref(sh), 16, 100, 16, 16, 8, 16, 64, None, None) == _lib.EINVAL  # ldq < 3D
    assert lib.pet_attn_fwd(ctypes.byref(sh), 20, 192, 16, 16, 8, 16, 64, None, None) == _lib.EALIGN
    assert lib.pet_attn_fwd(None, 16, 192, 16, 16, 8, 16, 64, None, None) == _lib.EINVAL
    sh = _lib.Shape(4, 20, 8, 2, 32, 0, 0.2)
    assert lib.pet_attention_bwd_workspace(ctypes.byref(sh)) >= 4 * (20 * 64 + 20 * 192 + 4 * 8 * 2)
    for code in range(9):
        assert _lib.strerror(code)


def test_linear_epilogue_arguments_without_device():
    """The dense layer's argument checks return before any device work: the
    backward epilogues (act 3, 4) need cin, take no row scale or pre, and
    read and write 2N columns for SwiGLU."""
    lib = _lib.load()
    A, Ws, C, z = 4096, 8192, 16384, 32768  # stand-in addresses: nothing is launched on a rejection
    for fn, w in ((lib.pet_linear_fused, (Ws, 32)), (lib.pet_linear_fused_split, (Ws,))):
        def call(ldc, cin, ldcin, act, rs=None, pre=None):
            args = [8, 8, 32, A, 32, *w, C, ldc, rs, None, cin, ldcin, 0.0, pre, 8, act, None]
            return fn(*args)
        assert call(8, None, 0, 3) == _lib.EINVAL  # no pre-activation
        assert call(8, z, 8, 4) == _lib.EINVAL  # SwiGLU's cin and C are 2N = 16 wide
        assert call(16, z, 8, 4) == _lib.EINVAL
        assert call(8, z, 8, 3, rs=z) == _lib.EINVAL  # no row scale
        assert call(8, z, 8, 3, pre=z) == _lib.EINVAL  # no pre
        assert call(8, z, 8, 5) == _lib.EINVAL
        assert call(8, z, 8, -1) == _lib.EINVAL


def test_error_raises():
    with pytest.raises(_lib.PetAttnError):
        _lib.check(_lib.EHEADDIM, "x")
    assert issubclass(_lib.PetAttnError, RuntimeError)
    _ = np


def _model_create(tensors, **over):
    from pet_kokkos_amd import weights
    h = weights.MODELS["tiny"]
    hy = dict(d_pet=h.d_pet, d_node=h.d_node, d_head=h.d_head, num_heads=h.num_heads,
              num_gnn_layers=h.num_gnn_layers, num_attention_layers=h.num_attention_layers, n_species=h.n_species,
              cutoff_function=1, cutoff_width=0.5, attention_temperature=1.0, energy_scale=1.0,
              featurizer=0)
    hy.update(over)
    keep = [np.ascontiguousarray(v, dtype=np.float64) for v in tensors.values()]
    arr = (_lib.ModelTensor * max(1, len(keep)))()
    for i, (name, v) in enumerate(zip(tensors.keys(), keep)):
        arr[i] = _lib.ModelTensor(name.encode(), v.shape[0], v.shape[1] if v.ndim == 2 else 0, v.ctypes.data)
    out = ctypes.c_void_p()
    code = _lib.load().pet_model_create(ctypes.byref(_lib.ModelHypers(**hy)), arr, len(keep), None, ctypes.byref(out))
    return code, out


def test_model_create_rejects_before_the_device():
    """Checks that fail before any device memory is touched (pet_model_create)."""
    from pet_kokkos_amd import weights
    w = weights.random_weights(weights.MODELS["tiny"], 0)
    missing = dict(w)
    del missing["gnn_layers.1.trans.layers.0.mlp.w_out.weight"]
    assert _model_create(missing)[0] == 20  # PET_MODEL_EMISSING
    bad = dict(w)
    bad["gnn_layers.0.compress.2.weight"] = np.zeros((3, 3))
    assert _model_create(bad)[0] == 21  # PET_MODEL_ESHAPE
    assert _model_create(w, d_node=64)[0] == _lib.EINVAL  # the feedforward family needs d_node != d_pet
    assert _model_create(w, featurizer=1)[0] == _lib.EINVAL  # the residual family needs d_node == d_pet
    assert _model_create(w, featurizer=2)[0] == _lib.EINVAL
    assert _model_create(w, num_heads=3)[0] == _lib.EINVAL  # d_pet not a multiple of the heads
    assert _model_create(w, d_pet=258, num_heads=2)[0] == _lib.EHEADDIM  # head_dim 129
    assert "missing" in _lib.strerror(20)
    lib = _lib.load()
    assert lib.pet_model_compute(None, None, 1, None, None, None, None, None, None) == _lib.EINVAL
