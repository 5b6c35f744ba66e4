"""pet_attn_bwd_noalloc (the backward with its cfh scratch in a fixed device
array) against pet_attn_bwd (a caller-owned cfh), through the C ABI, on two
calls in a row -- the C1 workload, then a smaller ragged one on the same
array -- bit for bit; and its size limit."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from pet_kokkos_amd import _lib
from pet_kokkos_amd import systems

pytestmark = pytest.mark.gpu


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _case(device, tk, H, hd, seed):
    rng = np.random.default_rng(seed)
    D = H * hd
    t = lambda a, dt=torch.float32: torch.as_tensor(np.ascontiguousarray(a), dtype=dt).to(device)
    qkv = t(rng.standard_normal((tk.n_rows, 3 * D)).astype(np.float32))
    dm = t(rng.standard_normal((tk.n_rows, D)).astype(np.float32))
    return dict(qkv=qkv, dm=dm, off=t(tk.off, torch.int32), cf=t(tk.cf_seq),
                ca0=t(rng.standard_normal((tk.n_atoms, tk.slots)).astype(np.float32)))


def _run(device, tk, H, hd, c):
    lib = _lib.load()
    N, T, S, D = tk.n_atoms, tk.n_rows, tk.slots, H * hd
    sh = _lib.Shape(N, T, S, H, hd, 0, lib.pet_attn_scale(hd, 1.0))
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    merged = torch.empty((T, D), device=device)
    ml = torch.empty((N * H * S, 2), device=device)
    _lib.check(lib.pet_attn_fwd(ctypes.byref(sh), _p(c["qkv"]), 3 * D, _p(c["off"]), _p(c["cf"]), S, _p(merged), D,
                                _p(ml), st), "pet_attn_fwd")
    out = {}
    for name in ("bwd", "noalloc"):
        qa = torch.full((T, 3 * D), 7.0, device=device)
        ca = c["ca0"].clone()
        if name == "bwd":
            cfh = torch.empty((N, H, S), device=device)
            code = lib.pet_attn_bwd(ctypes.byref(sh), _p(c["qkv"]), 3 * D, _p(c["off"]), _p(c["dm"]), D, _p(merged), D,
                                    _p(ml), _p(c["cf"]), S, _p(qa), 3 * D, _p(cfh), _p(ca), S, st)
        else:
            code = lib.pet_attn_bwd_noalloc(ctypes.byref(sh), _p(c["qkv"]), 3 * D, _p(c["off"]), _p(c["dm"]), D,
                                            _p(merged), D, _p(ml), _p(c["cf"]), S, _p(qa), 3 * D, _p(ca), S, st)
        _lib.check(code, name)
        torch.cuda.synchronize()
        out[name] = (qa.cpu().numpy(), ca.cpu().numpy())
    return out


def test_noalloc_matches_bwd_twice(device):
    conf, tk = systems.config_tokens("c1")
    print("[gpu] pet_attn_bwd_noalloc: c1, then a smaller ragged case", flush=True)
    first = _run(device, tk, conf.heads, conf.head_dim, _case(device, tk, conf.heads, conf.head_dim, 1))
    small = systems.tokens_from_counts([5, 0, 17, 40, 3], seed=2, cf_kind="zeros")
    second = _run(device, small, 2, 32, _case(device, small, 2, 32, 3))
    for out in (first, second):
        for a, b in zip(out["bwd"], out["noalloc"]):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_noalloc_size_limit(device):
    lib = _lib.load()
    cap = _lib.NOALLOC_MAX_SCRATCH // 4
    N, H = 40000, 8
    S = cap // (N * H) + 1  # one slot past the array
    sh = _lib.Shape(N, N, S, H, 32, 0, 0.1)
    dummy = torch.zeros(16, device=device)
    p = _p(dummy)
    code = lib.pet_attn_bwd_noalloc(ctypes.byref(sh), p, 3 * 256, p, p, 256, p, 256, p, p, S, p, 3 * 256, p, S, None)
    assert code == _lib.ESCRATCH
    assert "scratch" in _lib.strerror(code)


def test_noalloc_under_graph_capture(device):
    """After one warm call (the device's first: symbol lookup, LDS limit), the
    next call is captured into a HIP graph; three replays, each after the
    inputs it accumulates onto are reset eagerly, give the eager bits."""
    conf, tk = systems.config_tokens("c1")
    H, hd = conf.heads, conf.head_dim
    print("[gpu] pet_attn_bwd_noalloc under graph capture: c1", flush=True)
    c = _case(device, tk, H, hd, 5)
    lib = _lib.load()
    N, T, S, D = tk.n_atoms, tk.n_rows, tk.slots, H * hd
    sh = _lib.Shape(N, T, S, H, hd, 0, lib.pet_attn_scale(hd, 1.0))
    merged = torch.empty((T, D), device=device)
    ml = torch.empty((N * H * S, 2), device=device)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(lib.pet_attn_fwd(ctypes.byref(sh), _p(c["qkv"]), 3 * D, _p(c["off"]), _p(c["cf"]), S, _p(merged), D,
                                _p(ml), st), "pet_attn_fwd")
    qa = torch.empty((T, 3 * D), device=device)
    ca = c["ca0"].clone()

    def call(stream):
        return lib.pet_attn_bwd_noalloc(ctypes.byref(sh), _p(c["qkv"]), 3 * D, _p(c["off"]), _p(c["dm"]), D,
                                        _p(merged), D, _p(ml), _p(c["cf"]), S, _p(qa), 3 * D, _p(ca), S, stream)

    _lib.check(call(st), "warm call")
    torch.cuda.synchronize()
    want = (qa.cpu().numpy().copy(), ca.cpu().numpy().copy())
    g = torch.cuda.CUDAGraph()
    ca.copy_(c["ca0"])
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        code = call(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    _lib.check(code, "captured call")
    for _ in range(3):
        qa.fill_(7.0)
        ca.copy_(c["ca0"])
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(qa.cpu().numpy().view(np.uint32), want[0].view(np.uint32))
        assert np.array_equal(ca.cpu().numpy().view(np.uint32), want[1].view(np.uint32))
