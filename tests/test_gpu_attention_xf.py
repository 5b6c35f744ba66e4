"""pet_attn_fwd_xf / pet_attn_bwd_xf (qkv given raw, scaled by row and
biased by column as the attention loads it) against pet_attn_fwd /
pet_attn_bwd on the transformed qkv, computed beforehand: the same attention
within fp32 rounding of the transform (1e-5 of each output's largest
magnitude), for the row scale alone, the bias alone and both."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from pet_kokkos_amd import _lib
from pet_kokkos_amd import attention as A
from pet_kokkos_amd import systems

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("mode", ["scale", "bias", "both"])
@pytest.mark.parametrize("cfg", ["c1", "c2"])
def test_xf_matches_pretransformed(cfg, mode, device):
    conf, tk = systems.config_tokens(cfg)
    H, hd, D = conf.heads, conf.head_dim, conf.d_model
    N, S, T = tk.n_atoms, tk.slots, tk.n_rows
    g = torch.Generator(device=device).manual_seed(3)
    raw = torch.randn(T, 3 * D, device=device, generator=g)
    rs = torch.rand(T, device=device, generator=g) + 0.5 if mode != "bias" else None
    b = torch.randn(3 * D, device=device, generator=g) if mode != "scale" else None
    qkv = raw * (rs[:, None] if rs is not None else 1.0) + (b if b is not None else 0.0)
    off = torch.from_numpy(tk.off).to(device)
    cf = torch.from_numpy(tk.cf_seq).to(device)
    dm = torch.randn(T, D, device=device, generator=g)
    m0, ml0 = A.attn_fwd(qkv, off, cf, H, hd)
    qa0, ca0, _ = A.attn_bwd(qkv, off, dm, m0, ml0, cf, H, hd)
    lib = _lib.load()
    shp = _lib.Shape(N, T, S, H, hd, 0, lib.pet_attn_scale(hd, 1.0))
    p = lambda t: None if t is None else t.data_ptr()
    st = torch.cuda.current_stream().cuda_stream
    m1 = torch.empty(T, D, device=device)
    ml1 = torch.empty(N * H * S, 2, device=device)
    _lib.check(lib.pet_attn_fwd_xf(ctypes.byref(shp), p(raw), 3 * D, p(rs), p(b), p(off), p(cf), S, p(m1), D, p(ml1),
                                   st), "pet_attn_fwd_xf")
    qa1 = torch.empty(T, 3 * D, device=device)
    cfh = torch.empty(N, H, S, device=device)
    ca1 = torch.zeros(N, S, device=device)
    _lib.check(lib.pet_attn_bwd_xf(ctypes.byref(shp), p(raw), 3 * D, p(rs), p(b), p(off), p(dm), D, p(m1), D, p(ml1),
                                   p(cf), S, p(qa1), 3 * D, p(cfh), p(ca1), S, st), "pet_attn_bwd_xf")
    torch.cuda.synchronize()
    rel = lambda a, r: float((a.double() - r.double()).abs().max() / r.double().abs().max())
    assert rel(m1, m0) <= 1e-5
    assert rel(qa1, qa0) <= 1e-5
    assert rel(ca1, ca0) <= 1e-5
    live = ml0[:, 1] > 0
    assert torch.equal(live, ml1[:, 1] > 0)
