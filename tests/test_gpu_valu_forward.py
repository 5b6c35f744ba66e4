"""The vector-ALU forward (attn_fwd_valu_kernel, selected by the option
fwd_kernel = 3, kept to compare the matrix-core kernel against) checked
against the oracle element-wise (tests/parity.py's row-floor rule)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from parity import RTOL, row_err
from pet_kokkos_amd import _lib
from pet_kokkos_amd import attention as A
from pet_kokkos_amd import systems

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("cfg", ["c1", "c4"])
def test_valu_forward_matches_oracle(device, cfg):
    print(f"[gpu] vector-ALU forward (fwd_kernel=3) {cfg}", flush=True)
    conf, tk = systems.config_tokens(cfg)
    H, hd = conf.heads, conf.head_dim
    qkv = systems.attention_inputs(tk, conf.d_model, H, seed=2)["qkv"]
    with _lib.options(fwd_kernel=3):
        merged, ml = A.attn_fwd(torch.from_numpy(qkv).to(device), torch.from_numpy(tk.off).to(device),
                                torch.from_numpy(tk.cf_seq).to(device), H, hd)
        torch.cuda.synchronize()
    rm, rml = oracle.attn_fwd(qkv, tk.off, tk.cf_seq, H, hd)
    ml = ml.cpu().numpy()
    live = rml[:, 1] > 0
    assert np.array_equal(ml[~live], rml[~live])
    em = row_err(merged.cpu().numpy(), rm)
    el = row_err(np.where(live[:, None], ml, 0).reshape(-1, 2 * tk.slots),
                 np.where(live[:, None], rml, 0).reshape(-1, 2 * tk.slots))
    print(f"    merged {em:.2e}, ml {el:.2e}", flush=True)
    assert em <= RTOL and el <= RTOL
