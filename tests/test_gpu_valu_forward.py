"""The vector-ALU forward (attn_fwd_valu_kernel, selected by PET_ATTN_FWD=3,
kept to compare the matrix-core kernel against) checked against the oracle in
a process of its own, since the kernel choice is read once per process."""
from __future__ import annotations

import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

SCRIPT = r"""
import numpy as np, torch, oracle
from pet_kokkos_amd import attention as A, systems
dev = torch.device("cuda", 0)
for cfg in ("c1", "c4"):
    conf, tk = systems.config_tokens(cfg)
    H, hd = conf.heads, conf.head_dim
    qkv = systems.attention_inputs(tk, conf.d_model, H, seed=2)["qkv"]
    merged, ml = A.attn_fwd(torch.from_numpy(qkv).to(dev), torch.from_numpy(tk.off).to(dev),
                            torch.from_numpy(tk.cf_seq).to(dev), H, hd)
    torch.cuda.synchronize()
    rm, rml = oracle.attn_fwd(qkv, tk.off, tk.cf_seq, H, hd)
    em = np.abs(merged.cpu().numpy() - rm).max() / np.abs(rm).max()
    live = rml[:, 1] > 0
    el = np.abs(ml.cpu().numpy()[live] - rml[live]).max() / np.abs(rml[live]).max()
    assert np.array_equal(ml.cpu().numpy()[~live], rml[~live]), cfg
    print(cfg, em, el, flush=True)
    assert em <= 1e-5 and el <= 1e-5, cfg
print("ok")
"""


def test_valu_forward_matches_oracle():
    print("[gpu] vector-ALU forward (PET_ATTN_FWD=3) c1, c4", flush=True)
    env = dict(os.environ, PET_ATTN_FWD="3", PYTHONPATH=ROOT)
    res = subprocess.run([sys.executable, "-c", SCRIPT], env=env, cwd=ROOT, capture_output=True, text=True,
                         timeout=240)
    assert res.returncode == 0 and res.stdout.strip().endswith("ok"), res.stdout + res.stderr
