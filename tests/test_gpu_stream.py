"""The streaming attention kernels (csrc/attention_stream.hip) against the
oracle, element by element (tests/parity.py's rules, fp32 and fp64 oracles):
every head_dim 1..128 that is not a multiple of 16 (the reference's generic
path, src/attention.cpp:28-39), slot counts past the LDS-staged kernels'
envelope (its flat path takes any S, :195-203), and -- forced by the option
attn_stream -- the benchmark configurations the staged kernels also run."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from pet_kokkos_amd import _lib
from pet_kokkos_amd import systems
from test_gpu_attention import check_against_oracle, random_case, say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("hd", [1, 3, 8, 12, 20, 24, 40, 100, 127])
def test_any_head_dim(device, hd):
    counts = [0, 15, 16, 17, 63, 64, 65, 5, 130]
    tk, qkv, dm = random_case(counts, 3, hd, seed=300 + hd, cf_kind="zeros", extra=3)
    check_against_oracle(device, f"streaming head_dim {hd}", tk.off, tk.cf_seq, qkv, dm, 3, hd, temperature=0.9)


@pytest.mark.parametrize("hd", [128, 64, 32, 40])
def test_slots_past_the_staged_envelope(device, hd):
    lib = _lib.load()
    counts = [299, 3, 150, 0, 64, 200, 257]
    tk, qkv, dm = random_case(counts, 2, hd, seed=400 + hd, cf_kind="random")
    assert tk.slots == 300 and tk.slots > lib.pet_attn_max_slots(hd)
    check_against_oracle(device, f"S {tk.slots} hd {hd}", tk.off, tk.cf_seq, qkv, dm, 2, hd)


@pytest.mark.parametrize("cfg", ["c1", "c4", "c2"])
def test_forced_on_configs(device, cfg):
    conf, tk = systems.config_tokens(cfg)
    rng = np.random.default_rng(3)
    qkv = systems.attention_inputs(tk, conf.d_model, conf.heads, seed=1)["qkv"]
    dm = rng.standard_normal((tk.n_rows, conf.d_model), dtype=np.float32)
    with _lib.options(attn_stream=1):
        check_against_oracle(device, f"streaming {cfg}", tk.off, tk.cf_seq, qkv, dm, conf.heads, conf.head_dim)


def test_forced_edge_cases_and_dead_rows(device):
    with _lib.options(attn_stream=1):
        counts = [0, 0, 1, 14, 15, 16, 17, 31, 32, 33, 63, 0]
        tk, qkv, dm = random_case(counts, 4, 32, seed=5, cf_kind="zeros", extra=5)
        check_against_oracle(device, "streaming edge cases", tk.off, tk.cf_seq, qkv, dm, 4, 32)
        tk, qkv, dm = random_case([10, 22, 5], 2, 24, seed=8)
        rng = np.random.default_rng(1)
        qkv = np.concatenate([qkv, rng.standard_normal((9, qkv.shape[1])).astype(np.float32)])
        dm = np.concatenate([dm, rng.standard_normal((9, dm.shape[1])).astype(np.float32)])
        m, _, qa, _, _ = check_against_oracle(device, "streaming dead rows", tk.off, tk.cf_seq, qkv, dm, 2, 24,
                                              dead=True)
        assert np.all(m[tk.n_rows:] == 0) and np.all(qa[tk.n_rows:] == 0)


def test_streaming_bit_identical_repeats(device):
    from test_gpu_attention import gpu_fwd_bwd
    tk, qkv, dm = random_case([299, 40, 7], 2, 24, seed=9)
    say("[gpu] streaming bitwise repeats")
    first = gpu_fwd_bwd(device, tk.off, tk.cf_seq, qkv, dm, 2, 24)
    for _ in range(2):
        again = gpu_fwd_bwd(device, tk.off, tk.cf_seq, qkv, dm, 2, 24)
        for a, b in zip(first, again):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
