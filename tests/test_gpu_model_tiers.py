"""The whole evaluation's memory tiers (option model_recompute): "wide" keeps
neither the attention's qkv nor the edge MLP's pre-activation and remakes them
in the backward, running the edge MLP over chunks of edge rows (the
reference's Recompute::Wide, src/model.cpp:819-860, src/feedforward.cpp:110-118
and :307-317). Its results are the "never" tier's bit for bit: the remade
products are the forward's own calls, and a chunk's products (at least 64k
rows) run on the split-product kernel, whose rows do not depend on how many
there are -- on C2's water-648 (one chunk) and on a four-structure slice of
C5's batch (about 100k edges: two chunks). Its workspace is smaller."""
from __future__ import annotations

import pytest
import torch

from pet_kokkos_amd import _lib
from pet_kokkos_amd.model import PetModel, ef_workload, structures_input

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name,take", [("c2", None), ("c5", [1, 3, 5, 0])], ids=["c2", "c5-slice"])
def test_wide_tier_same_bits(name, take, device):
    h, w, comp, sts = ef_workload(name)
    if take:
        sts = [sts[k] for k in take]
    print(f"[gpu] memory tiers: {name}, {len(sts)} structures", flush=True)
    x = structures_input(h, sts, device)
    out, ws = {}, {}
    for tier in ("never", "wide"):
        m = PetModel(h, w, comp)
        with _lib.options(model_recompute=1 if tier == "never" else 2):
            got = m.compute(x, forces=True, edge_grad=True)
            torch.cuda.synchronize()
        assert m.last_tier == tier
        out[tier] = {k: v.clone() for k, v in got.items()}
        ws[tier] = m.workspace_bytes
        del m, got
        torch.cuda.empty_cache()
    print(f"    workspace: never {ws['never'] / 2**30:.2f} GiB, wide {ws['wide'] / 2**30:.2f} GiB, edges {x.n_edges}",
          flush=True)
    for k in out["never"]:
        assert torch.equal(out["never"][k], out["wide"][k]), k
    assert ws["wide"] < ws["never"]


def test_auto_tier_is_never_when_it_fits(device):
    h, w, comp, sts = ef_workload("c2")
    m = PetModel(h, w, comp)
    m.compute(structures_input(h, sts, device), forces=True)
    torch.cuda.synchronize()
    assert m.last_tier == "never"
