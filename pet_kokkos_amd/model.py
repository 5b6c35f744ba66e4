"""The whole PET evaluation over torch device memory: the Python mirror of the
reference's PetModel / Calculator for the feedforward featurizer
(peterspackman/pet-kokkos include/pet/model.hpp, include/pet/calculator.hpp:
187-239, src/model.cpp:782-811, src/feedforward.cpp:338-411), every step in
libpet_attn.so (include/pet_model.h). There is no CPU path: without the
library, or without a GPU, construction fails.
"""
from __future__ import annotations

import ctypes
import dataclasses

import numpy as np
import torch

from . import _lib
from .attention import _stream
from .forces import CUTOFF_KINDS
from .systems import Edges, Structure, neighbor_list, packed_edges
from .weights import Hypers


@dataclasses.dataclass
class ModelInput:
    """A batch on the device in the layout pet_model_compute reads
    (DeviceEdgeData + PackedEdges, include/pet/model.hpp:60-168)."""
    n_atoms: int
    n_edges: int
    max_neighbors: int
    struct_off: torch.Tensor  # int32 [B + 1]
    species: torch.Tensor  # int32 [N]
    off: torch.Tensor  # int32 [N + 1]
    center: torch.Tensor  # int32 [E]
    neigh_species: torch.Tensor  # int32 [E]
    reverse: torch.Tensor  # int32 [E]
    vec: torch.Tensor  # float64 [E, 3]
    dist: torch.Tensor  # float64 [E]
    pcut: torch.Tensor  # float64 [E]
    cut: torch.Tensor  # float32 [E]
    host: object = None  # the host PackedEdges, for checks

    @property
    def n_struct(self) -> int:
        return int(self.struct_off.numel()) - 1

    def c(self) -> _lib.ModelEdges:
        p = lambda t: t.data_ptr() if t.numel() else None
        return _lib.ModelEdges(self.n_atoms, self.n_edges, self.max_neighbors, self.n_struct, p(self.struct_off),
                               p(self.species), p(self.off), p(self.center), p(self.neigh_species), p(self.reverse),
                               p(self.vec), p(self.dist), p(self.pcut), p(self.cut))


def species_index(numbers, atomic_types) -> np.ndarray:
    lut = {int(z): i for i, z in enumerate(atomic_types)}
    try:
        return np.array([lut[int(z)] for z in numbers], dtype=np.int32)
    except KeyError as e:
        raise ValueError(f"atomic number {e.args[0]} is not among the model's types {tuple(atomic_types)}") from None


def make_input(h: Hypers, species: np.ndarray, edges: Edges, struct_off: np.ndarray, device="cuda:0",
               cut: np.ndarray | None = None) -> ModelInput:
    """Pack a host neighbour list (already grouped by centre) for the device."""
    N = len(species)
    pk = packed_edges(N, edges, h.cutoff, h.cutoff_width)
    if cut is not None:
        pk.cut = np.asarray(cut, dtype=np.float32)
    E = int(pk.off[-1])
    counts = np.diff(pk.off)
    t = lambda a, dt: torch.as_tensor(np.ascontiguousarray(a), dtype=dt).to(device)
    return ModelInput(N, E, int(counts.max()) if N else 0, t(struct_off, torch.int32), t(species, torch.int32),
                      t(pk.off, torch.int32), t(pk.center, torch.int32), t(species[pk.neigh], torch.int32),
                      t(pk.reverse, torch.int32), t(pk.vec, torch.float64), t(pk.dist, torch.float64),
                      t(pk.pcut, torch.float64), t(pk.cut, torch.float32), pk)


def structures_input(h: Hypers, structures: list[Structure], device="cuda:0") -> ModelInput:
    """A batch of structures: each one's neighbour list at the model's cutoff,
    atoms concatenated (energy_forces_batch, src/model.cpp:782-793)."""
    parts, species, soff, base = [], [], [0], 0
    for s in structures:
        e = neighbor_list(s, h.cutoff)
        parts.append(Edges(e.centre + base, e.neigh + base, e.vec, e.dist, e.shift))
        species.append(species_index(s.numbers, h.atomic_types))
        base += len(s.positions)
        soff.append(base)
    cat = lambda f: np.concatenate([getattr(p, f) for p in parts])
    edges = Edges(cat("centre").astype(np.int32), cat("neigh").astype(np.int32), cat("vec"), cat("dist"), cat("shift"))
    return make_input(h, np.concatenate(species), edges, np.array(soff, dtype=np.int32), device)


class PetModel:
    """Weights on the device and energy / forces / virial from packed edges
    (the reference's PetModel, include/pet/model.hpp)."""

    def __init__(self, h: Hypers, weights: dict[str, np.ndarray], composition=None, energy_scale: float = 1.0):
        self.h = h
        lib = _lib.load()
        hy = _lib.ModelHypers(h.d_pet, h.d_node, h.d_head, h.num_heads, h.num_gnn_layers, h.num_attention_layers,
                              h.n_species, CUTOFF_KINDS[h.cutoff_function], h.cutoff_width, h.attention_temperature,
                              energy_scale, 1 if h.residual else 0)
        keep = [np.ascontiguousarray(v, dtype=np.float64) for v in weights.values()]
        arr = (_lib.ModelTensor * len(keep))()
        for i, (name, v) in enumerate(zip(weights.keys(), keep)):
            arr[i] = _lib.ModelTensor(name.encode(), v.shape[0], v.shape[1] if v.ndim == 2 else 0, v.ctypes.data)
        comp = None if composition is None else np.ascontiguousarray(composition, dtype=np.float64)
        handle = ctypes.c_void_p()
        _lib.check(lib.pet_model_create(ctypes.byref(hy), arr, len(keep), None if comp is None else comp.ctypes.data,
                                        ctypes.byref(handle)), "pet_model_create")
        self._handle = handle
        self._lib = lib

    @classmethod
    def from_checkpoint(cls, json_path: str, safetensors_path: str) -> "PetModel":
        """A converted reference checkpoint (pet_kokkos_amd.checkpoint)."""
        from . import checkpoint
        c = checkpoint.load(json_path, safetensors_path)
        return cls(c.hypers, c.weights, c.composition, c.energy_scale)

    def __del__(self):
        if getattr(self, "_handle", None) and self._handle.value:
            self._lib.pet_model_destroy(self._handle)
            self._handle = ctypes.c_void_p()

    @property
    def workspace_bytes(self) -> int:
        return int(self._lib.pet_model_workspace_bytes(self._handle))

    @property
    def last_tier(self) -> str:
        """The memory tier of the last evaluation with forces: "never" or "wide" (option model_recompute)."""
        return {0: "none", 1: "never", 2: "wide"}[int(self._lib.pet_model_last_tier(self._handle))]

    @property
    def pairs_scratch_bytes(self) -> int:
        """Bytes of the model's pairs scratch (0: the large products split A as they stage it)."""
        return int(self._lib.pet_model_pairs_scratch_bytes(self._handle))

    def compute(self, x: ModelInput, forces: bool = True, edge_grad: bool = False, out: dict | None = None) -> dict:
        """energy [B], per_atom [N] and, with forces, forces [N, 3], virial
        [B, 3, 3] (and edge_grad [E, 3]): fp64 device tensors. `out` reuses
        the tensors of an earlier call of the same shapes."""
        dev = x.species.device
        f64 = dict(dtype=torch.float64, device=dev)
        if out is None:
            out = {"energy": torch.empty(x.n_struct, **f64), "per_atom": torch.empty(x.n_atoms, **f64)}
            if forces:
                out["forces"] = torch.empty(x.n_atoms, 3, **f64)
                out["virial"] = torch.empty(x.n_struct, 3, 3, **f64)
            if edge_grad:
                out["edge_grad"] = torch.empty(x.n_edges, 3, **f64)
        p = lambda k: out[k].data_ptr() if k in out and out[k].numel() else None
        e = x.c()
        _lib.check(self._lib.pet_model_compute(self._handle, ctypes.byref(e), int(forces), p("energy"), p("per_atom"),
                                               p("forces") if forces else None, p("virial") if forces else None,
                                               p("edge_grad") if forces else None, _stream()),
                   "pet_model_compute")
        return out


class Calculator:
    """pet::Calculator's evaluation calls (include/pet/calculator.hpp:187-239):
    compute() for a structure (host neighbour list), and for an MD engine that
    keeps its own list, set_neighbors() once per rebuild then compute_step()
    every step with new positions -- the list stays on the device and only
    positions move; pairs that drift past the cutoff weigh nothing --, or
    compute_edges() for both at once. Results on the host.

    With ``graph=True`` compute_step replays the step's device work (edge
    geometry and the whole evaluation) as one HIP graph per (forces,
    edge_gradients) from its second step on a list (``StepRecorder``): the
    positions are copied into a buffer the graph reads, the results are the
    same bits as an eager step, and a small structure's step loses most of its
    launch cost (64 atoms: 1.02 -> 0.77 ms). A new list (set_neighbors) drops
    the recorded graphs."""

    def __init__(self, model: PetModel, device="cuda:0", graph: bool = False):
        self.model, self.device = model, device
        self._x = None
        self._graph = graph
        self._graphs = None

    def compute(self, s: Structure, forces: bool = True):
        e = neighbor_list(s, self.model.h.cutoff)
        off = np.concatenate([[0], np.cumsum(np.bincount(e.centre, minlength=len(s.positions)))])
        return self.compute_edges(s.numbers, off, e.neigh, e.shift, s.positions, s.cell, forces)

    def set_neighbors(self, numbers, offsets, neighbors, shifts=None):
        """An engine's full list: atom i's neighbours neighbors[offsets[i]:offsets[i+1]],
        each with an optional integer lattice shift [E, 3]."""
        h = self.model.h
        offsets = np.asarray(offsets, dtype=np.int64)
        N = len(offsets) - 1
        E = int(offsets[-1])
        neigh = np.asarray(neighbors, dtype=np.int64)[:E]
        center = np.repeat(np.arange(N), np.diff(offsets))
        sh = np.zeros((E, 3), dtype=np.int64) if shifts is None else np.asarray(shifts, dtype=np.int64).reshape(E, 3)
        index = {(int(i), int(j), *map(int, t)): k for k, (i, j, t) in enumerate(zip(center, neigh, sh))}
        rev = np.array([index.get((int(j), int(i), *map(int, -t)), -1) for i, j, t in zip(center, neigh, sh)],
                       dtype=np.int32)
        sp = species_index(numbers, h.atomic_types)
        t = lambda a, dt: torch.as_tensor(np.ascontiguousarray(a), dtype=dt).to(self.device)
        f64 = dict(dtype=torch.float64, device=self.device)
        self._x = ModelInput(N, E, int(np.diff(offsets).max()) if N else 0, t(np.array([0, N]), torch.int32),
                             t(sp, torch.int32), t(offsets, torch.int32), t(center, torch.int32),
                             t(sp[neigh], torch.int32), t(rev, torch.int32), torch.empty(E, 3, **f64),
                             torch.empty(E, **f64), torch.empty(E, **f64),
                             torch.empty(E, dtype=torch.float32, device=self.device))
        self._neigh = t(neigh, torch.int32)
        self._shift = None if shifts is None else t(sh, torch.int32)
        self._out = None
        # the buffers a recorded step reads: positions and cell, refilled each step
        self._pos = torch.empty((N, 3), **f64)
        self._cell = torch.empty((3, 3), **f64)
        if self._graph:
            from .replay import StepRecorder
            self._graphs = StepRecorder(warm_runs=1, max_live=4)

    def compute_step(self, positions, cell=None, forces: bool = True, edge_gradients: bool = False):
        x = self._x
        if x is None:
            raise RuntimeError("compute_step before set_neighbors")
        if self._shift is not None and cell is None:
            raise ValueError("the list has shifts, so compute_step needs the cell")
        h = self.model.h
        self._pos.copy_(torch.as_tensor(np.ascontiguousarray(positions, dtype=np.float64).reshape(-1, 3)))
        if cell is not None:
            self._cell.copy_(torch.as_tensor(np.ascontiguousarray(cell, dtype=np.float64).reshape(3, 3)))
        p = lambda t: None if t is None or t.numel() == 0 else t.data_ptr()

        def step():
            _lib.check(_lib.load().pet_edge_geometry(x.n_edges, p(x.center), p(self._neigh), p(self._shift),
                                                     p(self._pos), p(self._cell) if self._shift is not None else None,
                                                     h.cutoff, h.cutoff_width, CUTOFF_KINDS[h.cutoff_function],
                                                     p(x.vec), p(x.dist), p(x.pcut), p(x.cut), _stream()),
                       "pet_edge_geometry")
            return self.model.compute(x, forces, edge_gradients)

        o = self._graphs.launch((forces, edge_gradients), step) if self._graphs is not None else step()
        torch.cuda.synchronize()
        res = {"energy": float(o["energy"][0]), "per_atom": o["per_atom"].cpu().numpy()}
        if forces:
            res["forces"] = o["forces"].cpu().numpy()
            res["virial"] = o["virial"][0].cpu().numpy()
            if edge_gradients:
                res["edge_gradient"] = o["edge_grad"].cpu().numpy()
        return res

    def compute_edges(self, numbers, offsets, neighbors, shifts, positions, cell=None, forces: bool = True,
                      edge_gradients: bool = False):
        self.set_neighbors(numbers, offsets, neighbors, shifts)
        return self.compute_step(positions, cell, forces, edge_gradients)


def ef_gemms(h: Hypers, n_atoms: int, n_edges: int) -> list:
    """The evaluation's dense products as (M, N, K), one per forward layer
    (the reference's accounting, tools/roofline.py:188-260); an energy+forces
    evaluation runs each once more as its input adjoint (M K N)."""
    N, E, T = n_atoms, n_edges, n_atoms + n_edges
    D, Dn, Dh, cw, ew = h.d_pet, h.d_node, h.d_head, h.center_width, h.edge_width
    g = []
    readout = [(N, Dh, Dn), (N, Dh, Dh), (N, 1, Dh), (E, Dh, D), (E, Dh, Dh), (E, 1, Dh)]
    if h.residual:  # per block QKV, output, the MLP over all tokens; a read-out a layer
        for L in range(h.num_gnn_layers):
            g += ([(E, D, D)] if L else []) + [(E, D, D)]
            g += h.num_attention_layers * [(T, 3 * D, D), (T, D, D), (T, ew, D), (T, D, ew)]
            g += readout
        return g
    for L in range(h.num_gnn_layers):
        g += ([(E, D, D)] if L else []) + [(E, D, D)]  # compress.0's input_edge block, compress.2
        g += h.num_attention_layers * [(N, D, Dn), (T, 3 * D, D), (T, D, D), (N, Dn, D), (N, cw, Dn),
                                       (N, Dn, cw // 2), (E, ew, D), (E, D, ew // 2)]
        g += [(E, 2 * D, 2 * D), (E, D, 2 * D)]  # combination MLP
    return g + readout


# The model's dense products with M N K >= 2^32 run on the split-product kernel
# by default (fp32 accuracy on the 16-bit matrix cores: from K = 256 as fp16
# pairs, three products; below as three bf16 parts, six products); the rest on
# rocBLAS fp32.
SPLIT_THRESHOLD = 2.0 ** 32
PAIR_MIN_K = 256


def ef_flops(h: Hypers, n_atoms: int, n_edges: int, sum_cnt2: float) -> dict:
    """Algorithmic FLOPs of one evaluation: 2 M N K per dense layer forward and
    once more for its input adjoint (M K N: forces need no weight gradients),
    the attention's 4 (forward) and 10 (backward) sum(cnt^2) D per block; and
    the parts of the forces FLOPs in dense products large enough for the
    split-product kernel, as fp16 pairs ("pair", contraction length >= 256)
    or bf16 parts ("split")."""
    gm = ef_gemms(h, n_atoms, n_edges)
    g = float(sum(m * n * k for m, n, k in gm))
    pair = split = 0.0
    for m, n, k in gm:
        if float(m) * n * k < SPLIT_THRESHOLD:
            continue
        for kk in (k, n):  # the forward's contraction, then the adjoint's
            if kk >= PAIR_MIN_K:
                pair += 2.0 * m * n * k
            else:
                split += 2.0 * m * n * k
    blocks = h.num_gnn_layers * h.num_attention_layers
    D = h.d_pet
    return dict(energy=2.0 * g + blocks * 4.0 * sum_cnt2 * D,
                forces=4.0 * g + blocks * 14.0 * sum_cnt2 * D, split=split, pair=pair)


def ef_workload(name: str, seed: int = 0):
    """(hypers, weights, composition, structures) of an energy+forces workload:
    "c2" configs[1] (648-atom water), "c2-residual" the same with the residual
    featurizer, "c5" configs[4] (32 structures, diamond-64 and water-648
    alternating, each seeded by its index)."""
    from . import systems, weights
    h = weights.MODELS[name]
    if name in ("c2", "c2-residual"):
        sts = [systems.water_box(6, 18.6, seed=seed)]
    elif name == "c5":
        sts = [systems.diamond(2, jitter=0.01, seed=seed + k) if k % 2 == 0 else
               systems.water_box(6, 18.6, seed=seed + k) for k in range(32)]
    else:
        raise ValueError(name)
    return h, weights.random_weights(h, seed), weights.random_composition(h, seed), sts
