"""ctypes binding of libpet_attn.so, the C ABI of include/pet_attn.h.

Loading fails loudly when the library is missing: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libpet_attn.so")

EXPORTS = (
    "pet_attn_scale",
    "pet_attn_strerror",
    "pet_attn_max_slots",
    "pet_attn_set_option",
    "pet_attn_get_option",
    "pet_attn_describe",
    "pet_attn_fwd_run",
    "pet_attn_bwd_run",
    "pet_attn_cf_adjoint",
    "pet_attn_zero_dead",
    "pet_attn_fwd",
    "pet_attn_bwd",
    "pet_attn_bwd_noalloc",
    "pet_attn_fwd_xf",
    "pet_attn_bwd_xf",
    "pet_attention",
    "pet_attention_bwd_workspace",
    "pet_attention_bwd",
    "pet_attention_chunked_workspace",
    "pet_attention_chunked",
    "pet_attention_bwd_chunked",
    "pet_attn_cf_seq",
    "pet_norm_rows",
    "pet_norm_rows_bwd",
    "pet_attention_layer_workspace",
    "pet_attention_layer",
    "pet_attention_layer_bwd",
    "pet_edge_grad",
    "pet_fold_edge_gradients",
    "pet_sum_by_structure",
    "pet_edge_geometry",
    "pet_model_create",
    "pet_model_destroy",
    "pet_model_compute",
    "pet_model_workspace_bytes",
    "pet_model_pairs_scratch_bytes",
    "pet_model_last_tier",
    "pet_linear_fused",
    "pet_linear_split_weights",
    "pet_linear_split_weights_transposed",
    "pet_linear_fused_split",
    "pet_linear_fused_split_ws",
    "pet_linear_pair_weights",
    "pet_attn_access_floor",
    "pet_linear_fused_smallk",
    "pet_linear_pair_rows",
    "pet_linear_fused_pairs",
    "pet_linear_fused_split_blocks",
    "pet_linear_fused_blocks",
    "pet_norm_rows_pairs",
    "pet_gemm_flop_tally",
)

OK, EINVAL, EHEADDIM, ESLOTS, EALIGN, ELAUNCH, EBLAS, EWORKSPACE, EINDEX, ESCRATCH = range(10)
NOALLOC_MAX_SCRATCH = 32 << 20  # bytes (PET_ATTN_NOALLOC_MAX_SCRATCH)
MAX_SLOTS = 256


class Shape(ctypes.Structure):
    _fields_ = [
        ("n_atoms", ctypes.c_int),
        ("n_rows", ctypes.c_int),
        ("slots", ctypes.c_int),
        ("heads", ctypes.c_int),
        ("head_dim", ctypes.c_int),
        ("dead", ctypes.c_int),
        ("scale", ctypes.c_float),
    ]


class Plan(ctypes.Structure):
    """pet_attn_plan (include/pet_attn.h)."""
    _fields_ = [(n, ctypes.c_int) for n in ("streaming", "waves", "fwd_split_scores", "fwd_valu", "fwd_lds_bytes",
                                             "fwd_workgroups_per_cu", "bwd_split_dp", "bwd_v_staged",
                                             "bwd_tile_buffers", "bwd_lds_bytes", "bwd_workgroups_per_cu", "bwd_pair", "fwd_pair")]


def describe(n_atoms, n_rows, slots, heads, head_dim) -> dict:
    """pet_attn_describe: what the core kernels run for this shape (no launch)."""
    sh = Shape(n_atoms, n_rows, slots, heads, head_dim, 0, 1.0)
    p = Plan()
    check(load().pet_attn_describe(ctypes.byref(sh), ctypes.byref(p)), "pet_attn_describe")
    return {n: getattr(p, n) for n, _ in Plan._fields_}


class ModelHypers(ctypes.Structure):
    """pet_model_hypers (include/pet_model.h)."""
    _fields_ = [(n, ctypes.c_int) for n in ("d_pet", "d_node", "d_head", "num_heads", "num_gnn_layers",
                                             "num_attention_layers", "n_species", "cutoff_function")] + \
               [(n, ctypes.c_double) for n in ("cutoff_width", "attention_temperature", "energy_scale")] + \
               [("featurizer", ctypes.c_int)]


class ModelTensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("rows", ctypes.c_int), ("cols", ctypes.c_int), ("data", ctypes.c_void_p)]


class ModelEdges(ctypes.Structure):
    """pet_model_edges (include/pet_model.h)."""
    _fields_ = [(n, ctypes.c_int) for n in ("n_atoms", "n_edges", "max_neighbors", "n_struct")] + \
               [(n, ctypes.c_void_p) for n in ("struct_off", "species", "off", "center", "neigh_species", "reverse",
                                               "vec", "dist", "pcut", "cut")]


class PetAttnError(RuntimeError):
    def __init__(self, code: int, what: str):
        self.code = code
        super().__init__(f"{what}: {strerror(code)} (code {code})")


_lib = None
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
# void make_qkv(void* ctx, float* qkv_rows, int64_t ld, int r0, int r1, void* stream)
MAKE_QKV = ctypes.CFUNCTYPE(None, _P, _P, _I64, _I, _I, _P)


def load() -> ctypes.CDLL:
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: build it with `python -m pet_kokkos_amd.build` "
                          "(the attention has no CPU fallback)")
    lib = ctypes.CDLL(LIB_PATH)
    lib.pet_attn_scale.restype = ctypes.c_float
    lib.pet_attn_scale.argtypes = [ctypes.c_int, ctypes.c_double]
    lib.pet_attn_strerror.restype = ctypes.c_char_p
    lib.pet_attn_strerror.argtypes = [ctypes.c_int]
    lib.pet_attn_max_slots.restype = ctypes.c_int
    lib.pet_attn_max_slots.argtypes = [ctypes.c_int]
    lib.pet_attn_set_option.restype = ctypes.c_int
    lib.pet_attn_set_option.argtypes = [ctypes.c_int, ctypes.c_int]
    lib.pet_attn_get_option.restype = ctypes.c_int
    lib.pet_attn_get_option.argtypes = [ctypes.c_int]
    sp = ctypes.POINTER(Shape)
    lib.pet_attn_describe.restype = ctypes.c_int
    lib.pet_attn_describe.argtypes = [sp, ctypes.POINTER(Plan)]
    lib.pet_attn_fwd.restype = ctypes.c_int
    lib.pet_attn_fwd.argtypes = [sp, _P, _I64, _P, _P, _I64, _P, _I64, _P, _P]
    lib.pet_attn_bwd.restype = ctypes.c_int
    lib.pet_attn_bwd.argtypes = [sp, _P, _I64, _P, _P, _I64, _P, _I64, _P, _P, _I64, _P, _I64, _P, _P, _I64, _P]
    lib.pet_attn_bwd_noalloc.restype = ctypes.c_int
    lib.pet_attn_bwd_noalloc.argtypes = [sp, _P, _I64, _P, _P, _I64, _P, _I64, _P, _P, _I64, _P, _I64, _P, _I64, _P]
    lib.pet_attn_fwd_run.restype = ctypes.c_int
    lib.pet_attn_fwd_xf.restype = ctypes.c_int
    lib.pet_attn_fwd_xf.argtypes = [sp, _P, _I64, _P, _P, _P, _P, _I64, _P, _I64, _P, _P]
    lib.pet_attn_bwd_xf.restype = ctypes.c_int
    lib.pet_attn_bwd_xf.argtypes = [sp, _P, _I64, _P, _P, _P, _P, _I64, _P, _I64, _P, _P, _I64, _P, _I64, _P, _P,
                                    _I64, _P]
    lib.pet_attn_fwd_run.argtypes = [sp, _I, _I, _I, _P, _I64, _P, _P, _I64, _P, _I64, _P, _P]
    lib.pet_attn_bwd_run.restype = ctypes.c_int
    lib.pet_attn_bwd_run.argtypes = [sp, _I, _I, _I, _P, _I64, _P, _P, _I64, _P, _I64, _P, _P, _I64, _P, _I64, _P,
                                     _P]
    lib.pet_attn_cf_adjoint.restype = ctypes.c_int
    lib.pet_attn_cf_adjoint.argtypes = [sp, _P, _P, _I64, _P, _I64, _P]
    lib.pet_attn_zero_dead.restype = ctypes.c_int
    lib.pet_attn_zero_dead.argtypes = [sp, _P, _I64, _I, _P, _P]
    lib.pet_attention_chunked_workspace.restype = ctypes.c_size_t
    lib.pet_attention_chunked_workspace.argtypes = [sp, _P, _I]
    lib.pet_attention_chunked.restype = ctypes.c_int
    lib.pet_attention_chunked.argtypes = [sp, _P, _I64, MAKE_QKV, _P, _P, _I64, _P, _P, _P, _P, _P, _P, _I, _P,
                                          ctypes.c_size_t, _P]
    lib.pet_attention_bwd_chunked.restype = ctypes.c_int
    lib.pet_attention_bwd_chunked.argtypes = [sp, _P, _I64, _I, _P, _I64, _P, _I64, MAKE_QKV, _P, _P, _I64, _P, _P,
                                              _P, _P, _P, _P, ctypes.c_float, _I, _P, ctypes.c_size_t, _P]
    lib.pet_attention.restype = ctypes.c_int
    lib.pet_attention.argtypes = [sp, _P, _I64, _P, _I64, _P, _I64, _P, _P, _P, _P, _P, _P]
    lib.pet_attention_bwd_workspace.restype = ctypes.c_size_t
    lib.pet_attention_bwd_workspace.argtypes = [sp]
    lib.pet_attention_bwd.restype = ctypes.c_int
    lib.pet_attention_bwd.argtypes = [sp, _P, _I64, ctypes.c_int, _P, _I64, _P, _I64, _P, _I64, _P, _I64, _P, _P,
                                      _P, _P, _P, ctypes.c_float, _P, ctypes.c_size_t, _P]
    _F = ctypes.c_float
    _D = ctypes.c_double
    lib.pet_attn_cf_seq.restype = ctypes.c_int
    lib.pet_attn_cf_seq.argtypes = [sp, _P, _P, _P, _I64, _P]
    lib.pet_norm_rows.restype = ctypes.c_int
    lib.pet_norm_rows.argtypes = [_I, _I, _P, _I64, _P, _I64, _P, _P, _P]
    lib.pet_norm_rows_bwd.restype = ctypes.c_int
    lib.pet_norm_rows_bwd.argtypes = [_I, _I, _P, _I64, _F, _P, _I64, _P, _I64, _P, _I, _P]
    lib.pet_attention_layer_workspace.restype = ctypes.c_size_t
    lib.pet_attention_layer_workspace.argtypes = [sp]
    lib.pet_attention_layer.restype = ctypes.c_int
    lib.pet_attention_layer.argtypes = [sp, _P, _I64, _P, _I64, _P, _P, _P, _P, _P, _I64, _P, _P, _P, _P, _P, _P,
                                        ctypes.c_size_t, _P]
    lib.pet_attention_layer_bwd.restype = ctypes.c_int
    lib.pet_attention_layer_bwd.argtypes = [sp, _P, _I64, _P, _I64, _P, _I64, _P, _I64, _P, _P, _P, _P, _P, _I64, _P,
                                            _P, _P, _P, _P, ctypes.c_size_t, _P]
    lib.pet_edge_grad.restype = ctypes.c_int
    lib.pet_edge_grad.argtypes = [_I, _I, _P, _P, _P, _I64, _P, _P, _I64, _P, _P, _P, _D, _I, _P, _P]
    lib.pet_fold_edge_gradients.restype = ctypes.c_int
    lib.pet_fold_edge_gradients.argtypes = [_I, _I, _P, _P, _P, _P, _D, _P, _P, _P]
    lib.pet_sum_by_structure.restype = ctypes.c_int
    lib.pet_sum_by_structure.argtypes = [_I, _I, _P, _P, _P, _I, _P]
    lib.pet_edge_geometry.restype = ctypes.c_int
    lib.pet_edge_geometry.argtypes = [_I, _P, _P, _P, _P, _P, _D, _D, _I, _P, _P, _P, _P, _P]
    lib.pet_model_create.restype = ctypes.c_int
    lib.pet_model_create.argtypes = [ctypes.POINTER(ModelHypers), ctypes.POINTER(ModelTensor), _I, _P,
                                     ctypes.POINTER(_P)]
    lib.pet_model_destroy.restype = None
    lib.pet_model_destroy.argtypes = [_P]
    lib.pet_model_compute.restype = ctypes.c_int
    lib.pet_model_compute.argtypes = [_P, ctypes.POINTER(ModelEdges), _I, _P, _P, _P, _P, _P, _P]
    lib.pet_linear_fused.restype = ctypes.c_int
    lib.pet_linear_fused.argtypes = [_I, _I, _I, _P, _I64, _P, _I64, _P, _I64, _P, _P, _P, _I64, _F, _P, _I64, _I, _P]
    lib.pet_linear_split_weights.restype = ctypes.c_int
    lib.pet_linear_split_weights.argtypes = [_P, _I, _I, _I64, _P, _P]
    lib.pet_linear_split_weights_transposed.restype = ctypes.c_int
    lib.pet_linear_split_weights_transposed.argtypes = [_P, _I, _I, _I64, _P, _P]
    lib.pet_linear_fused_split.restype = ctypes.c_int
    lib.pet_linear_fused_split.argtypes = [_I, _I, _I, _P, _I64, _P, _P, _I64, _P, _P, _P, _I64, _F, _P, _I64, _I, _P]
    lib.pet_attn_access_floor.restype = ctypes.c_int
    lib.pet_attn_access_floor.argtypes = [ctypes.POINTER(Shape), _I, _P, _I64, _P, _P, _I64, _P, _I64, _P, _P, _I64,
                                          _P, _P]
    lib.pet_linear_pair_weights.restype = ctypes.c_int
    lib.pet_linear_pair_weights.argtypes = [_P, _I, _I, _I64, _P, _P]
    lib.pet_linear_fused_smallk.restype = ctypes.c_int
    lib.pet_linear_fused_smallk.argtypes = [_I, _I, _I, _P, _I64, _P, _P, _I64, _P, _P, _P, _I64, _F, _P, _I64, _I, _P]
    lib.pet_linear_fused_split_ws.restype = ctypes.c_int
    lib.pet_linear_fused_split_ws.argtypes = [_I, _I, _I, _P, _I64, _P, _P, _I64, _P, _P, _P, _I64, _F, _P, _I64, _I,
                                              _P, ctypes.c_size_t, _P]
    lib.pet_linear_pair_rows.restype = ctypes.c_int
    lib.pet_linear_pair_rows.argtypes = [_P, _I, _I, _I64, _P, _P]
    lib.pet_linear_fused_pairs.restype = ctypes.c_int
    lib.pet_linear_fused_pairs.argtypes = [_I, _I, _I, _P, _P, _P, _I64, _P, _P, _P, _I64, _F, _P, _I64, _I, _P]
    lib.pet_linear_fused_split_blocks.restype = ctypes.c_int
    lib.pet_linear_fused_split_blocks.argtypes = [_I, _I, _I, _P, _I64, _P, _P, _P, _P, _P, _I64, _F, _P, _I64, _I,
                                                  _P, ctypes.c_size_t, ctypes.POINTER(ctypes.c_int), _P]
    lib.pet_norm_rows_pairs.restype = ctypes.c_int
    lib.pet_norm_rows_pairs.argtypes = [_I, _I, _P, _P, _I64, _P, _P, _P]
    lib.pet_gemm_flop_tally.restype = ctypes.c_int
    lib.pet_gemm_flop_tally.argtypes = [ctypes.POINTER(ctypes.c_double), _I]
    lib.pet_linear_fused_blocks.restype = ctypes.c_int
    lib.pet_linear_fused_blocks.argtypes = [_I, _I, _I, _P, _I, _P, _P, _I64, _P, _P, _P, _I64, _F, _P, _I64, _I, _P]
    lib.pet_model_workspace_bytes.restype = ctypes.c_size_t
    lib.pet_model_workspace_bytes.argtypes = [_P]
    lib.pet_model_pairs_scratch_bytes.restype = ctypes.c_size_t
    lib.pet_model_pairs_scratch_bytes.argtypes = [_P]
    lib.pet_model_last_tier.restype = ctypes.c_int
    lib.pet_model_last_tier.argtypes = [_P]
    _lib = lib
    return lib


OPTIONS = {"split": 1, "fwd_kernel": 2, "bwd_vlds": 3, "bwd_nbuf": 4, "model_gemm": 5, "attn_stream": 6, "bwd_kernel": 7,
           "model_recompute": 8, "model_pairs": 9}


def set_option(name: str, value: int) -> None:
    """pet_attn_set_option by name (the keys of OPTIONS)."""
    check(load().pet_attn_set_option(OPTIONS[name], int(value)), f"pet_attn_set_option({name}={value})")


def get_option(name: str) -> int:
    return int(load().pet_attn_get_option(OPTIONS[name]))


class options:
    """Context manager: the named options set for the block, restored after.

        with _lib.options(split=0, bwd_vlds=2): ...
    """

    def __init__(self, **values):
        self.values = values
        self.saved = {}

    def __enter__(self):
        for k, v in self.values.items():
            self.saved[k] = get_option(k)
            set_option(k, v)
        return self

    def __exit__(self, *exc):
        for k, v in self.saved.items():
            set_option(k, v)
        return False


def strerror(code: int) -> str:
    return load().pet_attn_strerror(code).decode()


def check(code: int, what: str) -> None:
    if code != OK:
        raise PetAttnError(code, what)


def gemm_flop_tally(reset: bool = False) -> dict:
    """FLOPs (2 M N K) of the dense products this library's kernels have
    launched in this process, by instruction class (pet_gemm_flop_tally):
    "fp32" the fp32 fused kernel, "split" bf16 parts (six products), "pair"
    fp16 pairs (three), "shortk" the short-K kernel (five fp16 products)."""
    out = (ctypes.c_double * 4)()
    check(load().pet_gemm_flop_tally(out, int(reset)), "pet_gemm_flop_tally")
    return dict(fp32=out[0], split=out[1], pair=out[2], shortk=out[3])
