"""The reference's attention interface over torch device tensors.

``attention`` and ``attention_bwd`` mirror pet::attention / pet::attention_bwd
(reference src/ops.hpp:121-148, src/attention.cpp:2189-2206): same arguments,
same meaning, same conventions -- row-major fp32 views with their own leading
dimension, ``out`` overwritten, ``in_adj`` computed onto ``beta * in_adj``,
``cf_seq_adj`` accumulated, the forward's saves kept in a Workspace under
``key + ":merged"`` and ``key + ":ml"`` for the backward to find. Errors raise
(PetAttnError, a RuntimeError, as the reference's std::runtime_error).

``attention_chunked`` / ``attention_bwd_chunked`` mirror the reference's
chunked forms (src/ops.hpp:133-146): runs of atoms of about ``chunk`` tokens,
qkv made per run by a ``make_qkv(qkv_rows, r0, r1)`` callable.

``attn_fwd`` / ``attn_bwd`` expose the core kernels alone (no linears),
``attn_fwd_run`` / ``attn_bwd_run`` their per-run forms. All
work runs in libpet_attn.so on the current torch stream; torch only provides
device memory and the stream.
"""
from __future__ import annotations

import dataclasses

import torch

from . import _lib


@dataclasses.dataclass
class Tokens:
    """CSR token layout (reference src/ops.hpp:31-37): atom n's tokens are row
    n and rows N + off[n] .. N + off[n+1] - 1; ``dead`` when rows past
    N + off[N] exist (an edge capacity)."""
    off: torch.Tensor  # int32 [N+1], device
    N: int
    dead: bool = False


class Workspace:
    """Named device buffers that outlive a call (the reference's Workspace
    n2/peek2, include/pet/kokkos.hpp:65-235): the forward's saves and the
    backward's scratch."""

    def __init__(self, device=None):
        self.device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self._named: dict[str, torch.Tensor] = {}

    def n2(self, key: str, rows: int, cols: int) -> torch.Tensor:
        t = self._named.get(key)
        if t is None or t.shape != (rows, cols):
            t = torch.empty((rows, cols), dtype=torch.float32, device=self.device)
            self._named[key] = t
        return t

    def bytes(self, key: str, nbytes: int) -> torch.Tensor:
        t = self._named.get(key)
        if t is None or t.numel() < nbytes:
            t = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=self.device)
            self._named[key] = t
        return t

    def peek2(self, key: str) -> torch.Tensor:
        if key not in self._named:
            raise RuntimeError(f"pet: workspace has no buffer named '{key}' (was the forward run with save=True?)")
        return self._named[key]


def _mat(t: torch.Tensor, name: str, width: int | None = None) -> int:
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a device tensor")
    if t.dtype != torch.float32:
        raise ValueError(f"{name} must be float32")
    if t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"{name} must be a row-major 2-D view")
    if width is not None and t.shape[1] != width:
        raise ValueError(f"{name} has {t.shape[1]} columns, expected {width}")
    return t.stride(0)


def _ptr(t):
    return None if t is None else t.data_ptr()


def _weight(t: torch.Tensor, name: str) -> int:
    # The kernels run after this returns: a temporary contiguous copy would be
    # freed under them, so the weight itself must be contiguous.
    if t.device.type != "cuda" or t.dtype != torch.float32 or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous float32 device tensor")
    return t.data_ptr()


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def shape(N: int, T: int, S: int, heads: int, head_dim: int, temperature: float = 1.0,
          dead: bool = False) -> _lib.Shape:
    lib = _lib.load()
    return _lib.Shape(N, T, S, heads, head_dim, int(dead), lib.pet_attn_scale(head_dim, temperature))


def attn_fwd(qkv: torch.Tensor, off: torch.Tensor, cf_seq: torch.Tensor, heads: int, head_dim: int,
             temperature: float = 1.0, N: int | None = None, dead: bool = False, merged: torch.Tensor | None = None,
             ml: torch.Tensor | None = None, save: bool = True):
    """The core forward: (merged [T, D], ml [N*H*S, 2] or None)."""
    lib = _lib.load()
    D = heads * head_dim
    T = qkv.shape[0]
    N = off.shape[0] - 1 if N is None else N
    S = cf_seq.shape[1]
    if merged is None:
        merged = torch.empty((T, D), dtype=torch.float32, device=qkv.device)
    if ml is None and save:
        ml = torch.empty((N * heads * S, 2), dtype=torch.float32, device=qkv.device)
    sh = shape(N, T, S, heads, head_dim, temperature, dead)
    _lib.check(lib.pet_attn_fwd(sh, qkv.data_ptr(), _mat(qkv, "qkv", 3 * D), off.data_ptr(), cf_seq.data_ptr(),
                                _mat(cf_seq, "cf_seq"), merged.data_ptr(), _mat(merged, "merged", D), _ptr(ml),
                                _stream()), "pet_attn_fwd")
    return merged, ml


def attn_bwd(qkv: torch.Tensor, off: torch.Tensor, dmerged: torch.Tensor, merged: torch.Tensor, ml: torch.Tensor,
             cf_seq: torch.Tensor, heads: int, head_dim: int, temperature: float = 1.0,
             cf_seq_adj: torch.Tensor | None = None, N: int | None = None, dead: bool = False,
             qkv_adj: torch.Tensor | None = None, cfh: torch.Tensor | None = None):
    """The core backward: (qkv_adj [T, 3D], cf_seq_adj [N, S] accumulated onto,
    cfh [N, H, S], each key slot's sum over queries of dS per head)."""
    lib = _lib.load()
    D = heads * head_dim
    T = qkv.shape[0]
    N = off.shape[0] - 1 if N is None else N
    S = cf_seq.shape[1]
    if qkv_adj is None:
        qkv_adj = torch.empty((T, 3 * D), dtype=torch.float32, device=qkv.device)
    if cfh is None:
        cfh = torch.empty((N, heads, S), dtype=torch.float32, device=qkv.device)
    if cf_seq_adj is None:
        cf_seq_adj = torch.zeros((N, S), dtype=torch.float32, device=qkv.device)
    sh = shape(N, T, S, heads, head_dim, temperature, dead)
    _lib.check(lib.pet_attn_bwd(sh, qkv.data_ptr(), _mat(qkv, "qkv", 3 * D), off.data_ptr(), dmerged.data_ptr(),
                                _mat(dmerged, "dmerged", D), merged.data_ptr(), _mat(merged, "merged", D),
                                ml.data_ptr(), cf_seq.data_ptr(), _mat(cf_seq, "cf_seq"), qkv_adj.data_ptr(),
                                _mat(qkv_adj, "qkv_adj", 3 * D), cfh.data_ptr(), cf_seq_adj.data_ptr(),
                                _mat(cf_seq_adj, "cf_seq_adj"), _stream()), "pet_attn_bwd")
    return qkv_adj, cf_seq_adj, cfh


def attention(ws: Workspace, key: str, out: torch.Tensor, qkv: torch.Tensor, cf_seq: torch.Tensor,
              w_out: torch.Tensor, b_out: torch.Tensor | None, tk: Tokens, S: int, heads: int, head_dim: int,
              temperature: float, save: bool) -> None:
    """pet::attention: multi-head attention over each atom's tokens with log cf
    as a per-key bias, then out = merged W_out^T + b_out. With ``save`` the
    backward's inputs stay in ``ws`` under ``key``."""
    lib = _lib.load()
    D = heads * head_dim
    T = qkv.shape[0]
    if cf_seq.shape[1] < S:
        raise ValueError("cf_seq narrower than S")
    merged = ws.n2(key + ":merged", T, D) if save else torch.empty((T, D), dtype=torch.float32, device=qkv.device)
    ml = ws.n2(key + ":ml", tk.N * heads * S, 2) if save else None
    sh = shape(tk.N, T, S, heads, head_dim, temperature, tk.dead)
    _lib.check(lib.pet_attention(sh, out.data_ptr(), _mat(out, "out", D), qkv.data_ptr(), _mat(qkv, "qkv", 3 * D),
                                 cf_seq.data_ptr(), _mat(cf_seq, "cf_seq"), _weight(w_out, "w_out"),
                                 None if b_out is None else _weight(b_out, "b_out"), tk.off.data_ptr(), merged.data_ptr(), _ptr(ml), _stream()),
               "pet_attention")


def attention_bwd(ws: Workspace, key: str, in_adj: torch.Tensor, cf_seq_adj: torch.Tensor, out_adj: torch.Tensor,
                  qkv: torch.Tensor, cf_seq: torch.Tensor, w_in: torch.Tensor, w_out: torch.Tensor, tk: Tokens,
                  S: int, heads: int, head_dim: int, temperature: float, beta: float) -> None:
    """pet::attention_bwd: in_adj (onto beta * in_adj) is the adjoint of the
    input linear's input; cf_seq_adj accumulates; ``key`` names the forward's
    saves."""
    lib = _lib.load()
    D = heads * head_dim
    T = qkv.shape[0]
    merged, ml = ws.peek2(key + ":merged"), ws.peek2(key + ":ml")
    sh = shape(tk.N, T, S, heads, head_dim, temperature, tk.dead)
    nbytes = lib.pet_attention_bwd_workspace(sh)
    scratch = ws.bytes("attention_bwd:scratch", nbytes)
    d_in = w_in.shape[1]
    _lib.check(lib.pet_attention_bwd(sh, in_adj.data_ptr(), _mat(in_adj, "in_adj", d_in), d_in,
                                     cf_seq_adj.data_ptr(), _mat(cf_seq_adj, "cf_seq_adj"), out_adj.data_ptr(),
                                     _mat(out_adj, "out_adj", D), qkv.data_ptr(), _mat(qkv, "qkv", 3 * D),
                                     cf_seq.data_ptr(), _mat(cf_seq, "cf_seq"), _weight(w_in, "w_in"),
                                     _weight(w_out, "w_out"), tk.off.data_ptr(), merged.data_ptr(),
                                     ml.data_ptr(), float(beta), scratch.data_ptr(), scratch.numel(), _stream()),
               "pet_attention_bwd")


def attn_fwd_run(n0: int, n1: int, e0: int, qkv_chunk: torch.Tensor, off: torch.Tensor, cf_seq: torch.Tensor,
                 merged: torch.Tensor, ml: torch.Tensor | None, heads: int, head_dim: int, T: int,
                 temperature: float = 1.0) -> None:
    """The core forward of atoms [n0, n1) from their chunk of qkv rows (own
    rows, then edges' rows from edge e0); merged [T, D] and ml at the whole's
    rows and slots."""
    lib = _lib.load()
    D = heads * head_dim
    N = off.shape[0] - 1
    sh = shape(N, T, cf_seq.shape[1], heads, head_dim, temperature)
    _lib.check(lib.pet_attn_fwd_run(sh, n0, n1, e0, qkv_chunk.data_ptr(), _mat(qkv_chunk, "qkv_chunk", 3 * D),
                                    off.data_ptr(), cf_seq.data_ptr(), _mat(cf_seq, "cf_seq"), merged.data_ptr(),
                                    _mat(merged, "merged", D), _ptr(ml), _stream()), "pet_attn_fwd_run")


def attn_bwd_run(n0: int, n1: int, e0: int, qkv_chunk: torch.Tensor, off: torch.Tensor, dmerged_chunk: torch.Tensor,
                 merged: torch.Tensor, ml: torch.Tensor, cf_seq: torch.Tensor, qkv_adj_chunk: torch.Tensor,
                 cfh: torch.Tensor, heads: int, head_dim: int, T: int, temperature: float = 1.0) -> None:
    """The core backward of atoms [n0, n1) in their chunk rows; cfh [N, H, S]
    at the whole's slots (no cf adjoint, no dead rows)."""
    lib = _lib.load()
    D = heads * head_dim
    N = off.shape[0] - 1
    sh = shape(N, T, cf_seq.shape[1], heads, head_dim, temperature)
    _lib.check(lib.pet_attn_bwd_run(sh, n0, n1, e0, qkv_chunk.data_ptr(), _mat(qkv_chunk, "qkv_chunk", 3 * D),
                                    off.data_ptr(), dmerged_chunk.data_ptr(),
                                    _mat(dmerged_chunk, "dmerged_chunk", D), merged.data_ptr(),
                                    _mat(merged, "merged", D), ml.data_ptr(), cf_seq.data_ptr(),
                                    _mat(cf_seq, "cf_seq"), qkv_adj_chunk.data_ptr(),
                                    _mat(qkv_adj_chunk, "qkv_adj_chunk", 3 * D), cfh.data_ptr(), _stream()),
               "pet_attn_bwd_run")


def atom_runs(off_host, chunk: int):
    """Runs [n0, n1) of consecutive atoms of at most about ``chunk`` tokens (at
    least one atom), with their first and end edges: the reference's atom_runs
    (src/attention.cpp:2060-2070)."""
    N = len(off_host) - 1
    runs, n0 = [], 0
    while n0 < N:
        n1 = n0 + 1
        while n1 < N and (n1 + 1 - n0) + (int(off_host[n1 + 1]) - int(off_host[n0])) <= chunk:
            n1 += 1
        runs.append((n0, n1, int(off_host[n0]), int(off_host[n1])))
        n0 = n1
    return runs


class _RunRows:
    """The make_qkv callback the library calls: the pointer it passes is inside
    the workspace tensor, so the Python callable gets a torch view of it."""

    def __init__(self, make_qkv, ws: torch.Tensor, width: int):
        self.make_qkv = make_qkv
        self.ws = ws.view(torch.float32) if ws.dtype == torch.uint8 else ws
        self.base = ws.data_ptr()
        self.width = width
        self.error = None
        self.cfunc = _lib.MAKE_QKV(self)

    def __call__(self, ctx, ptr, ld, r0, r1, stream):
        try:
            start = (ptr - self.base) // 4
            rows = self.ws[start:start + (r1 - r0) * ld].view(r1 - r0, ld)[:, :self.width]
            self.make_qkv(rows, r0, r1)
        except BaseException as e:  # an exception cannot cross the C frame
            self.error = e


def _chunk_workspace(ws: Workspace, tk: Tokens, off_host, sh, chunk: int):
    lib = _lib.load()
    import numpy as np
    oh = np.ascontiguousarray(off_host, dtype=np.int32)
    nbytes = lib.pet_attention_chunked_workspace(sh, oh.ctypes.data, chunk)
    return oh, ws.bytes("attention_chunked:scratch", nbytes), nbytes


def attention_chunked(ws: Workspace, key: str, out: torch.Tensor, make_qkv, cf_seq: torch.Tensor, w_out: torch.Tensor,
                      b_out: torch.Tensor | None, tk: Tokens, off_host, S: int, heads: int, head_dim: int,
                      temperature: float, save: bool, chunk: int) -> None:
    """pet::attention_chunked: attention() over runs of atoms of about
    ``chunk`` tokens; ``make_qkv(qkv_rows, r0, r1)`` writes the qkv rows of
    tokens [r0, r1) into ``qkv_rows``. ``off_host`` is off on the host."""
    lib = _lib.load()
    D = heads * head_dim
    T = out.shape[0]
    merged = ws.n2(key + ":merged", T, D) if save else torch.empty((T, D), dtype=torch.float32, device=out.device)
    ml = ws.n2(key + ":ml", tk.N * heads * S, 2) if save else None
    sh = shape(tk.N, T, S, heads, head_dim, temperature, tk.dead)
    oh, scratch, nbytes = _chunk_workspace(ws, tk, off_host, sh, chunk)
    cb = _RunRows(make_qkv, scratch, 3 * D)
    code = lib.pet_attention_chunked(sh, out.data_ptr(), _mat(out, "out", D), cb.cfunc, None, cf_seq.data_ptr(),
                                     _mat(cf_seq, "cf_seq"), _weight(w_out, "w_out"),
                                     None if b_out is None else _weight(b_out, "b_out"), tk.off.data_ptr(),
                                     oh.ctypes.data, merged.data_ptr(), _ptr(ml), chunk, scratch.data_ptr(), nbytes,
                                     _stream())
    if cb.error is not None:
        raise cb.error
    _lib.check(code, "pet_attention_chunked")


def attention_bwd_chunked(ws: Workspace, key: str, in_adj: torch.Tensor, cf_seq_adj: torch.Tensor,
                          out_adj: torch.Tensor, make_qkv, cf_seq: torch.Tensor, w_in: torch.Tensor,
                          w_out: torch.Tensor, tk: Tokens, off_host, S: int, heads: int, head_dim: int,
                          temperature: float, beta: float, chunk: int) -> None:
    """pet::attention_bwd_chunked over the same runs."""
    lib = _lib.load()
    D = heads * head_dim
    T = in_adj.shape[0]
    merged, ml = ws.peek2(key + ":merged"), ws.peek2(key + ":ml")
    sh = shape(tk.N, T, S, heads, head_dim, temperature, tk.dead)
    oh, scratch, nbytes = _chunk_workspace(ws, tk, off_host, sh, chunk)
    cb = _RunRows(make_qkv, scratch, 3 * D)
    d_in = w_in.shape[1]
    code = lib.pet_attention_bwd_chunked(sh, in_adj.data_ptr(), _mat(in_adj, "in_adj", d_in), d_in,
                                         cf_seq_adj.data_ptr(), _mat(cf_seq_adj, "cf_seq_adj"), out_adj.data_ptr(),
                                         _mat(out_adj, "out_adj", D), cb.cfunc, None, cf_seq.data_ptr(),
                                         _mat(cf_seq, "cf_seq"), _weight(w_in, "w_in"), _weight(w_out, "w_out"),
                                         tk.off.data_ptr(), oh.ctypes.data, merged.data_ptr(), ml.data_ptr(),
                                         float(beta), chunk, scratch.data_ptr(), nbytes, _stream())
    if cb.error is not None:
        raise cb.error
    _lib.check(code, "pet_attention_bwd_chunked")
