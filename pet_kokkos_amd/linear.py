"""The fused dense layers over torch device memory: C = epilogue(A W^T) on the
fp32 matrix cores (pet_linear_fused), or on the bf16 ones at fp32 accuracy
from weights split once (pet_linear_split_weights + pet_linear_fused_split).

The reference's fused GEMMs (src/ops.hpp:84-96, src/fused_gemm_hip.cpp:345-400)
by the same names: linear_fused (out = in W^T + b + beta out), silu_in_fused
(out = silu(in W^T + b), pre kept) and swiglu_in_fused (pre = in W^T + b with
W's rows interleaved value/gate, h = v sigmoid(g)). W is torch Linear's
[N, K]; every call raises on a bad shape or alignment instead of returning
false, since there is no other path here to fall back to.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib


class SplitWeights:
    """W [N, K] (K a multiple of 32) split for the 16-bit matrix cores (fp16
    pairs of power-of-two-scaled rows from K = 256, three bf16 parts below),
    at most N K 6 bytes of device memory: made once, then used in place of W
    by every call."""

    def __init__(self, W: torch.Tensor, transposed: bool = False):
        """transposed: the split of W^T, from W [K, N] as it is stored."""
        _check(W, "W")
        N, K = (W.shape[1], W.shape[0]) if transposed else W.shape
        self.shape = (N, K)
        self.data = torch.empty(N * K * 3, dtype=torch.int16, device=W.device)
        fn = _lib.load().pet_linear_split_weights_transposed if transposed else _lib.load().pet_linear_split_weights
        _lib.check(fn(W.data_ptr(), N, K, W.stride(0), self.data.data_ptr(), torch.cuda.current_stream().cuda_stream),
                   "pet_linear_split_weights" + ("_transposed" if transposed else ""))


class PairWeights:
    """W [N, K] (K a multiple of 32) as rows of three fp16 parts at any K
    (each row scaled by a power of two; hi, mid and lo, their sum W s
    exactly), N K 6 + N 4 bytes: the weights of the short-contraction layer
    (pet_linear_fused_smallk, K at most 128)."""

    def __init__(self, W: torch.Tensor):
        _check(W, "W")
        N, K = W.shape
        if K % 32:
            raise ValueError(f"W has K = {K}: pair weights need K a multiple of 32")
        self.shape = (N, K)
        self.data = torch.empty(N * K * 3 + 2 * N + 8, dtype=torch.int16, device=W.device)
        _lib.check(_lib.load().pet_linear_pair_weights(W.data_ptr(), N, K, W.stride(0), self.data.data_ptr(),
                                                       torch.cuda.current_stream().cuda_stream),
                   "pet_linear_pair_weights")


class PairRows:
    """A [M, K] (K a multiple of 32 and at least 256) as fp16 pairs of
    power-of-two-scaled rows, M K 4 + M 4 bytes of device memory: made once
    (pet_linear_pair_rows), then used in place of A by any number of products
    with split weights; their results are those of A itself, bit for bit."""

    def __init__(self, A: torch.Tensor):
        _check(A, "A")
        M, K = A.shape
        if K % 32 or K < 256:
            raise ValueError(f"A has K = {K}: the pair rows need K a multiple of 32 and at least 256")
        self.shape = (M, K)
        self.data = torch.empty(M * K * 2 + 2 * M + 8, dtype=torch.int16, device=A.device)
        _lib.check(_lib.load().pet_linear_pair_rows(A.data_ptr(), M, K, A.stride(0), self.data.data_ptr(),
                                                    torch.cuda.current_stream().cuda_stream),
                   "pet_linear_pair_rows")


class BlockPairs:
    """A product's output [M, cols] (cols a multiple of 32) as block pairs, made
    by fused_to_blocks (pet_linear_fused_split_blocks): fp16 pairs scaled per
    (row, block of kb columns), then the blocks' inverse scales. Read in place
    of A by fused() with SplitWeights (pet_linear_fused_blocks)."""

    def __init__(self, M: int, cols: int, device):
        if cols % 32:
            raise ValueError(f"block pairs need a multiple of 32 columns, not {cols}")
        self.shape = (M, cols)
        self.kb = None  # set by the product that writes them
        self.data = torch.empty(M * cols * 2 + 2 * M * (cols // 32) + 8, dtype=torch.int16, device=device)


def _out_cols(N, act):
    return N // 2 if act == 2 else 2 * N if act == 4 else N


def fused_to_blocks(A, W, out, row_scale=None, bias=None, cin=None, beta=0.0, pre=None, act=0, scratch=None):
    """fused() with the output act(...) written as block pairs into `out`
    (BlockPairs [M, N / 2 | 2 N | N] by act) instead of an fp32 C: W as
    SplitWeights, K a multiple of 32 and at least 256, N >= 512 and a multiple
    of 128, `scratch` the workspace A's rows are split into a chunk at a time."""
    _check(A, "A")
    if not isinstance(W, SplitWeights) or not isinstance(out, BlockPairs):
        raise ValueError("block pairs out need W as SplitWeights and out as BlockPairs")
    M, K = A.shape
    N = W.shape[0]
    if W.shape[1] != K:
        raise ValueError(f"A has K = {K}, W has K = {W.shape[1]}")
    if out.shape != (M, _out_cols(N, act)):
        raise ValueError(f"out is {out.shape}, the product gives {(M, _out_cols(N, act))}")
    if scratch is None or scratch.device != A.device or not scratch.is_contiguous():
        raise ValueError("scratch: a contiguous tensor on A's device")
    dev = A.device
    width = 2 * N if act == 4 else N
    if row_scale is not None:
        _check(row_scale, "row_scale", M, vector=True, device=dev)
    if bias is not None:
        _check(bias, "bias", width, vector=True, device=dev)
    if cin is not None:
        _check(cin, "cin", M, width, device=dev)
    if pre is not None:
        _check(pre, "pre", M, N, device=dev)
    p = lambda t: None if t is None else t.data_ptr()
    ld = lambda t: 0 if t is None else t.stride(0)
    kb = ctypes.c_int(0)
    _lib.check(_lib.load().pet_linear_fused_split_blocks(
        M, N, K, p(A), A.stride(0), W.data.data_ptr(), out.data.data_ptr(), p(row_scale), p(bias), p(cin), ld(cin),
        beta, p(pre), ld(pre), act, scratch.data_ptr(), scratch.numel() * scratch.element_size(), ctypes.byref(kb),
        torch.cuda.current_stream().cuda_stream), "pet_linear_fused_split_blocks")
    out.kb = kb.value


def norm_pair_rows(X, weight, bias=None):
    """norm(X) (RMSNorm, or LayerNorm with a bias: pet_norm_rows) made
    directly as PairRows (pet_norm_rows_pairs): the same bits as PairRows of
    the fp32 norm, with no fp32 round trip. X [M, K], K a multiple of 32 from
    256 to 2048."""
    _check(X, "X")
    M, K = X.shape
    if K % 32 or K < 256 or K > 2048:
        raise ValueError(f"X has K = {K}: the norm's pair rows need K a multiple of 32 from 256 to 2048")
    _check(weight, "weight", K, vector=True, device=X.device)
    if bias is not None:
        _check(bias, "bias", K, vector=True, device=X.device)
    out = PairRows.__new__(PairRows)
    out.shape = (M, K)
    out.data = torch.empty(M * K * 2 + 2 * M + 8, dtype=torch.int16, device=X.device)
    _lib.check(_lib.load().pet_norm_rows_pairs(M, K, out.data.data_ptr(), X.data_ptr(), X.stride(0),
                                               weight.data_ptr(), None if bias is None else bias.data_ptr(),
                                               torch.cuda.current_stream().cuda_stream), "pet_norm_rows_pairs")
    return out


def _check(t, name, rows=None, cols=None, vector=False, device=None):
    """A float32 CUDA tensor, unit stride along its last axis, of the stated
    extents (a row may be longer than `cols` in a 2-D view: the leading
    dimension is passed)."""
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: a torch tensor is needed")
    if t.dtype != torch.float32:
        raise ValueError(f"{name}: float32 is needed, not {t.dtype}")
    if not t.is_cuda or (device is not None and t.device != device):
        raise ValueError(f"{name}: on {t.device}, the operands' device is {device}")
    if t.dim() != (1 if vector else 2):
        raise ValueError(f"{name}: {1 if vector else 2}-D is needed, not shape {tuple(t.shape)}")
    if t.numel() > 1 and t.stride(-1) != 1:
        raise ValueError(f"{name}: the last axis must be contiguous (stride 1)")
    if vector:
        if rows is not None and t.shape[0] < rows:
            raise ValueError(f"{name}: {t.shape[0]} entries, {rows} needed")
        return
    if t.dim() == 2 and t.shape[0] > 1 and t.stride(0) < t.shape[1]:
        raise ValueError(f"{name}: rows overlap (stride {t.stride(0)} < width {t.shape[1]})")
    if rows is not None and t.shape[0] < rows:
        raise ValueError(f"{name}: {t.shape[0]} rows, {rows} needed")
    if cols is not None and t.shape[1] != cols:
        raise ValueError(f"{name}: {t.shape[1]} columns, {cols} needed")


def _call(A, W, C, row_scale=None, bias=None, cin=None, beta=0.0, pre=None, act=0, scratch=None):
    if act not in (0, 1, 2, 3, 4):
        raise ValueError(f"act {act}: 0 (none), 1 (SiLU), 2 (SwiGLU), 3 / 4 (their backward)")
    if isinstance(A, (PairRows, BlockPairs)):
        if not isinstance(W, SplitWeights):
            raise ValueError("A as pair rows or block pairs needs W as SplitWeights")
        if isinstance(A, BlockPairs) and A.kb is None:
            raise ValueError("A: block pairs no product has written")
        M, K = A.shape
        dev = A.data.device
    else:
        _check(A, "A")
        M, K = A.shape
        dev = A.device
    if isinstance(W, (SplitWeights, PairWeights)):
        N, Kw = W.shape
        if W.data.device != dev:
            raise ValueError(f"W: on {W.data.device}, A on {dev}")
    else:
        _check(W, "W", device=dev)
        N, Kw = W.shape
    if Kw != K:
        raise ValueError(f"A has K = {K}, W has K = {Kw}")
    if act == 2 and N % 2:
        raise ValueError("SwiGLU needs an even number of weight rows (value, gate pairs)")
    # the backward codes: cin is the saved pre-activation, 2N wide (pairs) for SwiGLU's
    width = 2 * N if act == 4 else N
    if act >= 3 and (cin is None or row_scale is not None or pre is not None):
        raise ValueError(f"act {act}: cin (the pre-activation) is required, row_scale and pre are not taken")
    _check(C, "C", M, N // 2 if act == 2 else width, device=dev)
    if row_scale is not None:
        _check(row_scale, "row_scale", M, vector=True, device=dev)
    if bias is not None:
        _check(bias, "bias", width, vector=True, device=dev)
    if cin is not None:
        _check(cin, "cin", M, width, device=dev)
    if pre is not None:
        _check(pre, "pre", M, N, device=dev)
    p = lambda t: None if t is None else t.data_ptr()
    ld = lambda t: 0 if t is None else t.stride(0)
    st = torch.cuda.current_stream().cuda_stream
    lib = _lib.load()
    if isinstance(W, PairWeights):
        if isinstance(A, PairRows) or K > 128:
            raise ValueError("pair weights take fp32 A and K at most 128 (pet_linear_fused_smallk)")
        _lib.check(lib.pet_linear_fused_smallk(M, N, K, p(A), A.stride(0), W.data.data_ptr(), p(C), C.stride(0),
                                               p(row_scale), p(bias), p(cin), ld(cin), beta, p(pre), ld(pre), act, st),
                   "pet_linear_fused_smallk")
    elif isinstance(A, BlockPairs):
        _lib.check(lib.pet_linear_fused_blocks(M, N, K, A.data.data_ptr(), A.kb, W.data.data_ptr(), p(C), C.stride(0),
                                               p(row_scale), p(bias), p(cin), ld(cin), beta, p(pre), ld(pre), act, st),
                   "pet_linear_fused_blocks")
    elif isinstance(A, PairRows):
        _lib.check(lib.pet_linear_fused_pairs(M, N, K, A.data.data_ptr(), W.data.data_ptr(), p(C), C.stride(0),
                                              p(row_scale), p(bias), p(cin), ld(cin), beta, p(pre), ld(pre), act, st),
                   "pet_linear_fused_pairs")
    elif isinstance(W, SplitWeights) and scratch is not None:
        if scratch.device != dev or not scratch.is_contiguous():
            raise ValueError("scratch: a contiguous tensor on A's device")
        _lib.check(lib.pet_linear_fused_split_ws(M, N, K, p(A), A.stride(0), W.data.data_ptr(), p(C), C.stride(0),
                                                 p(row_scale), p(bias), p(cin), ld(cin), beta, p(pre), ld(pre), act,
                                                 scratch.data_ptr(), scratch.numel() * scratch.element_size(), st),
                   "pet_linear_fused_split_ws")
    elif isinstance(W, SplitWeights):
        _lib.check(lib.pet_linear_fused_split(M, N, K, p(A), A.stride(0), W.data.data_ptr(), p(C), C.stride(0),
                                              p(row_scale), p(bias), p(cin), ld(cin), beta, p(pre), ld(pre), act, st),
                   "pet_linear_fused_split")
    else:
        _lib.check(lib.pet_linear_fused(M, N, K, p(A), A.stride(0), p(W), W.stride(0), p(C), C.stride(0),
                                        p(row_scale), p(bias), p(cin), ld(cin), beta, p(pre), ld(pre), act, st),
                   "pet_linear_fused")


def fused(A, W, C, row_scale=None, bias=None, cin=None, beta=0.0, pre=None, act=0, scratch=None):
    """C = act(row_scale * (A W^T) + bias + beta cin), pre = the value before
    act; act 0 none, 1 SiLU, 2 SwiGLU (C [M, N/2]). W a tensor or SplitWeights;
    A a tensor or, with W as SplitWeights, PairRows.
    act 3 / 4: A W^T is the adjoint of a SiLU / SwiGLU output and cin its saved
    pre-activation z (bias z's bias if not yet in it): C = adjoint silu'(z), or
    for SwiGLU (z and C [M, 2N], (value, gate) pairs) each pair's adjoint.
    With W as SplitWeights, `scratch` (a device tensor) is the workspace A's
    rows are split into a chunk at a time (pet_linear_fused_split_ws)."""
    _call(A, W, C, row_scale, bias, cin, beta, pre, act, scratch)


def linear_fused(out, inp, W, b=None, beta=0.0):
    """out = inp W^T + b + beta out (the reference's linear_fused, W transposed)."""
    _call(inp, W, out, bias=b, cin=out if beta != 0.0 else None, beta=beta)


def silu_in_fused(out, pre, inp, W, b=None):
    """out = silu(inp W^T + b), pre = inp W^T + b unless None."""
    _call(inp, W, out, bias=b, pre=pre, act=1)


def swiglu_in_fused(pre, h, inp, W, b):
    """pre = inp W^T + b (W's rows interleaved value/gate), h = v sigmoid(g)
    unless None (then only pre is made)."""
    if h is None:
        _call(inp, W, pre, bias=b)
    else:
        _call(inp, W, h, bias=b, pre=pre, act=2)
