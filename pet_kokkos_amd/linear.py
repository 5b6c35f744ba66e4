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

import torch

from . import _lib


class SplitWeights:
    """W [N, K] (K a multiple of 32) as its three bf16 parts, N K 6 bytes of
    device memory: made once, then used in place of W by every call."""

    def __init__(self, W: torch.Tensor):
        N, K = W.shape
        self.shape = (N, K)
        self.data = torch.empty(N * K * 3, dtype=torch.int16, device=W.device)
        _lib.check(_lib.load().pet_linear_split_weights(W.data_ptr(), N, K, W.stride(0), self.data.data_ptr(),
                                                        torch.cuda.current_stream().cuda_stream),
                   "pet_linear_split_weights")


def _call(A, W, C, row_scale=None, bias=None, cin=None, beta=0.0, pre=None, act=0):
    M, K = A.shape
    p = lambda t: None if t is None else t.data_ptr()
    ld = lambda t: 0 if t is None else t.stride(0)
    st = torch.cuda.current_stream().cuda_stream
    lib = _lib.load()
    if isinstance(W, SplitWeights):
        N = W.shape[0]
        if W.shape[1] != K:
            raise ValueError("A and W disagree on K")
        _lib.check(lib.pet_linear_fused_split(M, N, K, p(A), A.stride(0), W.data.data_ptr(), p(C), C.stride(0),
                                              p(row_scale), p(bias), p(cin), ld(cin), beta, p(pre), ld(pre), act, st),
                   "pet_linear_fused_split")
    else:
        N = W.shape[0]
        _lib.check(lib.pet_linear_fused(M, N, K, p(A), A.stride(0), p(W), W.stride(0), p(C), C.stride(0),
                                        p(row_scale), p(bias), p(cin), ld(cin), beta, p(pre), ld(pre), act, st),
                   "pet_linear_fused")


def fused(A, W, C, row_scale=None, bias=None, cin=None, beta=0.0, pre=None, act=0):
    """C = act(row_scale * (A W^T) + bias + beta cin), pre = the value before
    act; act 0 none, 1 SiLU, 2 SwiGLU (C [M, N/2]). W a tensor or SplitWeights."""
    _call(A, W, C, row_scale, bias, cin, beta, pre, act)


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
