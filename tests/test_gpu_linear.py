"""The fused dense layer (pet_linear_fused, csrc/gemm.hip) against float64
matrix products of the same fp32 inputs, for every epilogue: a row scale (the
RMSNorm fold), a bias, a residual accumulated in place, the kept
pre-activation, SiLU and SwiGLU. Tolerance 1e-5 of the largest output
magnitude (fp32 sums over K <= 1024); runs repeat bit for bit."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from pet_kokkos_amd import _lib

pytestmark = pytest.mark.gpu


def linear_fused(A, W, C, row_scale=None, bias=None, cin=None, beta=0.0, pre=None, act=0):
    M, K = A.shape
    N = W.shape[0]
    p = lambda t: None if t is None else t.data_ptr()
    _lib.check(_lib.load().pet_linear_fused(M, N, K, p(A), A.stride(0), p(W), W.stride(0), p(C), C.stride(0),
                                            p(row_scale), p(bias), p(cin), 0 if cin is None else cin.stride(0),
                                            beta, p(pre), 0 if pre is None else pre.stride(0), act,
                                            torch.cuda.current_stream().cuda_stream), "pet_linear_fused")


SHAPES = [(1, 16, 16), (37, 40, 32), (300, 128, 128), (2049, 96, 256), (5000, 384, 128), (1000, 1024, 512),
          (129, 64, 1024)]


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_plain_and_bias(M, N, K, device):
    g = torch.Generator(device=device).manual_seed(M + N + K)
    A = torch.randn(M, K, device=device, generator=g)
    W = torch.randn(N, K, device=device, generator=g) / K ** 0.5
    b = torch.randn(N, device=device, generator=g)
    C = torch.empty(M, N, device=device)
    linear_fused(A, W, C, bias=b)
    ref = (A.double() @ W.double().T + b.double()).cpu().numpy()
    got = C.cpu().numpy()
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()
    C2 = torch.empty_like(C)
    linear_fused(A, W, C2, bias=b)
    assert torch.equal(C, C2)


def test_epilogues(device):
    M, N, K = 777, 256, 128
    g = torch.Generator(device=device).manual_seed(5)
    A = torch.randn(M, K, device=device, generator=g)
    W = torch.randn(N, K, device=device, generator=g) / K ** 0.5
    b = torch.randn(N, device=device, generator=g)
    rs = torch.rand(M, device=device, generator=g) + 0.5
    R = torch.randn(M, N, device=device, generator=g)
    base = (A.double() @ W.double().T) * rs.double()[:, None] + b.double()
    # residual in place: C = base + 1.0 * C
    C = R.clone()
    linear_fused(A, W, C, row_scale=rs, bias=b, cin=C, beta=1.0)
    ref = base + R.double()
    assert (C.double() - ref).abs().max().item() <= 1e-5 * ref.abs().max().item()
    # SiLU with the pre-activation kept
    C = torch.empty(M, N, device=device)
    pre = torch.empty(M, N, device=device)
    linear_fused(A, W, C, row_scale=rs, bias=b, pre=pre, act=1)
    assert (pre.double() - base).abs().max().item() <= 1e-5 * base.abs().max().item()
    ref = base * torch.sigmoid(base)
    assert (C.double() - ref).abs().max().item() <= 1e-5 * ref.abs().max().item()
    # SwiGLU: columns (2c, 2c + 1) = (value, gate) -> column c
    C = torch.empty(M, N // 2, device=device)
    linear_fused(A, W, C, bias=b, pre=pre, act=2)
    z = A.double() @ W.double().T + b.double()
    ref = z[:, 0::2] * torch.sigmoid(z[:, 1::2])
    assert (C.double() - ref).abs().max().item() <= 1e-5 * ref.abs().max().item()
    assert (pre.double() - z).abs().max().item() <= 1e-5 * z.abs().max().item()


def test_rejects(device):
    A = torch.zeros(8, 20, device=device)
    W = torch.zeros(8, 20, device=device)
    C = torch.zeros(8, 8, device=device)
    with pytest.raises(_lib.PetAttnError):
        linear_fused(A, W, C)  # K not a multiple of 16
