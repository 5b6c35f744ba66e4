"""The fused dense layer (pet_linear_fused, csrc/gemm.hip) against float64
matrix products of the same fp32 inputs, for every epilogue: a row scale (the
RMSNorm fold), a bias, a residual accumulated in place, the kept
pre-activation, SiLU and SwiGLU, and their backward (act 3, 4). Tolerance 1e-5 of the largest output
magnitude (fp32 sums over K <= 1024); runs repeat bit for bit. The same for
its split-product form (pet_linear_fused_split over weights split by
pet_linear_split_weights), whose split is checked exactly: three bf16 parts
that sum to each weight."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from pet_kokkos_amd import _lib
from pet_kokkos_amd import linear as L

pytestmark = pytest.mark.gpu


def split_weights(W):
    return L.SplitWeights(W)


def linear_fused(A, W, C, row_scale=None, bias=None, cin=None, beta=0.0, pre=None, act=0, split=False):
    # split: False (fp32 products), True (split weights), "smallk" (pair weights, K <= 128)
    Wf = L.PairWeights(W) if split == "smallk" else split_weights(W) if split else W
    L.fused(A, Wf, C, row_scale, bias, cin, beta, pre, act)


# the last two are large enough for the split form's 128 x 128 and 128 x 64 tiles
# (1001, 38, 96): a width not a multiple of 4 (the short-K kernel's per-element
# epilogue) and 12 k groups a row (its rows padded to 16 lanes); (3, 130, 64),
# (5, 130, 128): fewer rows than one block, most XCDs' row ranges empty
SHAPES = [(1, 16, 16), (37, 40, 32), (300, 128, 128), (2049, 96, 256), (5000, 384, 128), (1000, 1024, 512),
          (129, 64, 1024), (16385, 1024, 64), (131071, 96, 64), (1001, 38, 96), (3, 130, 64), (5, 130, 128)]


@pytest.mark.parametrize("split", [False, True, "smallk"], ids=["fp32", "split", "smallk"])
@pytest.mark.parametrize("M,N,K", SHAPES)
def test_plain_and_bias(M, N, K, split, device):
    if split and K % 32:
        pytest.skip("the split form needs K a multiple of 32")
    if split == "smallk" and K > 128:
        pytest.skip("the short-contraction layer takes K at most 128")
    g = torch.Generator(device=device).manual_seed(M + N + K)
    A = torch.randn(M, K, device=device, generator=g)
    W = torch.randn(N, K, device=device, generator=g) / K ** 0.5
    b = torch.randn(N, device=device, generator=g)
    C = torch.empty(M, N, device=device)
    linear_fused(A, W, C, bias=b, split=split)
    ref = (A.double() @ W.double().T + b.double()).cpu().numpy()
    got = C.cpu().numpy()
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()
    C2 = torch.empty_like(C)
    linear_fused(A, W, C2, bias=b, split=split)
    assert torch.equal(C, C2)


@pytest.mark.parametrize("split", [False, True, "smallk"], ids=["fp32", "split", "smallk"])
@pytest.mark.parametrize("M,N,K", [(777, 256, 128), (1001, 38, 96)])
def test_epilogues(M, N, K, split, device):
    g = torch.Generator(device=device).manual_seed(5)
    A = torch.randn(M, K, device=device, generator=g)
    W = torch.randn(N, K, device=device, generator=g) / K ** 0.5
    b = torch.randn(N, device=device, generator=g)
    rs = torch.rand(M, device=device, generator=g) + 0.5
    R = torch.randn(M, N, device=device, generator=g)
    base = (A.double() @ W.double().T) * rs.double()[:, None] + b.double()
    # residual in place: C = base + 1.0 * C
    C = R.clone()
    linear_fused(A, W, C, row_scale=rs, bias=b, cin=C, beta=1.0, split=split)
    ref = base + R.double()
    assert (C.double() - ref).abs().max().item() <= 1e-5 * ref.abs().max().item()
    # SiLU with the pre-activation kept
    C = torch.empty(M, N, device=device)
    pre = torch.empty(M, N, device=device)
    linear_fused(A, W, C, row_scale=rs, bias=b, pre=pre, act=1, split=split)
    assert (pre.double() - base).abs().max().item() <= 1e-5 * base.abs().max().item()
    ref = base * torch.sigmoid(base)
    assert (C.double() - ref).abs().max().item() <= 1e-5 * ref.abs().max().item()
    # SwiGLU: columns (2c, 2c + 1) = (value, gate) -> column c
    C = torch.empty(M, N // 2, device=device)
    linear_fused(A, W, C, bias=b, pre=pre, act=2, split=split)
    z = A.double() @ W.double().T + b.double()
    ref = z[:, 0::2] * torch.sigmoid(z[:, 1::2])
    assert (C.double() - ref).abs().max().item() <= 1e-5 * ref.abs().max().item()
    assert (pre.double() - z).abs().max().item() <= 1e-5 * z.abs().max().item()


@pytest.mark.parametrize("split", [False, True, "smallk"], ids=["fp32", "split", "smallk"])
@pytest.mark.parametrize("M,N,K", [(300, 128, 128), (16385, 512, 256), (1001, 38, 96), (5000, 64, 32)])
def test_backward_epilogues(M, N, K, split, device):
    """act 3 / 4: the SiLU / SwiGLU backward fused into the input-adjoint
    product (A W^T is the activation output's adjoint, cin the saved
    pre-activation, bias its bias when not yet added), against float64."""
    if split == "smallk" and K > 128:
        pytest.skip("the short-contraction layer takes K at most 128")
    g = torch.Generator(device=device).manual_seed(M + N)
    A = torch.randn(M, K, device=device, generator=g)
    W = torch.randn(N, K, device=device, generator=g) / K ** 0.5
    v = A.double() @ W.double().T
    for with_bias in (False, True):
        # SiLU: C = v silu'(z), z = cin (+ bias)
        z = 3.0 * torch.randn(M, N, device=device, generator=g)
        b = torch.randn(N, device=device, generator=g) if with_bias else None
        zz = z.double() + (b.double() if with_bias else 0.0)
        sg = torch.sigmoid(zz)
        ref = v * (sg * (1.0 + zz * (1.0 - sg)))
        C = torch.empty(M, N, device=device)
        linear_fused(A, W, C, bias=b, cin=z, act=3, split=split)
        assert (C.double() - ref).abs().max().item() <= 1e-5 * ref.abs().max().item()
        C2 = torch.empty_like(C)
        linear_fused(A, W, C2, bias=b, cin=z, act=3, split=split)
        assert torch.equal(C, C2)
        # SwiGLU: z [M, 2N] of (value u, gate g) pairs; C [M, 2N] their adjoints
        z2 = 3.0 * torch.randn(M, 2 * N, device=device, generator=g)
        b2 = torch.randn(2 * N, device=device, generator=g) if with_bias else None
        zz = z2.double() + (b2.double() if with_bias else 0.0)
        u, sg = zz[:, 0::2], torch.sigmoid(zz[:, 1::2])
        ref = torch.empty(M, 2 * N, dtype=torch.float64, device=device)
        ref[:, 0::2] = v * sg
        ref[:, 1::2] = v * u * sg * (1.0 - sg)
        C = torch.empty(M, 2 * N, device=device)
        linear_fused(A, W, C, bias=b2, cin=z2, act=4, split=split)
        assert (C.double() - ref).abs().max().item() <= 1e-5 * ref.abs().max().item()
    A, W, C = torch.zeros(8, 32, device=device), torch.zeros(8, 32, device=device), torch.zeros(8, 8, device=device)
    with pytest.raises(ValueError):
        linear_fused(A, W, C, act=3, split=split)  # no pre-activation
    with pytest.raises(ValueError):
        linear_fused(A, W, C, cin=C, act=4, split=split)  # SwiGLU's C and cin are 2N wide
    with pytest.raises(ValueError):
        linear_fused(A, W, C, cin=C, pre=C, act=3, split=split)  # no pre taken
    with pytest.raises(ValueError):
        linear_fused(A, W, C, cin=C, act=5, split=split)


def test_rejects(device):
    A = torch.zeros(8, 20, device=device)
    W = torch.zeros(8, 20, device=device)
    C = torch.zeros(8, 8, device=device)
    with pytest.raises(_lib.PetAttnError):
        linear_fused(A, W, C)  # K not a multiple of 16
    with pytest.raises(_lib.PetAttnError):
        linear_fused(torch.zeros(8, 0, device=device), torch.zeros(8, 0, device=device), C)  # K = 0
    A, W = torch.zeros(8, 32, device=device), torch.zeros(8, 32, device=device)
    with pytest.raises(ValueError):
        linear_fused(A, W, torch.zeros(7, 8, device=device))  # C too short
    with pytest.raises(ValueError):
        linear_fused(A, W, torch.zeros(8, 4, device=device))  # C too narrow
    with pytest.raises(ValueError):
        linear_fused(A, W, torch.zeros(8, 8, device=device, dtype=torch.float64))  # not float32
    with pytest.raises(ValueError):
        linear_fused(A.double(), W, C)
    with pytest.raises(ValueError):
        linear_fused(A, W, torch.zeros(8, 16, device=device)[:, ::2])  # strided columns
    with pytest.raises(ValueError):
        linear_fused(A, W, C, bias=torch.zeros(7, device=device))  # bias too short
    with pytest.raises(ValueError):
        linear_fused(A, W, C, row_scale=torch.zeros(3, device=device))
    with pytest.raises(ValueError):
        linear_fused(A, W, C, pre=torch.zeros(8, 7, device=device), act=1)
    with pytest.raises(ValueError):
        linear_fused(A, W, C, cin=torch.zeros(4, 8, device=device), beta=1.0)
    with pytest.raises(ValueError):
        linear_fused(A, W.cpu(), C)  # not on the device
    with pytest.raises(ValueError):
        linear_fused(A, torch.zeros(7, 32, device=device), torch.zeros(8, 4, device=device), act=2)  # odd SwiGLU rows
    with pytest.raises(ValueError):
        split_weights(torch.zeros(8, 32, device=device, dtype=torch.float64))


@pytest.mark.parametrize("split", [False, True], ids=["fp32", "split"])
def test_rows_past_a_2d_grid(split, device):
    # more 64-row tiles than a grid's y extent (65535) holds: both kernels run
    # a 1-D grid of tiles
    M, N, K = 65535 * 64 + 100, 16, 32
    print(f"[gpu] linear M={M} N={N} K={K} split={split}", flush=True)
    g = torch.Generator(device=device).manual_seed(21)
    A = torch.randn(M, K, device=device, generator=g)
    W = torch.randn(N, K, device=device, generator=g) / K ** 0.5
    C = torch.empty(M, N, device=device)
    linear_fused(A, W, C, split=split)
    ref = A.double() @ W.double().T
    err = (C.double() - ref).abs().max().item()
    assert err <= 1e-5 * ref.abs().max().item()
    assert (C[-1].double() - ref[-1]).abs().max().item() <= 1e-5 * ref.abs().max().item()


def test_split_weights_transposed_exact(device):
    # the layer backward's split of W^T (pet_gemm_split_weights, transposed)
    # holds the same bytes as the plain split of W^T made contiguous
    N, K = 96, 64
    g = torch.Generator(device=device).manual_seed(4)
    W = torch.randn(K, N, device=device, generator=g) * torch.logspace(-10, 10, N, device=device)
    a = L.SplitWeights(W, transposed=True).data  # [N, K] split rows of W^T
    b = split_weights(W.t().contiguous()).data
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_split_weights_exact(device):
    """Each weight's three parts are bf16 values (an fp32 with a zero low half)
    that sum to it exactly, part 0 carrying its leading bits, laid out per row
    and 8-element k group as parts 0, 1, 2."""
    N, K = 48, 64
    g = torch.Generator(device=device).manual_seed(3)
    W = torch.randn(N, K, device=device, generator=g) * torch.logspace(-20, 20, K, device=device)
    Ws = split_weights(W).data.cpu().numpy().view(np.uint16).reshape(N, K // 8, 3, 8)
    parts = (Ws.astype(np.uint32) << 16).view(np.float32)  # [N, K/8, 3, 8]
    w = W.cpu().numpy().reshape(N, K // 8, 8)
    assert np.array_equal(parts[:, :, 0, :] + parts[:, :, 1, :] + parts[:, :, 2, :], w)
    assert np.array_equal(parts[:, :, 0, :], (w.view(np.uint32) & 0xFFFF0000).view(np.float32))
    assert np.all(np.abs(parts[:, :, 1, :]) <= np.abs(w) * 2.0 ** -7)


@pytest.mark.parametrize("transposed", [False, True], ids=["W", "W^T"])
def test_pair_weights_exact(transposed, device):
    """From K = 256 the split is fp16 pairs: per row a power-of-two scale s
    with max |w| s in [2^14, 2^15), then per 8-element k group a hi part (w s
    rounded to the nearest fp16) and a lo part (the rest, rounded to the
    nearest fp16: hi + lo within 2^-23 |w s|, or half an fp16 subnormal step
    below fp16's normal range), and after the N K 4 bytes of parts the rows' 1 / s.
    The split of W^T from W equals that of W^T made contiguous."""
    N, K = 40, 256
    g = torch.Generator(device=device).manual_seed(6)
    W = torch.randn(N, K, device=device, generator=g) * torch.logspace(-12, 12, K, device=device)
    W[3] *= 1e-30  # a row far below fp16's range before scaling
    W[5] = 0.0  # a zero row
    if transposed:
        Wt = W.t().contiguous()
        data = L.SplitWeights(Wt, transposed=True).data
        used = (N * K * 4 + 4 * N) // 2  # int16 elements written (the buffer is sized for the bf16 form)
        assert torch.equal(data[:used], split_weights(W).data[:used])
    else:
        data = split_weights(W).data
    raw = data.cpu().numpy().view(np.uint8)
    parts = raw[: N * K * 4].view(np.float16).reshape(N, K // 8, 2, 8).astype(np.float64)
    inv = raw[N * K * 4: N * K * 4 + 4 * N].view(np.float32).astype(np.float64)
    w = W.cpu().numpy().astype(np.float64).reshape(N, K // 8, 8)
    s = 1.0 / inv
    assert np.array_equal(np.exp2(np.round(np.log2(s))), s)  # powers of two
    m = np.abs(w).reshape(N, K).max(1)
    live = m > 0
    assert np.all((m[live] * s[live] >= 2.0 ** 14) & (m[live] * s[live] < 2.0 ** 15))
    assert s[5] == 1.0 and np.all(parts[5] == 0)
    ws = w * s[:, None, None]
    hi, lo = parts[:, :, 0, :], parts[:, :, 1, :]
    normal = np.abs(ws) >= 2.0 ** -14
    hi_ref = ws.astype(np.float32).astype(np.float16).astype(np.float64)  # to nearest (even)
    assert np.array_equal(hi[normal], hi_ref[normal])
    # lo of either sign (round to nearest), |lo| within half of hi's ulp
    assert np.any(lo[normal] < 0) and np.any(lo[normal] > 0)
    # below fp16's normal range hi and lo are rounded to the subnormal step (2^-24)
    assert np.all(np.abs(hi + lo - ws) <= 2.0 ** -23 * np.abs(ws) + 2.0 ** -25)


def test_split_rejects(device):
    W = torch.zeros(8, 48, device=device)
    with pytest.raises(_lib.PetAttnError):
        split_weights(W)  # K not a multiple of 32


def test_reference_named_wrappers(device):
    """linear_fused / silu_in_fused / swiglu_in_fused, as the reference names
    them, on both weight forms."""
    M, N, K = 300, 64, 96
    g = torch.Generator(device=device).manual_seed(9)
    A = torch.randn(M, K, device=device, generator=g)
    W = torch.randn(N, K, device=device, generator=g) / K ** 0.5
    b = torch.randn(N, device=device, generator=g)
    z = A.double() @ W.double().T + b.double()
    tol = lambda ref: 1e-5 * ref.abs().max().item()
    for w in (W, L.SplitWeights(W)):
        out = torch.randn(M, N, device=device, generator=g)
        base = out.double().clone()
        L.linear_fused(out, A, w, b, beta=1.0)
        assert (out.double() - (z + base)).abs().max().item() <= tol(z + base)
        out, pre = torch.empty(M, N, device=device), torch.empty(M, N, device=device)
        L.silu_in_fused(out, pre, A, w, b)
        assert (pre.double() - z).abs().max().item() <= tol(z)
        assert (out.double() - z * torch.sigmoid(z)).abs().max().item() <= tol(z * torch.sigmoid(z))
        h = torch.empty(M, N // 2, device=device)
        L.swiglu_in_fused(pre, h, A, w, b)
        ref = z[:, 0::2] * torch.sigmoid(z[:, 1::2])
        assert (h.double() - ref).abs().max().item() <= tol(ref)


# pairs-by-pairs (A split once into PairRows): whole 128 x 128 tiles take the
# LDS-staged epilogue, N = 300 and ragged M the per-element one; every epilogue
# must give the bits of the split-weights product from A itself
@pytest.mark.parametrize("M,N,K", [(1000, 1024, 512), (777, 300, 256), (20000, 2048, 512), (4096, 512, 1024),
                                   (300, 64, 288)])
def test_pair_rows_same_bits(M, N, K, device):
    print(f"[gpu] pair rows M={M} N={N} K={K}", flush=True)
    g = torch.Generator(device=device).manual_seed(M + N + K)
    A = torch.randn(M, K, device=device, generator=g) * 3.0
    W = torch.randn(N, K, device=device, generator=g) / K ** 0.5
    Ws, Ap = L.SplitWeights(W), L.PairRows(A)
    b = torch.randn(N, device=device, generator=g)
    b2 = torch.randn(2 * N, device=device, generator=g)
    rs = torch.rand(M, device=device, generator=g) + 0.5
    res = torch.randn(M, N, device=device, generator=g)
    z = torch.randn(M, N, device=device, generator=g)
    z2 = torch.randn(M, 2 * N, device=device, generator=g)
    cases = [dict(bias=b), dict(row_scale=rs, bias=b, cin=res, beta=0.5, pre="N"), dict(bias=b, pre="N", act=1),
             dict(bias=b, pre="N", act=2), dict(bias=b, cin=z, act=3), dict(bias=b2, cin=z2, act=4), dict()]
    for kw in cases:
        act = kw.get("act", 0)
        width = N // 2 if act == 2 else 2 * N if act == 4 else N
        outs = []
        for a in (A, Ap):
            C = torch.full((M, width), float("nan"), device=device)
            pre = torch.full((M, N), float("nan"), device=device) if kw.get("pre") else None
            L.fused(a, Ws, C, **{**kw, "pre": pre})
            outs.append((C, pre))
        assert torch.equal(outs[0][0], outs[1][0]), kw.keys()
        if outs[0][1] is not None:
            assert torch.equal(outs[0][1], outs[1][1])
    with pytest.raises(ValueError):
        L.fused(Ap, W, torch.empty(M, N, device=device))  # pair rows need split weights
    with pytest.raises(ValueError):
        L.PairRows(torch.zeros(8, 128, device=device))  # K below 256


def test_split_scratch_chunks_same_bits(device):
    # pet_linear_fused_split_ws with a scratch of 128 rows of pairs: A is split
    # and multiplied a chunk of 128 rows at a time (row_scale, cin, pre and C
    # moved along by each chunk's first row), 1000 rows in 8 chunks, the last
    # partial, against the product with no scratch, bit for bit, for every
    # epilogue
    M, N, K = 1000, 512, 256
    print(f"[gpu] split product with a 128-row scratch, M={M} N={N} K={K}", flush=True)
    g = torch.Generator(device=device).manual_seed(17)
    A = torch.randn(M, K, device=device, generator=g) * 3.0
    W = torch.randn(N, K, device=device, generator=g) / K ** 0.5
    Ws = L.SplitWeights(W)
    scratch = torch.empty(128 * (K * 4 + 4) // 4, device=device)
    b = torch.randn(N, device=device, generator=g)
    b2 = torch.randn(2 * N, device=device, generator=g)
    rs = torch.rand(M, device=device, generator=g) + 0.5
    res = torch.randn(M, N, device=device, generator=g)
    z = torch.randn(M, N, device=device, generator=g)
    z2 = torch.randn(M, 2 * N, device=device, generator=g)
    cases = [dict(bias=b), dict(row_scale=rs, bias=b, cin=res, beta=0.5, pre="N"), dict(bias=b, pre="N", act=1),
             dict(bias=b, pre="N", act=2), dict(bias=b, cin=z, act=3), dict(bias=b2, cin=z2, act=4), dict()]
    for kw in cases:
        act = kw.get("act", 0)
        width = N // 2 if act == 2 else 2 * N if act == 4 else N
        outs = []
        for sc in (None, scratch):
            C = torch.full((M, width), float("nan"), device=device)
            pre = torch.full((M, N), float("nan"), device=device) if kw.get("pre") else None
            L.fused(A, Ws, C, **{**kw, "pre": pre}, scratch=sc)
            outs.append((C, pre))
        assert not torch.isnan(outs[1][0]).any(), kw.keys()
        assert torch.equal(outs[0][0], outs[1][0]), kw.keys()
        if outs[0][1] is not None:
            assert torch.equal(outs[0][1], outs[1][1])


@pytest.mark.parametrize("K", [32, 64, 96, 128])
def test_smallk_rows_independent_of_M(K, device):
    # pet_linear_fused_smallk: a row's results are the same bits whatever
    # rows come with it (M, and where the row falls in a tile): the full
    # product against the product of rows 77 .. 77 + 301 alone, with SwiGLU and
    # the kept pre-activation, N 384 (six column tiles) and N 72 (a partial one)
    for N in (384, 72):
        M = 1000
        g = torch.Generator(device=device).manual_seed(K + N)
        A = torch.randn(M, K, device=device, generator=g) * torch.logspace(-3, 3, M, device=device)[:, None]
        W = L.PairWeights(torch.randn(N, K, device=device, generator=g) / K ** 0.5)
        b = torch.randn(N, device=device, generator=g)
        C, pre = torch.empty(M, N // 2, device=device), torch.empty(M, N, device=device)
        L.fused(A, W, C, bias=b, pre=pre, act=2)
        A2 = A[77:378].clone()
        C2, pre2 = torch.empty(301, N // 2, device=device), torch.empty(301, N, device=device)
        L.fused(A2, W, C2, bias=b, pre=pre2, act=2)
        assert torch.equal(C[77:378], C2) and torch.equal(pre[77:378], pre2)
        z = A.double() @ W_ref(W, device).T + b.double()
        assert (pre.double() - z).abs().max().item() <= 1e-5 * z.abs().max().item()


def smallk_parts(W):
    """The short-K weights' parts [N, K/8, 3, 8] (hi, mid, lo) and inverse scales [N], fp64."""
    N, K = W.shape
    raw = W.data.cpu().numpy().view(np.uint8)
    parts = raw[: N * K * 6].view(np.float16).reshape(N, K // 8, 3, 8).astype(np.float64)
    inv = raw[N * K * 6: N * K * 6 + 4 * N].view(np.float32).astype(np.float64)
    return parts, inv


def W_ref(W, device):
    """The fp64 matrix of part weights over each row's scale: the short-K
    weights' hi + mid + lo, or the pair form's hi + lo (SplitWeights from
    K = 256)."""
    N, K = W.shape
    if isinstance(W, L.PairWeights):
        parts, inv = smallk_parts(W)
    else:
        raw = W.data.cpu().numpy().view(np.uint8)
        parts = raw[: N * K * 4].view(np.float16).reshape(N, K // 8, 2, 8).astype(np.float64)
        inv = raw[N * K * 4: N * K * 4 + 4 * N].view(np.float32).astype(np.float64)
    w = parts.sum(axis=2).reshape(N, K) * inv[:, None]
    return torch.from_numpy(w).to(device)


def test_smallk_weights_exact(device):
    """pet_linear_pair_weights: per row a power-of-two scale s (max |w| s in
    [2^14, 2^15)), per element hi = w s to the nearest fp16, mid = the rest to
    the nearest fp16, lo = what is left: hi + mid + lo = w s exactly wherever
    |w s| >= 2^-1 (lo then holds at most 2 bits at an exponent fp16 reaches),
    within half an fp16 subnormal step below. So the weights the short-K
    kernel multiplies are W itself: a pair form (22 bits) would be a fixed
    perturbation of the model, the same error in every row's product."""
    N, K = 40, 128
    g = torch.Generator(device=device).manual_seed(16)
    W = torch.randn(N, K, device=device, generator=g) * torch.logspace(-10, 10, K, device=device)
    W[3] *= 1e-30  # a row far below fp16's range before scaling
    W[5] = 0.0  # a zero row
    W[7] = torch.randn(K, device=device, generator=g)  # an ordinary row
    parts, inv = smallk_parts(L.PairWeights(W))
    s = 1.0 / inv
    assert np.array_equal(np.exp2(np.round(np.log2(s))), s)
    w = W.cpu().numpy().astype(np.float64).reshape(N, K // 8, 8)
    m = np.abs(w).reshape(N, K).max(1)
    live = m > 0
    assert np.all((m[live] * s[live] >= 2.0 ** 14) & (m[live] * s[live] < 2.0 ** 15))
    assert s[5] == 1.0 and np.all(parts[5] == 0)
    ws = w * s[:, None, None]
    hi, mid, lo = parts[:, :, 0, :], parts[:, :, 1, :], parts[:, :, 2, :]
    big = np.abs(ws) >= 0.5
    assert np.array_equal(hi[big], ws[big].astype(np.float32).astype(np.float16).astype(np.float64))
    assert np.array_equal(mid[big], (ws[big] - hi[big]).astype(np.float32).astype(np.float16).astype(np.float64))
    assert np.array_equal((hi + mid + lo)[big], ws[big])
    assert np.all(np.abs(hi + mid + lo - ws) <= 2.0 ** -25)
    assert np.any(lo[big] != 0)  # the third part carries bits
    assert np.array_equal((hi + mid + lo)[7], ws[7])  # an ordinary row: every element exact


def blocks_ref(B, device):
    """The fp64 matrix of block pairs: (hi + lo) times each (row, block)'s
    inverse scale; and the scaled parts' largest |hi| per (row, block)."""
    M, cols = B.shape
    raw = B.data.cpu().numpy().view(np.uint8)
    parts = raw[: M * cols * 4].view(np.float16).reshape(M, cols // 8, 2, 8).astype(np.float64)
    nblk = cols // B.kb
    inv = raw[M * cols * 4: M * cols * 4 + 4 * M * nblk].view(np.float32).reshape(nblk, M).astype(np.float64)
    hi, lo = parts[:, :, 0, :].reshape(M, cols), parts[:, :, 1, :].reshape(M, cols)
    x = (hi + lo) * np.repeat(inv.T, B.kb, axis=1)
    hmax = np.abs(hi).reshape(M, nblk, B.kb).max(axis=2)
    return torch.from_numpy(x).to(device), hmax


@pytest.mark.parametrize("act", [0, 1, 2, 3, 4])
def test_block_pairs_out(act, device):
    # pet_linear_fused_split_blocks: the output act(...) as block pairs equals
    # the fp32 output of the same product (pet_linear_fused_split_ws, the same
    # kernel and epilogue arithmetic) within the split's rounding (hi and lo
    # both to nearest: 2^-22 of the value, or 2^-25 of the block's largest
    # below fp16's normal range), each block scaled so that its largest |hi|
    # lies in [2^14, 2^15]; rows 10^-3 .. 10^3 apart and one all-zero row;
    # the same bits whatever the scratch's chunking
    M, N, K = 1000, 512, 256
    print(f"[gpu] block pairs out, act {act}, M={M} N={N} K={K}", flush=True)
    g = torch.Generator(device=device).manual_seed(40 + act)
    A = torch.randn(M, K, device=device, generator=g) * torch.logspace(-3, 3, M, device=device)[:, None]
    A[500] = 0.0
    W = torch.randn(N, K, device=device, generator=g) / K ** 0.5
    Ws = L.SplitWeights(W)
    width = 2 * N if act == 4 else N
    kw = dict(bias=torch.randn(width, device=device, generator=g), act=act)
    if act >= 3:
        kw["cin"] = torch.randn(M, width, device=device, generator=g)
    else:
        kw["pre"] = torch.empty(M, N, device=device)
    if act == 0:
        kw["row_scale"] = torch.rand(M, device=device, generator=g) + 0.5
        kw["cin"], kw["beta"] = torch.randn(M, N, device=device, generator=g), 0.5
    cols = N // 2 if act == 2 else width
    big = torch.empty(M * (K * 4 + 4) // 4 + 64, device=device)
    small = torch.empty(128 * (K * 4 + 4) // 4, device=device)
    C = torch.empty(M, cols, device=device)
    L.fused(A, Ws, C, **kw, scratch=big)
    pre_ref = kw["pre"].clone() if "pre" in kw else None
    outs = []
    for sc in (big, small):
        B = L.BlockPairs(M, cols, device)
        L.fused_to_blocks(A, Ws, B, **kw, scratch=sc)
        torch.cuda.synchronize()
        outs.append(B)
        if pre_ref is not None:
            assert torch.equal(kw["pre"], pre_ref)
    assert outs[0].kb == (64 if act == 2 else 256 if act == 4 else 128)
    used = M * cols * 2 + 2 * M * (cols // outs[0].kb)  # int16s written: the pairs, then the inverse scales
    assert torch.equal(outs[0].data[:used], outs[1].data[:used])
    x, hmax = blocks_ref(outs[0], device)
    c = C.double()
    bmax = c.abs().reshape(M, cols // outs[0].kb, outs[0].kb).amax(dim=2)
    tol = 2.0 ** -22 * c.abs() + 2.0 ** -25 * bmax.repeat_interleave(outs[0].kb, dim=1)
    assert ((x - c).abs() <= tol).all(), (x - c).abs().max().item()
    live = bmax.cpu().numpy() > 0
    assert (hmax[live] >= 2.0 ** 14).all() and (hmax[live] <= 2.0 ** 15).all()
    assert (hmax[~live] == 0).all()


@pytest.mark.parametrize("act", [2, 4, 1])
def test_block_pairs_product(act, device):
    # pet_linear_fused_blocks: the product of block pairs (as the producer of
    # the test above made them) with split weights, against the fp64 product of
    # the decoded blocks and weights, per element within the fp32
    # accumulation's bound and the dropped lo * lo terms (below);
    # rows independent of M (a slice alone gives the same bits); epilogue with
    # bias and a residual from C itself
    M, N0, K0 = 3000, 512, 256
    g = torch.Generator(device=device).manual_seed(60 + act)
    A = torch.randn(M, K0, device=device, generator=g) * torch.logspace(-2, 2, M, device=device)[:, None]
    W0 = L.SplitWeights(torch.randn(N0, K0, device=device, generator=g) / K0 ** 0.5)
    width = 2 * N0 if act == 4 else N0
    kw = dict(bias=torch.randn(width, device=device, generator=g))
    if act >= 3:
        kw["cin"] = torch.randn(M, width, device=device, generator=g)
    cols = N0 // 2 if act == 2 else width
    scratch = torch.empty(M * (K0 * 4 + 4) // 4 + 64, device=device)
    B = L.BlockPairs(M, cols, device)
    L.fused_to_blocks(A, W0, B, **kw, act=act, scratch=scratch)
    N = 384
    print(f"[gpu] block pairs product, K={cols} (kb {B.kb}), N={N}", flush=True)
    W = L.SplitWeights(torch.randn(N, cols, device=device, generator=g) / cols ** 0.5)
    b = torch.randn(N, device=device, generator=g)
    res = torch.randn(M, N, device=device, generator=g)
    C = res.clone()
    L.fused(B, W, C, bias=b, cin=C, beta=1.0)
    torch.cuda.synchronize()
    x, _ = blocks_ref(B, device)
    w = W_ref(W, device)
    ref = x @ w.T + b.double() + res.double()
    bound = x.abs() @ w.abs().T + res.double().abs()
    # fp32 accumulation: one rounding a 32-wide K step (the matrix instruction
    # sums its 32 products), one a block's addition into the total, a few in
    # the epilogue; the dropped lo * lo terms 2^-22 of |a| |w|
    rel = (cols // 32 + cols // B.kb + 4) * 2.0 ** -24 + 2.0 ** -22
    assert ((C.double() - ref).abs() <= rel * bound + 1e-30).all(), ((C.double() - ref).abs() / bound).max().item()
    # a slice of the rows alone: block pairs of those rows only
    B2 = L.BlockPairs(1000, cols, device)
    L.fused_to_blocks(A[1000:2000].contiguous(), W0, B2, **{k: (v[1000:2000].contiguous() if v.dim() == 2 else v)
                                                           for k, v in kw.items()}, act=act, scratch=scratch)
    C2 = res[1000:2000].clone()
    L.fused(B2, W, C2, bias=b, cin=C2, beta=1.0)
    assert torch.equal(C2, C[1000:2000])


@pytest.mark.parametrize("K", [256, 512, 1024, 2048])
def test_norm_pair_rows_same_bits(K, device):
    # pet_norm_rows_pairs: the norm's output made directly as pair rows is the
    # same bits as pet_norm_rows then pet_linear_pair_rows, for RMSNorm and
    # LayerNorm, rows 10^-3 .. 10^3 apart, and a product from either the same
    from pet_kokkos_amd import attention as A_
    M = 777
    print(f"[gpu] norm as pair rows, K={K}", flush=True)
    g = torch.Generator(device=device).manual_seed(K)
    X = torch.randn(M, K, device=device, generator=g) * torch.logspace(-3, 3, M, device=device)[:, None]
    w = torch.rand(K, device=device, generator=g) + 0.5
    for bias in (None, torch.randn(K, device=device, generator=g)):
        Y = torch.empty(M, K, device=device)
        _lib.check(_lib.load().pet_norm_rows(M, K, Y.data_ptr(), K, X.data_ptr(), K, w.data_ptr(),
                                             None if bias is None else bias.data_ptr(),
                                             torch.cuda.current_stream().cuda_stream), "pet_norm_rows")
        ref = L.PairRows(Y)
        got = L.norm_pair_rows(X, w, bias)
        used = M * K * 2 + 2 * M
        assert torch.equal(ref.data[:used], got.data[:used]), bias is None


def test_flop_tally(device):
    """pet_gemm_flop_tally: each launch adds 2 M N K to its instruction class
    (the short-K kernel's, the fp32 fused kernel's), and reset zeroes them."""
    _lib.gemm_flop_tally(reset=True)
    M, N, K = 1000, 96, 64
    g = torch.Generator(device=device).manual_seed(70)
    A = torch.randn(M, K, device=device, generator=g)
    W = torch.randn(N, K, device=device, generator=g)
    C = torch.empty(M, N, device=device)
    linear_fused(A, W, C, split="smallk")
    linear_fused(A, W, C, split=False)
    torch.cuda.synchronize()
    t = _lib.gemm_flop_tally(reset=True)
    assert t["shortk"] == 2.0 * M * N * K and t["fp32"] == 2.0 * M * N * K
    assert t["split"] == 0.0 and t["pair"] == 0.0
    assert all(v == 0.0 for v in _lib.gemm_flop_tally().values())
