"""GPU: the GELU fused into the grouped GEMM epilogues, and the GELU expert FFN.

``grouped_gemm_gelu`` must return gelu(h) and gelu'(h) of the h that
``grouped_gemm_kernel`` returns; ``bwd_grouped_gemm_dX_gelu`` must return
(dOut @ W^T, rounded) * gelu'(h) (the stored, rounded gelu'(h)).
The FFN autograd Function is checked against the oracle's float64 grouped
GEMMs and erf GELU, rounded to the dtype wherever the FFN stores a tensor,
and against the unfused GPU composition (grouped_gemm_fn +
torch.nn.functional.gelu + grouped_gemm_fn).
Cases cover the MFMA path (both tile shapes), the generic path (d not a
multiple of 8, fp32) and an empty expert.
"""

import pytest
import torch

from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu

TOL = {
    torch.float32: dict(rtol=1e-4, atol=1e-5),
    torch.float16: dict(rtol=1e-2, atol=1e-2),
    torch.bfloat16: dict(rtol=2e-2, atol=2e-2),
}


def _offsets(counts, device="cuda"):
    c = torch.tensor(counts, dtype=torch.int64)
    off = torch.zeros(len(counts) + 1, dtype=torch.int32)
    off[1:] = torch.cumsum(c, 0).to(torch.int32)
    return off.to(device)


def _case(seed, counts, d, f, dtype):
    g = torch.Generator().manual_seed(seed)
    A = sum(counts)
    E = len(counts)
    X = torch.randn(A, d, generator=g).to(dtype)
    W_up = (torch.randn(E, d, f, generator=g) * 0.05).to(dtype)
    W_down = (torch.randn(E, f, d, generator=g) * 0.05).to(dtype)
    dY = torch.randn(A, d, generator=g).to(dtype)
    return X, W_up, W_down, dY, _offsets(counts)


def _gelu_grad(x):
    x = x.double()
    return 0.5 * (1 + torch.erf(x / 2 ** 0.5)) + x * torch.exp(-0.5 * x * x) / (2 * torch.pi) ** 0.5


CASES = [
    # (counts, d, f, dtype): MFMA 128x128 tiles with an empty expert
    ([300, 0, 517, 96], 64, 128, torch.bfloat16),
    ([300, 0, 517, 96], 64, 128, torch.float16),
    # generic path: d not a multiple of 8; fp32
    ([5, 11, 0, 7], 7, 24, torch.bfloat16),
    ([40, 0, 33], 32, 48, torch.float32),
]


@pytest.mark.parametrize("counts,d,f,dtype", CASES)
def test_gemm_gelu_forward(ext, counts, d, f, dtype):
    X, W_up, _, _, off = _case(11, counts, d, f, dtype)
    Xc, Wc = X.cuda(), W_up.cuda()
    act, act_grad = ext.grouped_gemm_gelu(Xc, off, Wc)
    h = ext.grouped_gemm_kernel(Xc, off, Wc)
    torch.cuda.synchronize()
    A = sum(counts)
    h = h[:A].cpu()
    torch.testing.assert_close(h.double(), O.grouped_gemm(X, off.cpu(), W_up), **TOL[dtype])
    # gelu and gelu' of the rounded h, each rounded once.
    torch.testing.assert_close(act[:A].cpu(), O.gelu(h.double()).to(dtype), **TOL[dtype])
    torch.testing.assert_close(act_grad[:A].cpu(), _gelu_grad(h).to(dtype), **TOL[dtype])


@pytest.mark.parametrize("counts,d,f,dtype", CASES)
def test_dx_gelu(ext, counts, d, f, dtype):
    X, W_up, W_down, dY, off = _case(12, counts, d, f, dtype)
    _, g = ext.grouped_gemm_gelu(X.cuda(), off, W_up.cuda())
    dH = ext.bwd_grouped_gemm_dX_gelu(W_down.cuda(), off, dY.cuda(), g)
    dA = ext.bwd_grouped_gemm_dX_kernel(W_down.cuda(), off, dY.cuda())
    torch.cuda.synchronize()
    A = sum(counts)
    # The unfused composition: rounded dA times the stored gelu'(h), rounded once.
    ref = (dA[:A].cpu().double() * g[:A].cpu().double()).to(dtype)
    torch.testing.assert_close(dH[:A].cpu(), ref, **TOL[dtype])
    ref64 = O.grouped_gemm_dx(W_down, off.cpu(), dY) * g[:A].cpu().double()
    torch.testing.assert_close(dH[:A].cpu().double(), ref64, **TOL[dtype])


@pytest.mark.parametrize("counts,d,f,dtype", CASES)
def test_gelu_ffn_autograd_vs_oracle(ext, counts, d, f, dtype):
    """Forward and every gradient against the oracle's float64 grouped GEMMs,
    rounded to the dtype at the points the FFN rounds (h, gelu(h), gelu'(h),
    y, dA, dH and the three gradients)."""
    from nanotitan_amd.moe_ops import grouped_gelu_ffn_fn

    X, W_up, W_down, dY, off = _case(13, counts, d, f, dtype)
    x = X.cuda().requires_grad_(True)
    wu = W_up.cuda().requires_grad_(True)
    wd = W_down.cuda().requires_grad_(True)
    y = grouped_gelu_ffn_fn(x, wu, wd, off)
    y.backward(dY.cuda())
    torch.cuda.synchronize()

    offc = off.cpu()
    r = lambda t: t.to(dtype)  # noqa: E731  (round a float64 result to the dtype)
    h = r(O.grouped_gemm(X, offc, W_up))
    act = r(O.gelu(h.double()))
    y_ref = r(O.grouped_gemm(act, offc, W_down))
    dA = r(O.grouped_gemm_dx(W_down, offc, dY))
    dH = r(dA.double() * r(_gelu_grad(h)).double())
    dwd = r(O.grouped_gemm_dw(act, offc, dY))
    dx = r(O.grouped_gemm_dx(W_up, offc, dH))
    dwu = r(O.grouped_gemm_dw(X, offc, dH))
    A = sum(counts)
    tol = TOL[dtype]
    torch.testing.assert_close(y[:A].detach().cpu(), y_ref, **tol)
    torch.testing.assert_close(x.grad.cpu(), dx, **tol)
    torch.testing.assert_close(wu.grad.cpu(), dwu, **tol)
    torch.testing.assert_close(wd.grad.cpu(), dwd, **tol)


@pytest.mark.parametrize("A,d,f,E", [(4096, 256, 512, 4), (32768, 256, 3072, 8)])
def test_gelu_ffn_matches_unfused_gpu(ext, A, d, f, E):
    """Both MFMA tile shapes (the larger case takes the 256x256 tiles): the fused
    FFN against the unfused GPU composition, same kernels for the GEMMs."""
    from nanotitan_amd.moe_ops import grouped_gelu_ffn_fn, grouped_gemm_fn

    counts = [A // E] * E
    counts[0] += A - sum(counts)
    X, W_up, W_down, dY, off = _case(14, counts, d, f, torch.bfloat16)
    ins = [t.cuda() for t in (X, W_up, W_down)]
    a = [t.clone().requires_grad_(True) for t in ins]
    b = [t.clone().requires_grad_(True) for t in ins]
    y_f = grouped_gelu_ffn_fn(a[0], a[1], a[2], off)
    y_f.backward(dY.cuda())
    h = grouped_gemm_fn(b[0], b[1], off)
    y_u = grouped_gemm_fn(torch.nn.functional.gelu(h.float()).to(h.dtype), b[2], off)
    y_u.backward(dY.cuda())
    torch.cuda.synchronize()
    # The fused path rounds gelu'(h) to bf16 before the multiply; over sums
    # of thousands of rows that moves entries near zero by more than a fixed
    # atol, so the absolute tolerance scales with the tensor's RMS.
    def close(u, v):
        rms = v.float().pow(2).mean().sqrt().item()
        torch.testing.assert_close(u, v, rtol=2e-2, atol=2e-2 * rms)
        rel = (u.float() - v.float()).norm() / v.float().norm()
        assert rel < 1e-2, f"relative L2 difference {rel:.3g}"

    close(y_f, y_u)
    for p, q in zip(a, b):
        close(p.grad, q.grad)


def test_gemm_gelu_table_edges(ext):
    """The 256-row tiles read gelu / gelu' from a table covering
    2^-16 <= |h| < 8 and compute the rest: h spans about +-40 here, with exact
    zeros (all-zero rows) and tiny values (rows scaled by 2^-20). In-range
    values must equal the double-precision result rounded once; out-of-range
    values must meet the bf16 tolerance."""
    E, d, f = 4, 64, 1024
    counts = [8192] * E
    A = sum(counts)
    g_ = torch.Generator().manual_seed(21)
    X = torch.randn(A, d, generator=g_)
    X[::7] *= 12.0                  # |h| up to ~40
    X[3::11] = 0.0                  # h == 0 exactly
    X[5::13] *= 2.0**-20            # |h| < 2^-16
    X = X.to(torch.bfloat16)
    W = (torch.randn(E, d, f, generator=g_) * 0.4).to(torch.bfloat16)
    off = _offsets(counts)
    act, act_grad = ext.grouped_gemm_gelu(X.cuda(), off, W.cuda())
    h = ext.grouped_gemm_kernel(X.cuda(), off, W.cuda())
    torch.cuda.synchronize()
    h = h.cpu().double()
    # double precision with an accurate lower tail (x * ndtr(x); 1 + erf
    # cancels below about -5 even in double)
    from scipy.special import ndtr

    hn = h.numpy()
    cdf = ndtr(hn)
    pdf = torch.from_numpy(hn).pow(2).mul(-0.5).exp().numpy() / (2 * torch.pi) ** 0.5
    want = torch.from_numpy(hn * cdf).to(torch.bfloat16)
    want_g = torch.from_numpy(cdf + hn * pdf).to(torch.bfloat16)
    a, ag = act.cpu(), act_grad.cpu()
    inr = (h.abs() >= 2.0**-16) & (h.abs() < 8.0)
    assert inr.float().mean() > 0.5 and (~inr).sum() > 1000 and (h == 0).sum() > 1000
    assert torch.equal(a[inr], want[inr])
    assert torch.equal(ag[inr], want_g[inr])
    torch.testing.assert_close(a.double(), want.double(), **TOL[torch.bfloat16])
    torch.testing.assert_close(ag.double(), want_g.double(), **TOL[torch.bfloat16])
    assert torch.equal(a[h == 0], torch.zeros_like(a[h == 0]))
    assert torch.all(ag[h == 0] == 0.5)
