"""GPU: the reference's SwiGLU expert FFN on the fused grouped GEMMs.

``grouped_gemm_swiglu`` computes the gate and value GEMMs of each output
tile in one kernel and writes gate, value and hidden = silu(gate) * value;
``bwd_grouped_gemm_dX_swiglu`` writes dgate and dvalue from dhidden =
dOut @ W_out^T and the stored gate / value; ``bwd_grouped_gemm_dX2`` sums the
two input-gradient products in one reduction. Checked against the separate
GPU grouped GEMMs with torch's own silu and autograd in between (the
reference's _forward_cuda dataflow), and against the oracle's float64
grouped GEMMs rounded where the FFN rounds. Cases: both MFMA tile paths,
the generic path (d or f not a multiple of 8, fp32), f not a multiple of
64 (the two-part dX on its generic path), and an empty expert.
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


def _case(seed, counts, d, f, dtype, wstd=0.08):
    g = torch.Generator().manual_seed(seed)
    A, E = sum(counts), len(counts)
    X = torch.randn(A, d, generator=g).to(dtype)
    Wg = (torch.randn(E, d, f, generator=g) * wstd).to(dtype)
    Wv = (torch.randn(E, d, f, generator=g) * wstd).to(dtype)
    Wo = (torch.randn(E, f, d, generator=g) * wstd).to(dtype)
    dY = torch.randn(A, d, generator=g).to(dtype)
    return X, Wg, Wv, Wo, dY, _offsets(counts)


CASES = [
    # (counts, d, f, dtype)
    ([700, 0, 517, 96], 64, 256, torch.bfloat16),   # MFMA, empty expert, partial tiles
    ([700, 0, 517, 96], 64, 256, torch.float16),
    ([300, 40, 9], 128, 200, torch.bfloat16),       # f % 64 != 0: two-part dX generic
    ([5, 11, 0, 7], 7, 24, torch.bfloat16),         # generic path everywhere
    ([40, 0, 33], 32, 48, torch.float32),
]


def _bits_close(a, b, dtype, frac=2e-3):
    """Equal to within one rounding on a small fraction of elements (the
    exponential inside silu is not the same routine as torch's), and within
    the dtype tolerance everywhere."""
    torch.testing.assert_close(a.float(), b.float(), **TOL[dtype])
    if dtype != torch.float32:
        diff = (a != b).float().mean().item()
        assert diff <= frac, f"{diff:.4f} of elements differ"


@pytest.mark.parametrize("counts,d,f,dtype", CASES)
def test_swiglu_forward(ext, counts, d, f, dtype):
    X, Wg, Wv, _, _, off = _case(31, counts, d, f, dtype)
    Xc, Wgc, Wvc = X.cuda(), Wg.cuda(), Wv.cuda()
    h, gt, vl = ext.grouped_gemm_swiglu(Xc, off, Wgc, Wvc)
    g_ref = ext.grouped_gemm_kernel(Xc, off, Wgc)
    v_ref = ext.grouped_gemm_kernel(Xc, off, Wvc)
    torch.cuda.synchronize()
    A = sum(counts)
    # gate and value: the same accumulation as the separate GEMMs, bit for bit
    assert torch.equal(gt[:A], g_ref[:A]) and torch.equal(vl[:A], v_ref[:A])
    h_ref = torch.nn.functional.silu(g_ref[:A]) * v_ref[:A]
    _bits_close(h[:A], h_ref, dtype)
    # against the oracle's float64 GEMMs
    offc = off.cpu()
    torch.testing.assert_close(gt[:A].cpu().double(), O.grouped_gemm(X, offc, Wg), **TOL[dtype])
    torch.testing.assert_close(vl[:A].cpu().double(), O.grouped_gemm(X, offc, Wv), **TOL[dtype])


@pytest.mark.parametrize("counts,d,f,dtype", CASES)
def test_dx_swiglu_matches_autograd(ext, counts, d, f, dtype):
    X, Wg, Wv, Wo, dY, off = _case(32, counts, d, f, dtype)
    _, gt, vl = ext.grouped_gemm_swiglu(X.cuda(), off, Wg.cuda(), Wv.cuda())
    dg, dv = ext.bwd_grouped_gemm_dX_swiglu(Wo.cuda(), off, dY.cuda(), gt, vl)
    dH = ext.bwd_grouped_gemm_dX_kernel(Wo.cuda(), off, dY.cuda())
    A = sum(counts)
    g_ = gt[:A].clone().requires_grad_(True)
    v_ = vl[:A].clone().requires_grad_(True)
    (torch.nn.functional.silu(g_) * v_).backward(dH[:A])
    torch.cuda.synchronize()
    _bits_close(dv[:A], v_.grad, dtype)
    _bits_close(dg[:A], g_.grad, dtype)


@pytest.mark.parametrize("counts,d,f,dtype", CASES)
def test_dx2_is_sum_of_products(ext, counts, d, f, dtype):
    g = torch.Generator().manual_seed(33)
    A, E = sum(counts), len(counts)
    W1 = (torch.randn(E, d, f, generator=g) * 0.1).to(dtype)
    W2 = (torch.randn(E, d, f, generator=g) * 0.1).to(dtype)
    d1 = torch.randn(A, f, generator=g).to(dtype)
    d2 = torch.randn(A, f, generator=g).to(dtype)
    off = _offsets(counts)
    dX = ext.bwd_grouped_gemm_dX2(W1.cuda(), W2.cuda(), off, d1.cuda(), d2.cuda())
    torch.cuda.synchronize()
    offc = off.cpu()
    want = O.grouped_gemm_dx(W1, offc, d1) + O.grouped_gemm_dx(W2, offc, d2)
    torch.testing.assert_close(dX[:A].cpu().double(), want, **TOL[dtype])
    if dtype == torch.float32:
        return  # fp32 sums: accumulation error, not output rounding, dominates
    # 16-bit outputs: one rounding of the sum is no worse than rounding each product
    two = (ext.bwd_grouped_gemm_dX_kernel(W1.cuda(), off, d1.cuda()).float()
           + ext.bwd_grouped_gemm_dX_kernel(W2.cuda(), off, d2.cuda()).float())
    err_one = (dX[:A].cpu().double() - want).abs().sum()
    err_two = (two[:A].cpu().double() - want).abs().sum()
    assert err_one <= err_two * 1.01 + 1e-9


@pytest.mark.parametrize("counts,d,f,dtype", CASES)
def test_swiglu_ffn_autograd_vs_unfused(ext, counts, d, f, dtype):
    """The fused FFN against the reference dataflow on the GPU: three
    grouped_gemm_fn with torch's silu * value between them."""
    from nanotitan_amd.moe_ops import grouped_gemm_fn, swiglu_ffn_fn

    X, Wg, Wv, Wo, dY, off = _case(34, counts, d, f, dtype)
    ins = [t.cuda() for t in (X, Wg, Wv, Wo)]
    a = [t.clone().requires_grad_(True) for t in ins]
    b = [t.clone().requires_grad_(True) for t in ins]
    y_f = swiglu_ffn_fn(a[0], a[1], a[2], a[3], off)
    y_f.backward(dY.cuda())
    gate = grouped_gemm_fn(b[0], b[1], off)
    value = grouped_gemm_fn(b[0], b[2], off)
    y_u = grouped_gemm_fn(torch.nn.functional.silu(gate) * value, b[3], off)
    y_u.backward(dY.cuda())
    torch.cuda.synchronize()
    A = sum(counts)

    def close(u, v):
        rms = v.float().pow(2).mean().sqrt().item() + 1e-30
        tol = TOL[dtype]
        torch.testing.assert_close(u.float(), v.float(), rtol=tol["rtol"],
                                   atol=max(tol["atol"] * rms, 1e-6))
        rel = (u.float() - v.float()).norm() / (v.float().norm() + 1e-30)
        assert rel < (1e-2 if dtype != torch.float32 else 1e-5), f"relative L2 {rel:.3g}"

    close(y_f[:A], y_u[:A])
    close(a[0].grad[:A], b[0].grad[:A])
    for p, q in zip(a[1:], b[1:]):
        close(p.grad, q.grad)


def test_swiglu_ffn_vs_oracle_float64(ext):
    """Whole FFN and every gradient against float64 restatements rounded at
    the points the FFN rounds (gate, value, silu, hidden, y, dhidden, ...)."""
    from nanotitan_amd.moe_ops import swiglu_ffn_fn

    counts, d, f, dtype = [600, 0, 300, 124], 64, 128, torch.bfloat16
    X, Wg, Wv, Wo, dY, off = _case(35, counts, d, f, dtype)
    a = [t.cuda().requires_grad_(True) for t in (X, Wg, Wv, Wo)]
    y = swiglu_ffn_fn(a[0], a[1], a[2], a[3], off)
    y.backward(dY.cuda())
    torch.cuda.synchronize()
    offc = off.cpu()
    r = lambda t: t.to(dtype)  # noqa: E731
    gt = r(O.grouped_gemm(X, offc, Wg))
    vl = r(O.grouped_gemm(X, offc, Wv))
    s = r(torch.nn.functional.silu(gt.double()))
    h = r(s.double() * vl.double())
    y_ref = r(O.grouped_gemm(h, offc, Wo))
    dH = r(O.grouped_gemm_dx(Wo, offc, dY))
    dv = r(dH.double() * s.double())
    ds = r(dH.double() * vl.double())
    sg = torch.sigmoid(gt.double())
    dg = r(ds.double() * sg * (1 + gt.double() * (1 - sg)))
    dX = r(O.grouped_gemm_dx(Wg, offc, dg) + O.grouped_gemm_dx(Wv, offc, dv))
    A = sum(counts)
    tol = TOL[dtype]
    torch.testing.assert_close(y[:A].detach().cpu(), y_ref, **tol)
    torch.testing.assert_close(a[0].grad[:A].cpu(), dX, **tol)
    torch.testing.assert_close(a[1].grad.cpu(), r(O.grouped_gemm_dw(X, offc, dg)), **tol)
    torch.testing.assert_close(a[2].grad.cpu(), r(O.grouped_gemm_dw(X, offc, dv)), **tol)
    torch.testing.assert_close(a[3].grad.cpu(), r(O.grouped_gemm_dw(h, offc, dY)), **tol)


def test_swiglu_large_tiles_deterministic(ext):
    """C2-sized experts (many 256-row tiles, persistent workgroups): two runs
    bit-identical, gate / value equal to the separate GEMMs."""
    counts, d, f, dtype = [7680] * 8, 512, 1024, torch.bfloat16
    X, Wg, Wv, Wo, dY, off = _case(36, counts, d, f, dtype, wstd=0.02)
    Xc, Wgc, Wvc, Woc, dYc = (t.cuda() for t in (X, Wg, Wv, Wo, dY))
    r1 = ext.grouped_gemm_swiglu(Xc, off, Wgc, Wvc)
    r2 = ext.grouped_gemm_swiglu(Xc, off, Wgc, Wvc)
    assert all(torch.equal(p, q) for p, q in zip(r1, r2))
    assert torch.equal(r1[1], ext.grouped_gemm_kernel(Xc, off, Wgc))
    assert torch.equal(r1[2], ext.grouped_gemm_kernel(Xc, off, Wvc))
    _bits_close(r1[0], torch.nn.functional.silu(r1[1]) * r1[2], dtype)
    b1 = ext.bwd_grouped_gemm_dX_swiglu(Woc, off, dYc, r1[1], r1[2])
    b2 = ext.bwd_grouped_gemm_dX_swiglu(Woc, off, dYc, r1[1], r1[2])
    assert all(torch.equal(p, q) for p, q in zip(b1, b2))
    x1 = ext.bwd_grouped_gemm_dX2(Wgc, Wvc, off, b1[0], b1[1])
    x2 = ext.bwd_grouped_gemm_dX2(Wgc, Wvc, off, b1[0], b1[1])
    assert torch.equal(x1, x2)
    torch.cuda.synchronize()
