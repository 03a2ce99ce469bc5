"""GPU parity: expert-grouped GEMM forward, dX and dW vs the float64 oracle.

Tolerances are the reference's (tests/test_grouped_gemm.py:35-39): fp32
rtol 1e-4 / atol 5e-4, bf16 and fp16 2e-2 (scaled by the reduction length
where the values grow with it).
"""

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]
TOL = {
    torch.float32: dict(rtol=1e-4, atol=5e-4),
    torch.float64: dict(rtol=1e-9, atol=1e-9),
    torch.float16: dict(rtol=2e-2, atol=2e-2),
    torch.bfloat16: dict(rtol=2e-2, atol=2e-2),
}


def check(got, want, dtype, scale=1.0):
    """Compare against the fp64 oracle rounded to dtype (the best a dtype output can do)."""
    want_c = want.to(dtype).double()
    tol = dict(TOL[dtype])
    tol["atol"] = tol["atol"] * scale
    torch.testing.assert_close(got.cpu().double(), want_c, **tol)


def run_all(ext, X, W, offsets, G):
    Xg, Wg, og, Gg = X.cuda(), W.cuda(), offsets.cuda(), G.cuda()
    out = ext.grouped_gemm_kernel(Xg, og, Wg)
    dX = ext.bwd_grouped_gemm_dX_kernel(Wg, og, Gg)
    dW = ext.bwd_grouped_gemm_dW_kernel(Xg, og, Gg)
    torch.cuda.synchronize()
    return out, dX, dW


@pytest.mark.parametrize("dtype", DTYPES + [torch.float64])
@pytest.mark.parametrize("shape", [(4, 2, 4, 4), (128, 4, 16, 32), (8192, 3, 1, 8192)])
def test_small_smoke_shapes(ext, dtype, shape):
    """reference tests/test_grouped_gemm.py:51-82 shapes (even splits i*A//E)."""
    A, E, K, N = shape
    g = torch.Generator().manual_seed(A + K)
    X = torch.randn(A, K, generator=g).to(dtype)
    W = torch.randn(E, K, N, generator=g).to(dtype)
    offsets = torch.tensor([i * A // E for i in range(E + 1)], dtype=torch.int32)
    G = torch.randn(A, N, generator=g).to(dtype)
    out, dX, dW = run_all(ext, X, W, offsets, G)
    check(out, O.grouped_gemm(X, offsets, W), dtype, scale=max(1, K) ** 0.5)
    check(dX, O.grouped_gemm_dx(W, offsets, G), dtype, scale=max(1, N) ** 0.5)
    check(dW, O.grouped_gemm_dw(X, offsets, G), dtype, scale=max(1, A // E) ** 0.5)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("K,N", [(2048, 8192), (8192, 2048)])
def test_moe_projection_counts_3_1_4(ext, dtype, K, N):
    """reference tests/test_grouped_gemm.py:85-145: counts [3,1,4], offsets [0,3,4,8]."""
    g = torch.Generator().manual_seed(K)
    offsets = torch.tensor([0, 3, 4, 8], dtype=torch.int32)
    X = torch.randn(8, K, generator=g).to(dtype)
    W = (torch.randn(3, K, N, generator=g) / K ** 0.5).to(dtype)
    G = torch.randn(8, N, generator=g).to(dtype)
    out, dX, dW = run_all(ext, X, W, offsets, G)
    check(out, O.grouped_gemm(X, offsets, W), dtype)
    check(dX, O.grouped_gemm_dx(W, offsets, G), dtype, scale=(N / K) ** 0.5)
    check(dW, O.grouped_gemm_dw(X, offsets, G), dtype, scale=2.0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("counts", [[0, 5, 0, 130, 1, 0], [257, 0, 0, 0], [0, 0, 0],
                                    [1, 1, 1, 1, 1, 1, 1, 1], [700, 3, 129, 128, 127]])
def test_empty_and_skewed_experts(ext, dtype, counts):
    """Empty experts, M_e = 1, tile-edge rows; dW of an empty expert is exactly zero."""
    K, N = 96, 136
    offsets = torch.tensor(np.concatenate([[0], np.cumsum(counts)]), dtype=torch.int32)
    A = int(offsets[-1]) + 5  # rows past offsets[E] are never read or written
    g = torch.Generator().manual_seed(sum(counts) + len(counts))
    X = torch.randn(A, K, generator=g).to(dtype)
    W = (torch.randn(len(counts), K, N, generator=g) / K ** 0.5).to(dtype)
    G = torch.randn(A, N, generator=g).to(dtype)
    out, dX, dW = run_all(ext, X, W, offsets, G)
    used = int(offsets[-1])
    check(out[:used], O.grouped_gemm(X, offsets, W)[:used], dtype)
    check(dX[:used], O.grouped_gemm_dx(W, offsets, G)[:used], dtype, scale=2.0)
    check(dW, O.grouped_gemm_dw(X, offsets, G), dtype, scale=max(counts + [1]) ** 0.5)
    for e, c in enumerate(counts):
        if c == 0:
            assert not dW[e].any()


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("K,N", [(2048, 8192), (8192, 2048)])
def test_autograd_wrapper_noncontiguous_grad(ext, dtype, K, N):
    """reference tests/test_grouped_gemm.py:148-208, including the transposed d_out."""
    from nanotitan_amd.moe_ops import grouped_gemm_fn

    torch.manual_seed(0)
    offsets = torch.tensor([0, 3, 4, 8], dtype=torch.int32, device="cuda")
    X = torch.randn(8, K, dtype=dtype, device="cuda", requires_grad=True)
    W = (torch.randn(3, K, N, dtype=dtype, device="cuda") / K ** 0.5).requires_grad_(True)
    out = grouped_gemm_fn(X, W, offsets)
    d_out = torch.randn(N, 8, dtype=dtype, device="cuda").T
    out.backward(d_out)
    Xc, Wc, Gc = X.detach().cpu(), W.detach().cpu(), d_out.detach().cpu()
    off = offsets.cpu()
    check(out.detach(), O.grouped_gemm(Xc, off, Wc), dtype)
    check(X.grad, O.grouped_gemm_dx(Wc, off, Gc), dtype, scale=(N / K) ** 0.5)
    check(W.grad, O.grouped_gemm_dw(Xc, off, Gc), dtype, scale=2.0)


@pytest.mark.parametrize("cfg_id,T", [(2, 4096), (3, 4096)])
def test_config_shapes_routed(ext, cfg_id, T):
    """Real routed segment sizes at the configs' widths (C3: Zipf skew, tiny experts)."""
    d = O.make_inputs(cfg_id, T=T)
    c = d["cfg"]
    gates, idx, _ = O.route(d["logits"], c.k)
    counts = O.count_experts(idx, None, c.E)
    offsets = torch.from_numpy(O.offsets_from_counts(counts))
    A = T * c.k
    g = torch.Generator().manual_seed(cfg_id)
    X = torch.randn(A, c.d, generator=g).to(c.dtype)
    W = d["weights"]["up"]
    G = torch.randn(A, c.f, generator=g).to(c.dtype)
    out, dX, dW = run_all(ext, X, W, offsets, G)
    check(out, O.grouped_gemm(X, offsets, W), c.dtype)
    check(dX, O.grouped_gemm_dx(W, offsets, G), c.dtype)
    check(dW, O.grouped_gemm_dw(X, offsets, G), c.dtype, scale=max(int(counts.max()), 1) ** 0.5)


def test_gemm_is_deterministic(ext):
    g = torch.Generator().manual_seed(3)
    offsets = torch.tensor([0, 1000, 1000, 3000], dtype=torch.int32).cuda()
    X = torch.randn(3000, 256, generator=g).to(torch.bfloat16).cuda()
    G = torch.randn(3000, 512, generator=g).to(torch.bfloat16).cuda()
    a = ext.bwd_grouped_gemm_dW_kernel(X, offsets, G)
    b = ext.bwd_grouped_gemm_dW_kernel(X, offsets, G)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("counts", [[30000, 7, 0, 4000, 3000, 993, 0, 2000],
                                    [0, 0, 45000, 0, 5000]])
def test_dw_split_reduction_for_skewed_experts(ext, dtype, counts):
    """A head expert far above the mean is reduced in chunks (fp32 partials in
    the workspace, summed in chunk order by a second kernel); every expert,
    split or not, empty or not, matches the oracle, and the result is
    bit-identical run to run and equal to the unsplit C-ABI result within
    one summation-order rounding."""
    from nanotitan_amd import capi

    g = torch.Generator().manual_seed(21)
    A, K, N = sum(counts), 64, 128
    X = torch.randn(A, K, generator=g).to(dtype)
    G = torch.randn(A, N, generator=g).to(dtype)
    offsets = torch.zeros(len(counts) + 1, dtype=torch.int32)
    offsets[1:] = torch.cumsum(torch.tensor(counts), 0).to(torch.int32)
    E = len(counts)
    lib = capi.load()
    code = capi.NT_BF16 if dtype == torch.bfloat16 else capi.NT_F16
    assert lib.nt_grouped_gemm_workspace_bytes(code, E, A, K, N) > 0  # splitting is possible
    Xg, Gg, og = X.cuda(), G.cuda(), offsets.cuda()
    a = ext.bwd_grouped_gemm_dW_kernel(Xg, og, Gg)
    b = ext.bwd_grouped_gemm_dW_kernel(Xg, og, Gg)
    # Same GEMM without a workspace: every expert in one chunk.
    c = torch.empty_like(a)
    st = lib.nt_grouped_gemm_dw(code, Xg.data_ptr(), og.data_ptr(), Gg.data_ptr(), E, A, K, N,
                                c.data_ptr(), None, 0, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert st == 0
    assert torch.equal(a, b)
    check(a, O.grouped_gemm_dw(X, offsets, G), dtype, scale=max(counts) ** 0.5)
    check(c, O.grouped_gemm_dw(X, offsets, G), dtype, scale=max(counts) ** 0.5)
    for e, n in enumerate(counts):
        if n == 0:
            assert not a[e].any()


def _ceil(a, b):
    return -(-a // b)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_dw_skewed_split_threshold(ext, dtype):
    """C3 widths (K=512, N=256, 64 experts), 128x128 dW tiles. The dW launch
    splits an expert only when it is longer than a split threshold (about
    1.25 workgroup shares of rows), into chunks of about half a share. The
    counts are picked from the device's CU count so that one head expert is
    split into many chunks, one expert is longer than a chunk but below the
    threshold (so it stays one whole tile), and the rest are small or empty.
    Every expert matches the oracle and the unsplit C-ABI call."""
    from nanotitan_amd import capi

    cus = torch.cuda.get_device_properties(0).multi_processor_count
    E, K, N = 64, 512, 256
    small = [0 if e % 16 == 5 else 600 for e in range(E - 2)]
    A0 = 20000 + 1100 + sum(small)
    W = _ceil(A0 * _ceil(K, 128) * _ceil(N, 128), 2 * cus)
    R = _ceil(max(_ceil(W, 2), 1024), 64) * 64
    thr = max(_ceil(_ceil(5 * W, 4), 64) * 64, R)
    mid = (R + thr) // 2 if thr > R + 1 else R  # longer than a chunk, not split
    counts = [20000, mid] + small
    assert counts[0] > thr and (thr == R or R < mid <= thr)
    g = torch.Generator().manual_seed(23)
    A = sum(counts)
    X = torch.randn(A, K, generator=g).to(dtype)
    G = torch.randn(A, N, generator=g).to(dtype)
    offsets = torch.zeros(E + 1, dtype=torch.int32)
    offsets[1:] = torch.cumsum(torch.tensor(counts), 0).to(torch.int32)
    lib = capi.load()
    code = capi.NT_BF16 if dtype == torch.bfloat16 else capi.NT_F16
    Xg, Gg, og = X.cuda(), G.cuda(), offsets.cuda()
    a = ext.bwd_grouped_gemm_dW_kernel(Xg, og, Gg)
    c = torch.empty_like(a)
    st = lib.nt_grouped_gemm_dw(code, Xg.data_ptr(), og.data_ptr(), Gg.data_ptr(), E, A, K, N,
                                c.data_ptr(), None, 0, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert st == 0
    want = O.grouped_gemm_dw(X, offsets, G)
    check(a, want, dtype, scale=max(counts) ** 0.5)
    check(c, want, dtype, scale=max(counts) ** 0.5)
    # Unsplit experts are reduced in the same order either way.
    for e in range(1, E):
        assert torch.equal(a[e], c[e]), e


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("K,N", [(1032, 1000), (1000, 1032)])
def test_split_duty_tiles_ragged(ext, dtype, K, N):
    """Shapes large enough for 256x256 tiles with split load/store duties
    (at least 1.5 tiles per CU, reduction >= 1024): uneven experts (tiles
    cross expert ends), output columns and the reduction not multiples of
    the tile, for forward, dX and the two-part dX."""
    counts = [6000, 0, 9777, 3, 13220]
    A = sum(counts)
    # the launcher's rule: ceil(A/256) * ceil(out_cols/256) >= 1.5 tiles per CU
    tiles = -(-A // 256) * -(-min(K, N) // 256)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert 2 * tiles >= 3 * cus, "shape too small to reach the 256x256 split path"
    g = torch.Generator().manual_seed(K * 7 + N)
    offsets = torch.zeros(len(counts) + 1, dtype=torch.int32)
    offsets[1:] = torch.cumsum(torch.tensor(counts), 0).to(torch.int32)
    E = len(counts)
    X = torch.randn(A, K, generator=g).to(dtype)
    W = (torch.randn(E, K, N, generator=g) / K ** 0.5).to(dtype)
    W2 = (torch.randn(E, K, N, generator=g) / K ** 0.5).to(dtype)
    G = torch.randn(A, N, generator=g).to(dtype)
    G2 = torch.randn(A, N, generator=g).to(dtype)
    Xg, Wg, W2g, og, Gg, G2g = X.cuda(), W.cuda(), W2.cuda(), offsets.cuda(), G.cuda(), G2.cuda()
    out = ext.grouped_gemm_kernel(Xg, og, Wg)
    dX = ext.bwd_grouped_gemm_dX_kernel(Wg, og, Gg)
    dX2 = ext.bwd_grouped_gemm_dX2(Wg, W2g, og, Gg, G2g)
    torch.cuda.synchronize()
    check(out, O.grouped_gemm(X, offsets, W), dtype)
    want_dx = O.grouped_gemm_dx(W, offsets, G)
    check(dX, want_dx, dtype, scale=(N / K) ** 0.5)
    check(dX2, want_dx + O.grouped_gemm_dx(W2, offsets, G2), dtype, scale=(2 * N / K) ** 0.5)
    # deterministic, and rows past the experts' end untouched by neighbours
    again = ext.grouped_gemm_kernel(Xg, og, Wg)
    assert torch.equal(out.view(torch.int16), again.view(torch.int16))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("counts,K,N", [([7680] * 8, 2048, 512), ([7680] * 8, 512, 2048),
                                        ([20000, 0, 3, 9000, 5000], 1024, 256),
                                        ([12000, 11000, 40, 9000], 520, 264),
                                        ([5, 0, 17], 64, 128)])
def test_paired_dw_dx_matches_separate_calls(ext, dtype, counts, K, N):
    """bwd_grouped_gemm_dW_dX[_gelu]: the dW runs beside the dX in one
    launch when it has few 256x256 tiles (the first four cases), else after
    it. The third splits its head expert's reduction, the fourth three
    experts, on tiles cut by K and N; the paired launch sums their partial
    slabs itself, in the order of the separate reduce pass. Outputs equal
    the separate calls bit for bit, and work queued next on the current
    stream sees them complete."""
    g = torch.Generator().manual_seed(K + N + len(counts))
    A, E = sum(counts), len(counts)
    offsets = torch.zeros(E + 1, dtype=torch.int32)
    offsets[1:] = torch.cumsum(torch.tensor(counts), 0).to(torch.int32)
    dev = "cuda"
    X = torch.randn(A, K, generator=g).to(dtype).to(dev)
    W = (torch.randn(E, K, N, generator=g) / K ** 0.5).to(dtype).to(dev)
    dOut = torch.randn(A, N, generator=g).to(dtype).to(dev)
    act_grad = torch.rand(A, K, generator=g).to(dtype).to(dev)
    og = offsets.to(dev)
    dW_ref = ext.bwd_grouped_gemm_dW_kernel(X, og, dOut)
    dX_ref = ext.bwd_grouped_gemm_dX_kernel(W, og, dOut)
    dH_ref = ext.bwd_grouped_gemm_dX_gelu(W, og, dOut, act_grad)
    for _ in range(2):  # the second call reuses the caching allocator's workspace
        dW, dX = ext.bwd_grouped_gemm_dW_dX(X, W, og, dOut)
        same = torch.equal(dW.view(torch.int16), dW_ref.view(torch.int16)) and \
            torch.equal(dX.view(torch.int16), dX_ref.view(torch.int16))
        assert same
        dW2, dH = ext.bwd_grouped_gemm_dW_dX_gelu(X, W, og, dOut, act_grad)
        assert torch.equal(dW2.view(torch.int16), dW_ref.view(torch.int16))
        assert torch.equal(dH.view(torch.int16), dH_ref.view(torch.int16))
    if A <= 4096:  # the separate calls themselves against the oracle
        check(dW_ref, O.grouped_gemm_dw(X.cpu(), offsets, dOut.cpu()), dtype,
              scale=max(counts) ** 0.5)
        check(dX_ref, O.grouped_gemm_dx(W.cpu(), offsets, dOut.cpu()), dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("counts,K,N", [([7680] * 8, 2048, 512), ([7680] * 8, 512, 2048),
                                        ([9000, 0, 1, 4000], 256, 1024), ([5, 0, 17], 64, 128)])
def test_paired_swiglu_backward_matches_separate_calls(ext, dtype, counts, K, N):
    """bwd_grouped_gemm_dW_dX_swiglu (dW of the output projection beside the
    SwiGLU-backward dX) and bwd_grouped_gemm_dW_dX2 (dW of the gate
    projection beside the two-part dX) equal the separate calls bit for bit."""
    g = torch.Generator().manual_seed(K * 3 + N + len(counts))
    A, E = sum(counts), len(counts)
    offsets = torch.zeros(E + 1, dtype=torch.int32)
    offsets[1:] = torch.cumsum(torch.tensor(counts), 0).to(torch.int32)
    og = offsets.cuda()

    def rnd(*shape, scale=1.0):
        return (torch.randn(*shape, generator=g) * scale).to(dtype).cuda()

    bits = lambda t: t.view(torch.int16)  # noqa: E731
    # output projection: hidden/gate/value [A,K], W_out [E,K,N], dy [A,N]
    h, gate, value = rnd(A, K), rnd(A, K), rnd(A, K)
    W_out, dy = rnd(E, K, N, scale=K ** -0.5), rnd(A, N)
    dW_ref = ext.bwd_grouped_gemm_dW_kernel(h, og, dy)
    dg_ref, dv_ref = ext.bwd_grouped_gemm_dX_swiglu(W_out, og, dy, gate, value)
    for _ in range(2):
        dW, dg, dv = ext.bwd_grouped_gemm_dW_dX_swiglu(h, W_out, og, dy, gate, value)
        assert torch.equal(bits(dW), bits(dW_ref))
        assert torch.equal(bits(dg), bits(dg_ref)) and torch.equal(bits(dv), bits(dv_ref))
    # input projections: X [A,K], W_gate / W_val [E,K,N], dgate / dvalue [A,N]
    X, W1, W2 = rnd(A, K), rnd(E, K, N, scale=K ** -0.5), rnd(E, K, N, scale=K ** -0.5)
    d1, d2 = rnd(A, N), rnd(A, N)
    dW1_ref = ext.bwd_grouped_gemm_dW_kernel(X, og, d1)
    dX_ref = ext.bwd_grouped_gemm_dX2(W1, W2, og, d1, d2)
    for _ in range(2):
        dW1, dX = ext.bwd_grouped_gemm_dW_dX2(X, W1, W2, og, d1, d2)
        assert torch.equal(bits(dW1), bits(dW1_ref)) and torch.equal(bits(dX), bits(dX_ref))


@pytest.mark.parametrize("dtype,counts,K,N", [
    (torch.float32, [700, 0, 300], 96, 160),      # generic FMA path: no pairing
    (torch.bfloat16, [700, 0, 300], 40, 24),      # K, N not multiples of 64 / 8
    (torch.bfloat16, [0, 0, 0], 64, 128),         # no rows at all
    (torch.bfloat16, [500] * 20, 256, 256),       # more experts than the pairing limit
])
def test_paired_calls_edge_cases(ext, dtype, counts, K, N):
    """Paired ops fall back to the separate GEMMs where they cannot pair and
    still match them (and the oracle within tolerance)."""
    g = torch.Generator().manual_seed(K + N)
    A, E = sum(counts), len(counts)
    offsets = torch.zeros(E + 1, dtype=torch.int32)
    offsets[1:] = torch.cumsum(torch.tensor(counts), 0).to(torch.int32)
    X = torch.randn(A, K, generator=g).to(dtype)
    W = (torch.randn(E, K, N, generator=g) / K ** 0.5).to(dtype)
    G = torch.randn(A, N, generator=g).to(dtype)
    Xg, Wg, og, Gg = X.cuda(), W.cuda(), offsets.cuda(), G.cuda()
    dW, dX = ext.bwd_grouped_gemm_dW_dX(Xg, Wg, og, Gg)
    assert torch.equal(dW, ext.bwd_grouped_gemm_dW_kernel(Xg, og, Gg))
    assert torch.equal(dX, ext.bwd_grouped_gemm_dX_kernel(Wg, og, Gg))
    check(dW, O.grouped_gemm_dw(X, offsets, G), dtype, scale=max(max(counts), 1) ** 0.5)
    if A:
        check(dX, O.grouped_gemm_dx(W, offsets, G), dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16])
def test_dw_non_monotone_offsets_stay_in_the_workspace(ext, dtype):
    """Offsets [0, A, 0, A, ...]: each expert's range is clamped on its own, so
    experts 0, 2, 4, 6 each span all A rows and 1, 3, 5, 7 none. At these sizes
    the dW split would cut every full expert into chunks (64 in all), more than
    the workspace's 32 partial slabs; the kernels then run every expert
    unsplit. dW[e] = X^T dOut over the expert's clamped range, for the plain
    and the paired (dW beside dX) calls alike."""
    A, K, N, E = 16384, 256, 1024, 8
    g = torch.Generator().manual_seed(77)
    X = torch.randn(A, K, generator=g).to(dtype)
    G = torch.randn(A, N, generator=g).to(dtype)
    W = (torch.randn(E, K, N, generator=g) / 16).to(dtype)
    offsets = torch.tensor([0 if e % 2 == 0 else A for e in range(E + 1)], dtype=torch.int32)
    Xg, Gg, Wg, og = X.cuda(), G.cuda(), W.cuda(), offsets.cuda()
    dW = ext.bwd_grouped_gemm_dW_kernel(Xg, og, Gg)
    dW2, _dX = ext.bwd_grouped_gemm_dW_dX(Xg, Wg, og, Gg)
    torch.cuda.synchronize()
    full = (X.float().t() @ G.float()).double()
    for e in range(E):
        if e % 2 == 0:
            check(dW[e], full, dtype, scale=A ** 0.5)
        else:
            assert not dW[e].cpu().any(), e
    assert torch.equal(dW.cpu().view(torch.int16), dW2.cpu().view(torch.int16))


@pytest.mark.parametrize("K,N", [(4, 4), (36, 20), (100, 132), (260, 4), (512, 2048)])
@pytest.mark.parametrize("counts", [[0, 5, 0, 130, 1, 0], [257, 0, 300], [1, 1, 1, 1]])
def test_f32_mfma_tails_and_empty_experts(ext, K, N, counts):
    """fp32 on the MFMA kernel (K, N multiples of 4): reduction tails of 4,
    ragged column tiles, empty experts (dW exactly zero), M_e = 1, and the
    two-part dX of the SwiGLU backward against the sum of two oracle dX."""
    dtype = torch.float32
    offsets = torch.tensor(np.concatenate([[0], np.cumsum(counts)]), dtype=torch.int32)
    A = int(offsets[-1]) + 3
    g = torch.Generator().manual_seed(K * 7 + N + len(counts))
    X = torch.randn(A, K, generator=g)
    W = torch.randn(len(counts), K, N, generator=g) / K ** 0.5
    W2 = torch.randn(len(counts), K, N, generator=g) / K ** 0.5
    G = torch.randn(A, N, generator=g)
    G2 = torch.randn(A, N, generator=g)
    out, dX, dW = run_all(ext, X, W, offsets, G)
    dX2 = ext.bwd_grouped_gemm_dX2(W.cuda(), W2.cuda(), offsets.cuda(), G.cuda(), G2.cuda())
    torch.cuda.synchronize()
    used = int(offsets[-1])
    check(out[:used], O.grouped_gemm(X, offsets, W)[:used], dtype, scale=max(1, K) ** 0.5)
    check(dX[:used], O.grouped_gemm_dx(W, offsets, G)[:used], dtype, scale=max(1, N) ** 0.5)
    want2 = O.grouped_gemm_dx(W, offsets, G) + O.grouped_gemm_dx(W2, offsets, G2)
    check(dX2[:used], want2[:used], dtype, scale=(2 * max(1, N)) ** 0.5)
    check(dW, O.grouped_gemm_dw(X, offsets, G), dtype, scale=max(counts + [1]) ** 0.5)
    for e, c in enumerate(counts):
        if c == 0:
            assert not dW[e].any()


@pytest.mark.parametrize("counts,K,N", [([7680] * 8, 2048, 512), ([20000, 0, 3, 9000, 5000], 1024, 256)])
def test_paired_dw_dx_under_graph_replay(ext, counts, K, N):
    """A paired dW + dX call captured into a HIP graph: every replay equals
    the eager call on the inputs of that replay, bit for bit. The graph
    replays the launch with the tag it was captured with, so the call clears
    its claim (and, for the split head expert of the second case, arrival)
    counters with a kernel captured just before it; without that, the
    second replay would find the first one's final counts. Eager work and
    synchronisations run between the replays."""
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(K + len(counts))
    A, E = sum(counts), len(counts)
    offsets = torch.zeros(E + 1, dtype=torch.int32)
    offsets[1:] = torch.cumsum(torch.tensor(counts), 0).to(torch.int32)
    og = offsets.cuda()
    X = torch.empty(A, K, dtype=dtype, device="cuda")
    W = torch.empty(E, K, N, dtype=dtype, device="cuda")
    dOut = torch.empty(A, N, dtype=dtype, device="cuda")

    def fill(seed):
        gg = torch.Generator().manual_seed(seed)
        X.copy_(torch.randn(A, K, generator=gg).to(dtype))
        W.copy_((torch.randn(E, K, N, generator=gg) / K ** 0.5).to(dtype))
        dOut.copy_(torch.randn(A, N, generator=gg).to(dtype))

    fill(0)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm the allocator outside the capture
        ext.bwd_grouped_gemm_dW_dX(X, W, og, dOut)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        dW_g, dX_g = ext.bwd_grouped_gemm_dW_dX(X, W, og, dOut)
    for seed in (1, 2, 3, 4):
        fill(seed)
        dW_e = ext.bwd_grouped_gemm_dW_kernel(X, og, dOut)  # eager, separate calls
        dX_e = ext.bwd_grouped_gemm_dX_kernel(W, og, dOut)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        print(f"[graph] replay with inputs of seed {seed}", flush=True)
        assert torch.equal(dW_g.view(torch.int16), dW_e.view(torch.int16)), seed
        assert torch.equal(dX_g.view(torch.int16), dX_e.view(torch.int16)), seed
