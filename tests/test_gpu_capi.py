"""GPU parity through the raw C ABI (ctypes, device pointers, hipStream_t):
the boundary a non-torch host binds. Buffers are torch allocations; every
result is checked against the CPU oracle."""

import numpy as np
import pytest
import torch

from nanotitan_amd import capi
from nanotitan_amd.capi import call, current_stream, dtype_code, ptr
from oracle import moe_oracle as O
from tests.test_gpu_dispatch import bits

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return capi.load()


def ws(nbytes):
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device="cuda")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_capi_dispatch_combine_roundtrip(lib, dtype):
    d = O.make_inputs(3, T=2048, with_weights=False)
    c = d["cfg"]
    gates, idx, _ = O.route(d["logits"], c.k)
    X = d["X"][:, :64].to(dtype).contiguous()
    T, dd, k, E = X.shape[0], X.shape[1], c.k, c.E
    A = T * k
    counts, offsets, p = O.dispatch(X, gates, idx, E)
    Xg, wg, ig = X.cuda(), gates.cuda(), idx.cuda()
    g_counts = torch.empty(E, dtype=torch.int32, device="cuda")
    g_off = torch.empty(E + 1, dtype=torch.int32, device="cuda")
    g_px = torch.empty(A, dd, dtype=dtype, device="cuda")
    g_tid = torch.empty(A, dtype=torch.int32, device="cuda")
    g_ex = torch.empty(A, dtype=torch.int32, device="cuda")
    g_pw = torch.empty(A, dtype=torch.float32, device="cuda")
    g_inv = torch.empty(T, k, dtype=torch.int32, device="cuda")
    nb = lib.nt_dispatch_workspace_bytes(T, k, E, dd, dtype_code(dtype))
    w = ws(nb)
    s = current_stream()
    call("nt_dispatch", dtype_code(dtype), ptr(Xg), ptr(wg), ptr(ig), T, k, dd, E, ptr(g_counts),
         ptr(g_off), ptr(g_px), ptr(g_tid), ptr(g_ex), ptr(g_pw), ptr(g_inv), ptr(w), nb, s)
    torch.cuda.synchronize()
    assert np.array_equal(g_counts.cpu().numpy(), counts)
    assert np.array_equal(g_off.cpu().numpy(), offsets)
    assert np.array_equal(g_tid.cpu().numpy(), p.token_id)
    assert torch.equal(bits(g_px), bits(p.packed_X))

    # combine through token ids (CSR path) and through the inverse map
    out = torch.empty(T, dd, dtype=torch.float32, device="cuda")
    cb = lib.nt_combine_workspace_bytes(A, T)
    w2 = ws(cb)
    call("nt_combine_tokens", dtype_code(dtype), ptr(g_px), ptr(g_tid), ptr(g_pw), A, T, dd,
         ptr(out), ptr(w2), cb, s)
    out2 = torch.empty_like(out)
    call("nt_combine_inv", dtype_code(dtype), ptr(g_px), ptr(g_inv), ptr(g_pw), T, k, dd,
         capi.NT_F32, ptr(out2), s)
    torch.cuda.synchronize()
    want = O.combine_tokens(p.packed_X, p.token_id, p.packed_w, T)
    assert torch.equal(bits(out), bits(torch.from_numpy(want)))
    assert torch.equal(bits(out2), bits(out))


def test_capi_route_count_then_dispatch_counted(lib):
    """nt_route_topk_count writes the per-block counts at the start of the
    dispatch workspace; nt_dispatch_counted then matches the oracle."""
    d = O.make_inputs(2, T=3000, with_weights=False)
    c = d["cfg"]
    X = d["X"][:, :512].contiguous()
    T, dd, k, E = X.shape[0], X.shape[1], c.k, c.E
    A = T * k
    want_g, want_i, _ = O.route(d["logits"], k)
    counts, offsets, p = O.dispatch(X, want_g, want_i, E)
    code = dtype_code(X.dtype)
    TB = lib.nt_dispatch_block_tokens(T, k, dd, code)
    nbytes = lib.nt_dispatch_workspace_bytes(T, k, E, dd, code)
    w = ws(nbytes)
    lg, Xg = d["logits"].cuda(), X.cuda()
    gates = torch.empty(T, k, device="cuda")
    topk = torch.empty(T, k, dtype=torch.int32, device="cuda")
    s = current_stream()
    call("nt_route_topk_count", ptr(lg), T, E, k, ptr(gates), ptr(topk), None, TB, ptr(w), s)
    g_counts = torch.empty(E, dtype=torch.int32, device="cuda")
    g_off = torch.empty(E + 1, dtype=torch.int32, device="cuda")
    g_px = torch.empty(A, dd, dtype=X.dtype, device="cuda")
    g_tid = torch.empty(A, dtype=torch.int32, device="cuda")
    g_ex = torch.empty(A, dtype=torch.int32, device="cuda")
    g_pw = torch.empty(A, dtype=torch.float32, device="cuda")
    g_inv = torch.empty(T, k, dtype=torch.int32, device="cuda")
    call("nt_dispatch_counted", code, ptr(Xg), ptr(gates), ptr(topk), T, k, dd, E, ptr(g_counts),
         ptr(g_off), ptr(g_px), ptr(g_tid), ptr(g_ex), ptr(g_pw), ptr(g_inv), ptr(w), nbytes, s)
    torch.cuda.synchronize()
    assert np.array_equal(topk.cpu().numpy(), want_i.numpy())
    assert np.array_equal(g_counts.cpu().numpy(), counts)
    assert np.array_equal(g_off.cpu().numpy(), offsets)
    assert np.array_equal(g_tid.cpu().numpy(), p.token_id)
    assert np.array_equal(g_inv.cpu().numpy(), p.inv)
    assert torch.equal(bits(g_px), bits(p.packed_X))


def test_capi_workspace_too_small(lib):
    T, k, E, dd = 64, 2, 8, 16
    z = torch.zeros(1, device="cuda")
    code = lib.nt_dispatch(capi.NT_F32, ptr(z), ptr(z), ptr(z), T, k, dd, E, ptr(z), ptr(z),
                           ptr(z), ptr(z), ptr(z), ptr(z), None, ptr(z), 4, current_stream())
    assert code == capi.NT_ERR_WORKSPACE


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_capi_grouped_gemm_three_ops(lib, dtype):
    counts = [40, 0, 300, 7]
    offsets = torch.tensor(np.concatenate([[0], np.cumsum(counts)]), dtype=torch.int32)
    A, K, N, E = int(offsets[-1]), 64, 256, len(counts)
    g = torch.Generator().manual_seed(5)
    X = torch.randn(A, K, generator=g).to(dtype)
    W = (torch.randn(E, K, N, generator=g) / 8).to(dtype)
    G = torch.randn(A, N, generator=g).to(dtype)
    Xg, Wg, og, Gg = X.cuda(), W.cuda(), offsets.cuda(), G.cuda()
    out = torch.empty(A, N, dtype=dtype, device="cuda")
    dX = torch.empty(A, K, dtype=dtype, device="cuda")
    dW = torch.empty(E, K, N, dtype=dtype, device="cuda")
    nb = lib.nt_grouped_gemm_workspace_bytes(dtype_code(dtype), E, A, K, N)
    w = ws(nb)
    s = current_stream()
    dc = dtype_code(dtype)
    call("nt_grouped_gemm", dc, ptr(Xg), ptr(og), ptr(Wg), E, A, K, N, ptr(out), ptr(w), nb, s)
    call("nt_grouped_gemm_dx", dc, ptr(Wg), ptr(og), ptr(Gg), E, A, K, N, ptr(dX), ptr(w), nb, s)
    call("nt_grouped_gemm_dw", dc, ptr(Xg), ptr(og), ptr(Gg), E, A, K, N, ptr(dW), ptr(w), nb, s)
    torch.cuda.synchronize()
    tol = dict(rtol=2e-2, atol=2e-2)
    torch.testing.assert_close(out.cpu().double(), O.grouped_gemm(X, offsets, W).to(dtype).double(),
                               **tol)
    torch.testing.assert_close(dX.cpu().double(),
                               O.grouped_gemm_dx(W, offsets, G).to(dtype).double(), **tol)
    torch.testing.assert_close(dW.cpu().double(),
                               O.grouped_gemm_dw(X, offsets, G).to(dtype).double(), rtol=2e-2,
                               atol=0.4)
    assert not dW[1].cpu().any()


@pytest.mark.parametrize("fill", ["zeros", "ones", "random", "reuse"])
def test_capi_paired_dw_dx_any_workspace_contents(lib, fill):
    """The paired dW + dX call claims its dX tiles from counters in the
    caller's workspace that carry a per-launch tag: whatever the workspace
    held before (zeros, all-ones bytes, random bytes, the same workspace's
    previous call), the results are the separate calls' bits."""
    E, K, N, A = 8, 512, 2048, 8192
    g = torch.Generator().manual_seed(41)
    X = torch.randn(A, K, generator=g).to(torch.bfloat16).cuda()
    W = (torch.randn(E, K, N, generator=g) * 0.05).to(torch.bfloat16).cuda()
    G = torch.randn(A, N, generator=g).to(torch.bfloat16).cuda()
    off = torch.tensor([i * A // E for i in range(E + 1)], dtype=torch.int32, device="cuda")
    dt = dtype_code(torch.bfloat16)
    nb = lib.nt_grouped_gemm_workspace_bytes(dt, E, A, K, N)
    s = current_stream()
    dW_ref = torch.empty(E, K, N, dtype=torch.bfloat16, device="cuda")
    dX_ref = torch.empty(A, K, dtype=torch.bfloat16, device="cuda")
    w0 = torch.zeros(max(nb, 1), dtype=torch.uint8, device="cuda")
    call("nt_grouped_gemm_dw", dt, ptr(X), ptr(off), ptr(G), E, A, K, N, ptr(dW_ref), ptr(w0), nb, s)
    call("nt_grouped_gemm_dx", dt, ptr(W), ptr(off), ptr(G), E, A, K, N, ptr(dX_ref), None, 0, s)
    w = ws(nb)
    if fill == "zeros":
        w.zero_()
    elif fill == "ones":
        w.fill_(0xFF)
    else:
        w.copy_(torch.randint(0, 256, (w.numel(),), generator=g, dtype=torch.uint8).cuda())
    runs = 2 if fill == "reuse" else 1
    for _ in range(runs):
        dW = torch.full((E, K, N), float("nan"), dtype=torch.bfloat16, device="cuda")
        dX = torch.full((A, K), float("nan"), dtype=torch.bfloat16, device="cuda")
        call("nt_grouped_gemm_dw_dx", dt, ptr(X), ptr(W), ptr(off), ptr(G), E, A, K, N, ptr(dW),
             ptr(dX), ptr(w), nb, s)
        torch.cuda.synchronize()
        assert torch.equal(bits(dW), bits(dW_ref))
        assert torch.equal(bits(dX), bits(dX_ref))
