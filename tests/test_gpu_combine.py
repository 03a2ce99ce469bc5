"""GPU parity: combine forward/backward and pack backward vs the CPU oracle.

Combine forward is bit-exact against the oracle's ordered fp32 sum; dy and
pack-backward dX (fp32 ordered sum, one cast) are bit-exact; the gate
gradient dw is a dot product compared within rel 1e-5 (fp32 accumulation,
fixed reduction order on the GPU).
"""

import json

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from tests.conftest import GOLDEN
from tests.test_gpu_dispatch import bits

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16, torch.float64]
DW_TOL = dict(rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("case", ["top1", "top2"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_combine_reference_kat(ext, case, dtype):
    """reference tests/test_combine.py:12-90."""
    kat = json.loads((GOLDEN / "combine_kat.json").read_text())[case]
    y = torch.tensor(kat["expert_outputs"], dtype=dtype, device="cuda")
    tid = torch.tensor(kat["packed_tokenId"], dtype=torch.int32, device="cuda")
    w = torch.tensor(kat["packed_topk_weights"], dtype=torch.float32, device="cuda")
    out = ext.combine_tokens_kernel(y, tid, w, kat["num_tokens"], 2)
    assert out.dtype == torch.float32
    want = O.combine_tokens(y.cpu(), tid.cpu(), w.cpu(), kat["num_tokens"])
    assert torch.equal(bits(out), bits(torch.from_numpy(want)))
    tol = {torch.float32: 1e-5, torch.float16: 1e-2, torch.bfloat16: 2e-2}[dtype]
    torch.testing.assert_close(out.cpu().to(dtype).float(),
                               torch.tensor(kat["expected"]).to(dtype).float(), rtol=tol, atol=tol)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("T,A,d", [(3, 6, 8), (5, 11, 7), (100, 1000, 64), (64, 64 * 300, 24),
                                   (1, 1, 1), (50, 0, 16)])
def test_combine_generic_bit_exact(ext, dtype, T, A, d):
    """Arbitrary token-id multiplicity (reference tests/test_combine_bwd.py:39-43 style)."""
    g = torch.Generator().manual_seed(T + A + d)
    y = torch.randn(A, d, generator=g).to(dtype)
    w = torch.randn(A, generator=g)
    tid = torch.randint(0, T, (A,), generator=g, dtype=torch.int32)
    out = ext.combine_tokens_kernel(y.cuda(), tid.cuda(), w.cuda(), T, d)
    want = O.combine_tokens(y, tid, w, T)
    assert torch.equal(bits(out), bits(torch.from_numpy(want)))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("T,A,d", [(3, 6, 8), (5, 11, 7), (200, 1600, 40), (4, 0, 8)])
def test_combine_backward_generic(ext, dtype, T, A, d):
    g = torch.Generator().manual_seed(A + 5)
    y = torch.randn(A, d, generator=g).to(dtype)
    w = torch.randn(A, generator=g)
    tid = torch.tensor([i % T for i in range(A)], dtype=torch.int32)
    dY = torch.randn(T, d, generator=g)
    dy, dw = ext.combine_kernel_backward(y.cuda(), tid.cuda(), w.cuda(), dY.cuda(), d)
    want_dy, want_dw = O.combine_backward(y, tid, w, dY, out_dtype=dtype)
    assert torch.equal(bits(dy), bits(want_dy))
    np.testing.assert_allclose(dw.cpu().numpy(), want_dw, **DW_TOL)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("T,k,E,d", [(3, 2, 3, 8), (5, 3, 3, 7), (500, 8, 64, 96), (77, 1, 4, 5)])
def test_pack_backward_generic_and_inv(ext, dtype, T, k, E, d):
    g = torch.Generator().manual_seed(T * k)
    X = torch.randn(T, d, generator=g).to(dtype)
    w = torch.rand(T, k, generator=g)
    # distinct experts per token, like torch.topk
    topk = torch.argsort(torch.rand(T, E, generator=g), dim=1)[:, :k].to(torch.int32)
    counts, offsets, p = O.dispatch(X, w, topk, E)
    A = T * k
    dpX = torch.randn(A, d, generator=g).to(dtype)
    dpw = torch.randn(A, generator=g)
    want_dX, want_dw = O.pack_backward(dpX, dpw, p.token_id, p.expert, topk, out_dtype=dtype)
    dX, dw = ext.pack_kernel_backward(dpX.cuda(), dpw.cuda(), torch.from_numpy(p.token_id).cuda(),
                                      torch.from_numpy(p.expert).cuda(), topk.cuda())
    assert torch.equal(bits(dX), bits(want_dX))
    assert torch.equal(bits(dw), bits(torch.from_numpy(want_dw)))
    dX2, dw2 = ext.pack_backward_inv(dpX.cuda(), dpw.cuda(), torch.from_numpy(p.inv).cuda())
    assert torch.equal(bits(dX2), bits(want_dX))
    assert torch.equal(bits(dw2), bits(torch.from_numpy(want_dw)))


def test_pack_backward_first_match_rule(ext):
    """Duplicate experts in a row: the reference's first-match rule (backward_pack_kernel.cu:35-42)."""
    topk = torch.tensor([[2, 2], [0, 1]], dtype=torch.int32)
    tid = torch.tensor([0, 0, 1, 1], dtype=torch.int32)
    ex = torch.tensor([2, 2, 0, 1], dtype=torch.int32)
    dpw = torch.tensor([1.0, 2.0, 3.0, 4.0])
    dX, dw = ext.pack_kernel_backward(torch.zeros(4, 3, device="cuda"), dpw.cuda(), tid.cuda(),
                                      ex.cuda(), topk.cuda())
    assert dw.tolist() == [[3.0, 0.0], [3.0, 4.0]]


@pytest.mark.parametrize("cfg_id,T", [(2, 30720), (3, 8192), (5, 4096)])
def test_combine_inv_matches_generic_and_oracle(ext, cfg_id, T):
    """Layer path (inverse map) == reference surface (token ids) == oracle, bit for bit."""
    d = O.make_inputs(cfg_id, T=T, with_weights=False)
    c = d["cfg"]
    gates, idx, _ = O.route(d["logits"], c.k)
    dd = 128 if cfg_id == 5 else c.d
    X = d["X"][:, :dd].contiguous()
    counts, offsets, p = O.dispatch(X, gates, idx, c.E)
    g = torch.Generator().manual_seed(cfg_id)
    y = torch.randn(T * c.k, dd, generator=g).to(c.dtype)
    tid = torch.from_numpy(p.token_id)
    pw = torch.from_numpy(p.packed_w)
    inv = torch.from_numpy(p.inv)
    want = O.combine_tokens(y, tid, pw, T)
    a = ext.combine_tokens_kernel(y.cuda(), tid.cuda(), pw.cuda(), T, dd)
    b = ext.combine_inv(y.cuda(), inv.cuda(), pw.cuda(), torch.float32)
    c16 = ext.combine_inv(y.cuda(), inv.cuda(), pw.cuda(), c.dtype)
    assert torch.equal(bits(a), bits(torch.from_numpy(want)))
    assert torch.equal(bits(b), bits(a))
    assert torch.equal(bits(c16), bits(a.to(c.dtype)))
    # backward: inverse-map form == generic form, bit for bit; dw within tolerance of oracle
    dY = d["dY"][:, :dd].float()
    dy1, dw1 = ext.combine_kernel_backward(y.cuda(), tid.cuda(), pw.cuda(), dY.cuda(), dd)
    dy2, dw2 = ext.combine_backward_inv(y.cuda(), inv.cuda(), pw.cuda(), dY.cuda())
    dy3, dw3 = ext.combine_backward_inv(y.cuda(), inv.cuda(), pw.cuda(), dY.to(c.dtype).cuda())
    assert torch.equal(bits(dy1), bits(dy2)) and torch.equal(bits(dw1), bits(dw2))
    want_dy, want_dw = O.combine_backward(y, tid, pw, dY, out_dtype=c.dtype)
    assert torch.equal(bits(dy1), bits(want_dy))
    np.testing.assert_allclose(dw1.cpu().numpy(), want_dw, **DW_TOL)
    want_dy3, want_dw3 = O.combine_backward(y, tid, pw, dY.to(c.dtype).float(), out_dtype=c.dtype)
    assert torch.equal(bits(dy3), bits(want_dy3))
    np.testing.assert_allclose(dw3.cpu().numpy(), want_dw3, **DW_TOL)


def test_combine_is_deterministic(ext):
    g = torch.Generator().manual_seed(9)
    y = torch.randn(8192, 256, generator=g).to(torch.bfloat16).cuda()
    tid = torch.randint(0, 1000, (8192,), generator=g, dtype=torch.int32).cuda()
    w = torch.rand(8192, generator=g).cuda()
    a = ext.combine_tokens_kernel(y, tid, w, 1000, 256)
    b = ext.combine_tokens_kernel(y, tid, w, 1000, 256)
    assert torch.equal(bits(a), bits(b))
    dY = torch.randn(1000, 256, generator=g).cuda()
    r1 = ext.combine_kernel_backward(y, tid, w, dY, 256)
    r2 = ext.combine_kernel_backward(y, tid, w, dY, 256)
    assert torch.equal(bits(r1[1]), bits(r2[1]))


def test_combine_rejects_non_fp32_grad(ext):
    y = torch.randn(4, 2, device="cuda")
    tid = torch.zeros(4, dtype=torch.int32, device="cuda")
    w = torch.ones(4, device="cuda")
    with pytest.raises(RuntimeError, match="float32"):
        ext.combine_kernel_backward(y, tid, w, torch.zeros(1, 2, device="cuda",
                                                           dtype=torch.float16), 2)


def _check_inverse_map_kernels(ext, T, k, d, dtype, seed, empty_tokens=0):
    """combine_inv / combine_backward_inv / pack_backward_inv on an inverse
    map with dropped (-1) and out-of-range slots, slots in random packed
    order, and the first `empty_tokens` tokens left with no valid slot:
    bit-equal to the oracle's token-id forms (dw within DW_TOL)."""
    A = T * k
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(A, generator=g).to(torch.int32)
    inv = perm.view(T, k).clone()
    drop = torch.rand(T, k, generator=g) < 0.07
    inv[drop] = -1
    inv[torch.rand(T, k, generator=g) < 0.02] = A + 5  # out of range: skipped
    inv[:empty_tokens] = -1
    token_id = torch.full((A,), -1, dtype=torch.int32)
    slot = torch.zeros(A, dtype=torch.int32)
    for t in range(T):
        for j in range(k):
            p = int(inv[t, j])
            if 0 <= p < A:
                token_id[p] = t
                slot[p] = j
    y = torch.randn(A, d, generator=g).to(dtype)
    w = torch.randn(A, generator=g)
    out = ext.combine_inv(y.cuda(), inv.cuda(), w.cuda(), torch.float32)
    want = O.combine_tokens(y, token_id, w, T)
    assert torch.equal(bits(out), bits(torch.from_numpy(want)))

    dY = torch.randn(T, d, generator=g)
    dy, dw = ext.combine_backward_inv(y.cuda(), inv.cuda(), w.cuda(), dY.cuda())
    want_dy, want_dw = O.combine_backward(y, token_id, w, dY, out_dtype=dtype)
    valid = (token_id >= 0).numpy()
    assert torch.equal(bits(dy.cpu()[valid]), bits(want_dy[valid]))
    # the token-id kernel does the same fp32 arithmetic per packed row
    dyg, dwg = ext.combine_kernel_backward(y.cuda(), token_id.cuda(), w.cuda(), dY.cuda(), d)
    assert torch.equal(bits(dy.cpu()[valid]), bits(dyg.cpu()[valid]))
    assert torch.equal(bits(dw.cpu()[valid]), bits(dwg.cpu()[valid]))
    # against the oracle's float64 sum: an fp32 dot product summed d/64
    # deep per lane, then over a 64-lane tree, errs by at most
    # (d/64 + 6) * 2^-24 * sum|dY * y| (< 1e-5 * sum|dY * y| for d <= 8192)
    tv = token_id[torch.from_numpy(valid)].long()
    mag = (dY[tv].double() * y[torch.from_numpy(valid)].double()).abs().sum(1).numpy()
    err = np.abs(dw.cpu().numpy()[valid].astype(np.float64) - want_dw[valid].astype(np.float64))
    assert (err <= 1e-5 * mag + 1e-30).all(), float((err / mag).max())

    dpX = torch.randn(A, d, generator=g).to(dtype)
    dpw = torch.randn(A, generator=g)
    topk = torch.arange(k, dtype=torch.int32).repeat(T, 1)  # slot j <-> "expert" j
    want_dX, want_dw2 = O.pack_backward(dpX, dpw, token_id, slot, topk, out_dtype=dtype)
    dX, dw2 = ext.pack_backward_inv(dpX.cuda(), dpw.cuda(), inv.cuda())
    assert torch.equal(bits(dX), bits(want_dX))
    assert torch.equal(bits(dw2), bits(torch.from_numpy(want_dw2)))


@pytest.mark.parametrize("k", [1, 2, 5, 8, 12])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_inverse_map_kernels_with_dropped_slots(ext, k, dtype):
    """Short rows (one vector per lane), an odd token count, and k on both
    sides of the small-fan-in kernels' limit (8)."""
    _check_inverse_map_kernels(ext, 301, k, 40, dtype, 100 + k, empty_tokens=2)


@pytest.mark.parametrize("k", [1, 2, 5, 8])
@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 2568), (torch.float32, 1100),
                                     (torch.bfloat16, 4096), (torch.float16, 2048)])
def test_inverse_map_kernels_long_rows(ext, k, dtype, d):
    """Rows of several 16-byte vectors per lane, where the gathers issue the
    loads of several row chunks per pass: rows that end inside a pass (2568
    bf16 and 1100 fp32 elements leave some lanes one chunk more than the
    others), whole passes (C4's 4096, C5's 2048), dropped slots and tokens
    with no valid slot."""
    _check_inverse_map_kernels(ext, 97, k, d, dtype, 200 + k + d, empty_tokens=3)


@pytest.mark.parametrize("k,E,d,dtype", [(1, 4, 40, torch.bfloat16), (2, 8, 512, torch.bfloat16),
                                         (5, 17, 40, torch.float32), (8, 64, 512, torch.bfloat16),
                                         (8, 128, 2048, torch.float16), (12, 40, 64, torch.bfloat16)])
def test_pack_backward_inv_route_equals_the_two_ops(ext, k, E, d, dtype):
    """pack_backward_inv_route: the pack backward and the router's backward
    on its dw, in one launch (k <= 8) or two (k = 12). Bit-equal to
    pack_backward_inv followed by route_topk_backward, with gates and ids from
    the router on random logits and an inverse map with dropped (-1) and
    out-of-range slots in random packed order."""
    T = 1501
    A = T * k
    g = torch.Generator().manual_seed(7 * k + E)
    gates, topk = ext.route_topk(torch.randn(T, E, generator=g).cuda(), k)
    inv = torch.randperm(A, generator=g).to(torch.int32).view(T, k).clone()
    inv[torch.rand(T, k, generator=g) < 0.05] = -1
    inv[torch.rand(T, k, generator=g) < 0.02] = A + 3
    inv = inv.cuda()
    dpX = torch.randn(A, d, generator=g).to(dtype).cuda()
    dpw = torch.randn(A, generator=g).cuda()
    dX_ref, dw_ref = ext.pack_backward_inv(dpX, dpw, inv)
    dl_ref = ext.route_topk_backward(gates, topk, dw_ref, E)
    dX, dl = ext.pack_backward_inv_route(dpX, dpw, inv, gates, topk, E)
    torch.cuda.synchronize()
    assert torch.equal(bits(dX), bits(dX_ref))
    assert torch.equal(bits(dl), bits(dl_ref))
    assert (dl != 0).sum(1).max().item() <= k


def test_inverse_map_ops_check_row_counts(ext):
    """The inverse-map ops read rows p < T*k of their packed inputs: a tensor
    with another row count is rejected before any launch."""
    T, k, d = 16, 2, 8
    inv = torch.arange(T * k, dtype=torch.int32, device="cuda").view(T, k)
    y = torch.randn(T * k, d, device="cuda")
    w = torch.rand(T * k, device="cuda")
    dY = torch.randn(T, d, device="cuda")
    short_y, short_w = y[: T * k - 1].contiguous(), w[: T * k - 1].contiguous()
    for call in (lambda: ext.combine_inv(short_y, inv, w, torch.float32),
                 lambda: ext.combine_inv(y, inv, short_w, torch.float32),
                 lambda: ext.combine_backward_inv(short_y, inv, w, dY),
                 lambda: ext.combine_backward_inv(y, inv, short_w, dY),
                 lambda: ext.pack_backward_inv(short_y, w, inv),
                 lambda: ext.pack_backward_inv(y, short_w, inv)):
        with pytest.raises(RuntimeError, match=r"inv\.numel\(\)"):
            call()
    with pytest.raises(RuntimeError, match="GPU tensor|same device"):
        ext.combine_inv(y, inv, w.cpu(), torch.float32)
