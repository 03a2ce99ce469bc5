"""Pins the CPU oracle (CPU only, no GPU).

Each oracle function is checked against something other than itself: the
reference's known-answer tests (golden fixtures), the reference's own
invariant checks, independent library routines (torch.index_add_,
torch.autograd), brute-force loops on small inputs, and float64 bounds. A
plausible slip (dropped weight, transposed operand, wrong slot, off-by-one
segment) fails at least one of these.
"""

import itertools
import json

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from tests.conftest import GOLDEN


def load(name):
    return json.loads((GOLDEN / name).read_text())


# ------------------------------------------------------------- pack / count


def test_pack_matches_reference_kat():
    kat = load("pack_kat.json")
    i, ex = kat["inputs"], kat["expected"]
    X = torch.tensor(i["X"], dtype=torch.float32)
    topk = np.array(i["topk_experts"], dtype=np.int32)
    p = O.pack_tokens(X, np.array(i["topk_weights"], np.float32), topk,
                      np.array(i["expert_offset_cpy"], np.int32))
    assert p.token_id.tolist() == ex["packed_tokenId"]
    assert p.expert.tolist() == ex["packed_expert"]
    np.testing.assert_array_equal(p.packed_w, np.array(ex["packed_topk_weights"], np.float32))
    assert torch.equal(p.packed_X, torch.tensor(ex["packed_X"], dtype=torch.float32))
    assert p.inv.tolist() == ex["inv"]
    assert p.cursor_after.tolist() == ex["cursor_after"]
    assert O.count_experts(topk, None, 3).tolist() == ex["counts"]
    assert O.offsets_from_counts(ex["counts"]).tolist() == i["expert_offset_cpy"]


def test_pack_backward_matches_kat():
    kat = load("pack_kat.json")
    i, ex, bw = kat["inputs"], kat["expected"], kat["backward"]
    dX, dw = O.pack_backward(
        torch.tensor(bw["packed_X_grad"], dtype=torch.float32),
        np.array(bw["packed_topk_weights_grad"], np.float32),
        np.array(ex["packed_tokenId"], np.int32),
        np.array(ex["packed_expert"], np.int32),
        np.array(i["topk_experts"], np.int32),
    )
    assert dX.tolist() == bw["X_grad"]
    np.testing.assert_array_equal(dw, np.array(bw["topk_weights_grad"], np.float32))


def brute_pack(topk, cursor):
    """Pure-Python canonical pack: walk assignments in flat order, bump a cursor."""
    T, k = len(topk), len(topk[0])
    E = len(cursor) - 1
    cur = list(cursor)
    slots = {}
    for t in range(T):
        for j in range(k):
            e = topk[t][j]
            if 0 <= e < E:
                s = cur[e]
                cur[e] += 1
                if 0 <= s < T * k:
                    slots[(t, j)] = s
    return slots, cur


@pytest.mark.parametrize("seed", range(6))
def test_pack_brute_force(seed):
    rng = np.random.default_rng(seed)
    T, k, E = int(rng.integers(1, 40)), int(rng.integers(1, 5)), int(rng.integers(1, 9))
    topk = rng.integers(0, E, size=(T, k)).astype(np.int32)
    if seed % 2:  # duplicate experts inside a row, and an out-of-range id
        topk[0, :] = topk[0, 0]
        topk[-1, -1] = E + 3
    counts = O.count_experts(topk, None, E)
    cursor = O.offsets_from_counts(counts)
    X = torch.arange(T * 3, dtype=torch.float32).reshape(T, 3)
    w = rng.random((T, k)).astype(np.float32)
    p = O.pack_tokens(X, w, topk, cursor)
    slots, cur = brute_pack(topk.tolist(), cursor.tolist())
    assert p.cursor_after.tolist() == cur
    for (t, j), s in slots.items():
        assert p.inv[t, j] == s
        assert p.token_id[s] == t and p.expert[s] == topk[t, j] and p.packed_w[s] == w[t, j]
        assert torch.equal(p.packed_X[s], X[t])
    assert (p.inv >= 0).sum() == len(slots)


def test_count_closed_form_and_mask():
    rng = np.random.default_rng(7)
    topk = rng.integers(0, 6, size=(50, 3)).astype(np.int32)
    mask = (rng.random(50) > 0.3).astype(np.int32)
    want = [0] * 6
    for t in range(50):
        if mask[t]:
            for j in range(3):
                want[topk[t, j]] += 1
    assert O.count_experts(topk, mask, 6).tolist() == want
    assert O.count_experts(topk, None, 6).sum() == 150


def test_pack_reference_invariants_large():
    """The reference benchmark's own checks (benchmarks/bench_pack_tokens.py:176-223)."""
    d = O.make_inputs(3, T=2048, with_weights=False)
    gates, idx, _ = O.route(d["logits"], 8)
    counts, offsets, p = O.dispatch(d["X"], gates, idx, 64)
    A = 2048 * 8
    assert p.written.all()
    assert torch.equal(p.packed_X, d["X"][torch.from_numpy(p.token_id.astype(np.int64))])
    for e in range(64):
        assert (p.expert[offsets[e]:offsets[e + 1]] == e).all()
    # every packed assignment matches the routing, with its gate
    t = p.token_id.astype(np.int64)
    match = idx.numpy()[t] == p.expert[:, None]
    assert match.any(axis=1).all()
    np.testing.assert_array_equal(p.packed_w, gates.numpy()[t, match.argmax(axis=1)])
    # stability: within a segment, flat assignment index increases
    flat = (p.token_id.astype(np.int64) * 8 + match.argmax(axis=1))
    for e in range(64):
        seg = flat[offsets[e]:offsets[e + 1]]
        assert (np.diff(seg) > 0).all()
    assert offsets[-1] == A


# ---------------------------------------------------------------- combine


@pytest.mark.parametrize("case", ["top1", "top2"])
def test_combine_matches_reference_kat(case):
    kat = load("combine_kat.json")[case]
    out = O.combine_tokens(np.array(kat["expert_outputs"], np.float32),
                           np.array(kat["packed_tokenId"], np.int32),
                           np.array(kat["packed_topk_weights"], np.float32), kat["num_tokens"])
    np.testing.assert_allclose(out, np.array(kat["expected"]), rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("T,A,d", [(3, 6, 8), (5, 11, 7), (64, 300, 33)])
def test_combine_equals_index_add(T, A, d):
    """Sequential fp32 scatter-add in packed order == torch.index_add_ (CPU), bit for bit."""
    g = torch.Generator().manual_seed(A)
    y = torch.randn(A, d, generator=g)
    w = torch.randn(A, generator=g)
    tid = torch.randint(0, T, (A,), generator=g, dtype=torch.int32)
    ref = torch.zeros(T, d).index_add_(0, tid.long(), y * w[:, None])
    got = O.combine_tokens(y, tid, w, T)
    np.testing.assert_array_equal(got, ref.numpy())
    exact = np.zeros((T, d))
    np.add.at(exact, tid.numpy(), (y.double() * w.double()[:, None]).numpy())
    np.testing.assert_allclose(got, exact, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_combine_backward_vs_autograd(dtype):
    T, A, d = 5, 11, 7
    g = torch.Generator().manual_seed(0)
    y = torch.randn(A, d, generator=g).to(dtype).requires_grad_(True)
    w = torch.randn(A, generator=g).requires_grad_(True)
    tid = torch.tensor([i % T for i in range(A)], dtype=torch.int32)
    out = torch.zeros(T, d).index_add(0, tid.long(), y.float() * w[:, None])
    dY = torch.randn(T, d, generator=g)
    out.backward(dY)
    dy, dw = O.combine_backward(y.detach(), tid, w.detach(), dY, out_dtype=dtype)
    assert torch.equal(dy, y.grad)
    np.testing.assert_allclose(dw, w.grad.numpy(), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_pack_backward_vs_autograd(dtype):
    T, k, d = 5, 3, 7
    g = torch.Generator().manual_seed(1)
    x = torch.randn(T, d, generator=g).to(dtype).requires_grad_(True)
    wts = torch.rand(T, k, generator=g).requires_grad_(True)
    topk = (torch.arange(T * k) % 3).reshape(T, k).to(torch.int32)
    counts = O.count_experts(topk, None, 3)
    p = O.pack_tokens(x.detach(), wts.detach(), topk, O.offsets_from_counts(counts))
    tid = torch.from_numpy(p.token_id.astype(np.int64))
    slot = (topk[tid] == torch.from_numpy(p.expert)[:, None]).long().argmax(dim=1)
    packed = x[tid].float()
    pw = wts[tid, slot]
    gp = torch.randn(T * k, d, generator=g)
    gw = torch.randn(T * k, generator=g)
    ((packed * gp).sum() + (pw * gw).sum()).backward()
    dX, dw = O.pack_backward(gp, gw, p.token_id, p.expert, topk, out_dtype=torch.float32)
    # autograd accumulates a bf16 leaf's gradient in bf16; the oracle sums in fp32
    tol = dict(rtol=1e-5, atol=1e-6) if dtype == torch.float32 else dict(rtol=2e-2, atol=2e-2)
    torch.testing.assert_close(dX, x.grad.float(), **tol)
    np.testing.assert_allclose(dw, wts.grad.numpy(), rtol=1e-6, atol=1e-7)


def test_pack_backward_first_match_rule():
    """Duplicate experts in a row: every matching row lands on the first slot."""
    topk = np.array([[2, 2], [0, 1]], np.int32)
    tid = np.array([0, 0, 1, 1], np.int32)
    ex = np.array([2, 2, 0, 1], np.int32)
    dpw = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    _, dw = O.pack_backward(torch.zeros(4, 1), dpw, tid, ex, topk)
    assert dw.tolist() == [[3.0, 0.0], [3.0, 4.0]]


# ---------------------------------------------------------- grouped GEMM


def torch_grouped_gemm(X, W, offsets):
    """The reference test's formula (tests/test_grouped_gemm.py:42-48)."""
    return torch.cat([X[offsets[e]:offsets[e + 1]] @ W[e] for e in range(len(offsets) - 1)])


@pytest.mark.parametrize("offsets", [[0, 3, 4, 8], [0, 0, 5, 5, 9], [0, 9]])
def test_grouped_gemm_vs_autograd(offsets):
    g = torch.Generator().manual_seed(len(offsets))
    A, K, N, E = offsets[-1], 6, 5, len(offsets) - 1
    X = torch.randn(A, K, generator=g, dtype=torch.float64).requires_grad_(True)
    W = torch.randn(E, K, N, generator=g, dtype=torch.float64).requires_grad_(True)
    G = torch.randn(A, N, generator=g, dtype=torch.float64)
    out = torch_grouped_gemm(X, W, offsets)
    out.backward(G)
    off = np.array(offsets, np.int32)
    torch.testing.assert_close(O.grouped_gemm(X, off, W), out.detach())
    torch.testing.assert_close(O.grouped_gemm_dx(W, off, G), X.grad)
    torch.testing.assert_close(O.grouped_gemm_dw(X, off, G), W.grad)
    # an empty expert has an all-zero weight gradient
    for e in range(E):
        if offsets[e] == offsets[e + 1]:
            assert not O.grouped_gemm_dw(X, off, G)[e].any()


def test_grouped_gemm_nonsquare_transpose_guard():
    """K != N so a transposed W in dX or a swapped operand in dW cannot type-check."""
    off = np.array([0, 2, 7], np.int32)
    X = torch.randn(7, 3, dtype=torch.float64)
    W = torch.randn(2, 3, 4, dtype=torch.float64)
    G = torch.randn(7, 4, dtype=torch.float64)
    assert O.grouped_gemm(X, off, W).shape == (7, 4)
    assert O.grouped_gemm_dx(W, off, G).shape == (7, 3)
    assert O.grouped_gemm_dw(X, off, G).shape == (2, 3, 4)


# --------------------------------------------------------------- routing


def test_route_tie_rule_brute_force():
    logits = torch.tensor([[0.0, 0.0, 0.0, 0.0], [1.0, 3.0, 3.0, -1.0], [2.0, 2.0, 5.0, 2.0]])
    gates, idx, _ = O.route(logits, 2)
    for t in range(logits.shape[0]):
        order = sorted(range(4), key=lambda e: (-float(logits[t, e]), e))[:2]
        assert idx[t].tolist() == order
    torch.testing.assert_close(gates.sum(-1), torch.ones(3))


def test_route_c5_ties_and_dead_experts():
    d = O.make_inputs(5, T=8192, with_weights=False)
    gates, idx, probs = O.route(d["logits"], 8)
    dead = torch.isinf(d["logits"][0]).nonzero().squeeze(1)
    assert dead.numel() == 16
    assert not torch.isin(idx.long(), dead).any()
    tied = (d["logits"] == 0).sum(1) == 112
    live = torch.ones(128, dtype=torch.bool)
    live[dead] = False
    lowest8 = live.nonzero().squeeze(1)[:8]
    for t in tied.nonzero().squeeze(1)[:20]:
        assert idx[t].tolist() == lowest8.tolist()
        torch.testing.assert_close(gates[t], torch.full((8,), 0.125))


# ----------------------------------------------------------------- layer


@pytest.mark.parametrize("ffn", ["gelu", "swiglu"])
def test_moe_layer_torch_vs_dense(ffn):
    g = torch.Generator().manual_seed(3)
    T, d, f, E, k = 12, 6, 10, 4, 2
    x = torch.randn(T, d, generator=g)
    logits = torch.randn(T, E, generator=g)
    names = ["up", "down"] if ffn == "gelu" else ["gate", "val", "out"]
    weights = {n: torch.randn(E, f, d, generator=g) * 0.3 if n in ("down", "out")
               else torch.randn(E, d, f, generator=g) * 0.3 for n in names}
    dY = torch.randn(T, d, generator=g)
    out, grads = O.moe_layer_torch(x, logits, weights, k, ffn=ffn, dY=dY)
    xr = x.clone().double().requires_grad_(True)
    lr = logits.clone().double().requires_grad_(True)
    wr = {n: w.double().requires_grad_(True) for n, w in weights.items()}
    dense = O.moe_layer_dense(xr, lr, wr, k, ffn=ffn)
    torch.testing.assert_close(out.double(), dense.detach(), rtol=1e-5, atol=1e-5)
    dense.backward(dY.double())
    torch.testing.assert_close(grads["x"].double(), xr.grad, rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(grads["logits"].double(), lr.grad, rtol=1e-4, atol=1e-5)
    for n in names:
        torch.testing.assert_close(grads[n].double(), wr[n].grad, rtol=1e-4, atol=1e-5)


def test_pinning_table_covers_every_function():
    public = {n for n in ("count_experts", "offsets_from_counts", "pack_tokens", "combine_tokens",
                          "combine_backward", "pack_backward", "grouped_gemm", "grouped_gemm_dx",
                          "grouped_gemm_dw", "route", "moe_layer")}
    assert public <= set(O.PINNING)
    for n in itertools.chain(public - {"moe_layer"}):
        assert hasattr(O, n)
