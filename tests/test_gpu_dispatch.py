"""GPU parity: expert counting and token packing vs the CPU oracle (bit-exact)."""

import json

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from tests.conftest import GOLDEN

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16, torch.float64]


def bits(t: torch.Tensor) -> torch.Tensor:
    """Bit pattern view for exact comparison of float tensors."""
    t = t.detach().cpu().contiguous()
    view = {torch.float32: torch.int32, torch.float64: torch.int64, torch.float16: torch.int16,
            torch.bfloat16: torch.int16}.get(t.dtype)
    return t.view(view) if view is not None else t


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_pack_reference_kat(ext, dtype):
    """reference tests/test_packing.py:13-76, with the canonical order asserted exactly."""
    kat = json.loads((GOLDEN / "pack_kat.json").read_text())
    i, ex = kat["inputs"], kat["expected"]
    X = torch.tensor(i["X"], dtype=dtype, device="cuda")
    w = torch.tensor(i["topk_weights"], dtype=torch.float32, device="cuda")
    topk = torch.tensor(i["topk_experts"], dtype=torch.int32, device="cuda")
    cursor = torch.tensor(i["expert_offset_cpy"], dtype=torch.int32, device="cuda")
    packed_X, tid, expert, pw = ext.pack_tokens_kernel(X, w, topk, cursor)
    torch.cuda.synchronize()
    assert tid.tolist() == ex["packed_tokenId"]
    assert expert.tolist() == ex["packed_expert"]
    assert bits(pw).tolist() == bits(torch.tensor(ex["packed_topk_weights"])).tolist()
    assert torch.equal(bits(packed_X), bits(torch.tensor(ex["packed_X"], dtype=dtype)))
    assert cursor.tolist() == ex["cursor_after"]
    # the reference test's own checks (:65-76)
    for idx in range(8):
        assert torch.equal(packed_X[idx], X[tid[idx]])
    mask = torch.ones(4, dtype=torch.int32, device="cuda")
    assert ext.count_expert_kernel(topk, mask, 3, 2).tolist() == ex["counts"]


def route_case(cfg_id, T):
    d = O.make_inputs(cfg_id, T=T, with_weights=False)
    gates, idx, _ = O.route(d["logits"], d["cfg"].k)
    return d, gates, idx


@pytest.mark.parametrize("cfg_id,T", [(1, 4096), (2, 30720), (3, 30720), (5, 65536), (5, 777)])
def test_dispatch_bit_exact_config_routing(ext, cfg_id, T):
    """Fused count/offsets/pack at the configs' routing vs the oracle, bit for bit."""
    d, gates, idx = route_case(cfg_id, T)
    c = d["cfg"]
    X = d["X"]
    if cfg_id == 5:  # keep host memory modest: narrower rows, same routing
        X = X[:, :256].contiguous()
    counts, offsets, p = O.dispatch(X, gates, idx, c.E)
    Xg, wg, ig = X.cuda(), gates.cuda(), idx.cuda()
    g_counts, g_off, g_px, g_tid, g_ex, g_pw, g_inv = ext.dispatch_tokens(Xg, wg, ig, c.E)
    torch.cuda.synchronize()
    assert np.array_equal(g_counts.cpu().numpy(), counts)
    assert np.array_equal(g_off.cpu().numpy(), offsets)
    assert np.array_equal(g_tid.cpu().numpy(), p.token_id)
    assert np.array_equal(g_ex.cpu().numpy(), p.expert)
    assert np.array_equal(g_inv.cpu().numpy(), p.inv)
    assert torch.equal(bits(g_pw), bits(torch.from_numpy(p.packed_w)))
    assert torch.equal(bits(g_px), bits(p.packed_X))
    if cfg_id in (3, 5):
        assert (counts == 0).any() or cfg_id == 3  # C5 has dead experts


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("T,k,E,d", [(1, 1, 1, 1), (3, 2, 3, 8), (5, 3, 3, 7), (300, 4, 13, 33),
                                     (1000, 8, 128, 64), (257, 2, 1024, 16)])
def test_pack_tokens_random_vs_oracle(ext, dtype, T, k, E, d):
    g = torch.Generator().manual_seed(T * 7 + k)
    X = torch.randn(T, d, generator=g).to(dtype)
    w = torch.rand(T, k, generator=g)
    topk = torch.randint(0, E, (T, k), generator=g, dtype=torch.int32)
    counts = O.count_experts(topk, None, E)
    cursor = O.offsets_from_counts(counts)
    p = O.pack_tokens(X, w, topk, cursor)
    cur_g = torch.from_numpy(cursor).cuda()
    px, tid, ex, pw, inv = ext.pack_tokens_inv(X.cuda(), w.cuda(), topk.cuda(), cur_g)
    torch.cuda.synchronize()
    assert np.array_equal(cur_g.cpu().numpy(), p.cursor_after)
    assert np.array_equal(tid.cpu().numpy(), p.token_id)
    assert np.array_equal(ex.cpu().numpy(), p.expert)
    assert np.array_equal(inv.cpu().numpy(), p.inv)
    assert torch.equal(bits(pw), bits(torch.from_numpy(p.packed_w)))
    assert torch.equal(bits(px), bits(p.packed_X))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("T,k,E,d", [(300, 1, 13, 1000), (300, 3, 13, 1000), (200, 8, 40, 4104),
                                     (150, 2, 8, 4104), (100, 9, 16, 1000)])
def test_pack_tokens_long_rows_vs_oracle(ext, dtype, T, k, E, d):
    """Rows longer than one 16-byte vector per lane (the batched long-row
    copy): rows that end inside a batch (1000 and 4104 elements), k on both
    sides of the copy's register-slot limit (8), and out-of-range expert ids
    (their slots are skipped)."""
    g = torch.Generator().manual_seed(T * 11 + k + d)
    X = torch.randn(T, d, generator=g).to(dtype)
    w = torch.rand(T, k, generator=g)
    topk = torch.randint(0, E, (T, k), generator=g, dtype=torch.int32)
    topk[torch.rand(T, k, generator=g) < 0.05] = E + 3
    counts = O.count_experts(topk, None, E)
    cursor = O.offsets_from_counts(counts)
    p = O.pack_tokens(X, w, topk, cursor)
    cur_g = torch.from_numpy(cursor).cuda()
    px, tid, ex, pw, inv = ext.pack_tokens_inv(X.cuda(), w.cuda(), topk.cuda(), cur_g)
    torch.cuda.synchronize()
    n = int(counts.sum())  # the valid assignments fill slots [0, n)
    assert p.written[:n].all() and not p.written[n:].any()
    assert np.array_equal(cur_g.cpu().numpy(), p.cursor_after)
    assert np.array_equal(inv.cpu().numpy(), p.inv)
    assert np.array_equal(tid.cpu().numpy()[:n], p.token_id[:n])
    assert torch.equal(bits(px[:n]), bits(p.packed_X[:n]))


def test_count_with_mask(ext):
    g = torch.Generator().manual_seed(11)
    topk = torch.randint(0, 16, (5000, 4), generator=g, dtype=torch.int32)
    mask = (torch.rand(5000, generator=g) > 0.25).to(torch.int32)
    want = O.count_experts(topk, mask, 16)
    got = ext.count_expert_kernel(topk.cuda(), mask.cuda(), 16, 4)
    assert np.array_equal(got.cpu().numpy(), want)


def test_pack_drops_out_of_range_ids(ext):
    """Ids outside [0,E) are skipped (never written), like the oracle; no fault."""
    topk = torch.tensor([[0, 5], [1, -1], [1, 0]], dtype=torch.int32)
    w = torch.rand(3, 2)
    X = torch.randn(3, 4)
    cursor = torch.tensor([0, 2, 4], dtype=torch.int32)  # E = 2, ids 5 and -1 invalid
    p = O.pack_tokens(X, w, topk, cursor)
    cur_g = cursor.cuda()
    px, tid, ex, pw, inv = ext.pack_tokens_inv(X.cuda(), w.cuda(), topk.cuda(), cur_g)
    torch.cuda.synchronize()
    assert np.array_equal(inv.cpu().numpy(), p.inv)
    written = torch.from_numpy(p.written)
    assert torch.equal(px.cpu()[written], p.packed_X[written])
    assert np.array_equal(tid.cpu().numpy()[p.written], p.token_id[p.written])
    assert cur_g.tolist() == p.cursor_after.tolist()


def test_pack_is_deterministic(ext):
    d, gates, idx = route_case(3, 8192)
    X = d["X"].cuda()
    a = ext.dispatch_tokens(X, gates.cuda(), idx.cuda(), 64)
    b = ext.dispatch_tokens(X, gates.cuda(), idx.cuda(), 64)
    for x, y in zip(a, b):
        assert torch.equal(bits(x), bits(y))


def test_empty_tokens(ext):
    X = torch.empty(0, 8, device="cuda", dtype=torch.bfloat16)
    w = torch.empty(0, 2, device="cuda")
    topk = torch.empty(0, 2, device="cuda", dtype=torch.int32)
    counts, offsets, px, tid, ex, pw, inv = ext.dispatch_tokens(X, w, topk, 4)
    assert counts.tolist() == [0, 0, 0, 0]
    assert offsets.tolist() == [0, 0, 0, 0, 0]
    assert px.shape == (0, 8)


def test_errors_raise_runtime_error(ext):
    X = torch.randn(4, 3, device="cuda")
    w = torch.rand(4, 2, device="cuda")
    topk = torch.zeros(4, 2, dtype=torch.int32, device="cuda")
    with pytest.raises(RuntimeError):
        ext.pack_tokens_kernel(X.t(), w, topk, torch.zeros(3, dtype=torch.int32, device="cuda"))
    with pytest.raises(RuntimeError):
        ext.pack_tokens_kernel(X, w, topk.long(), torch.zeros(3, dtype=torch.int32, device="cuda"))
    with pytest.raises(RuntimeError):
        ext.count_expert_kernel(topk, torch.ones(4, dtype=torch.int32, device="cuda"), 2000, 2)


def block_hist(idx: np.ndarray, E: int, TB: int) -> np.ndarray:
    """[E, nb] expert counts of each TB-token block, by numpy bincount (independent of the kernels)."""
    T = idx.shape[0]
    nb = -(-T // TB)
    out = np.zeros((E, nb), dtype=np.int32)
    for b in range(nb):
        out[:, b] = np.bincount(idx[b * TB:(b + 1) * TB].reshape(-1), minlength=E)
    return out


def check_route_count(ext, logits, k, X, E):
    """route_topk_count + dispatch_tokens_counted vs route_topk + the oracle's dispatch."""
    from nanotitan_amd import capi

    T = logits.shape[0]
    want_g, want_i, _ = O.route(logits, k)
    g, i, ws = ext.route_topk_count(logits.cuda(), k, X.cuda())
    g_ref, i_ref = ext.route_topk(logits.cuda(), k)
    torch.cuda.synchronize()
    assert np.array_equal(i.cpu().numpy(), want_i.numpy())
    assert torch.equal(bits(g), bits(g_ref)) and torch.equal(i.cpu(), i_ref.cpu())
    TB = capi.load().nt_dispatch_block_tokens(T, k, X.shape[1], capi.dtype_code(X.dtype))
    nb = -(-T // TB)
    hist = ws[: E * nb * 4].view(torch.int32).cpu().numpy().reshape(E, nb)
    assert np.array_equal(hist, block_hist(want_i.numpy(), E, TB))
    counts, offsets, p = O.dispatch(X, want_g, want_i, E)
    outs = ext.dispatch_tokens_counted(X.cuda(), g, i, E, ws)
    g_counts, g_off, g_px, g_tid, g_ex, g_pw, g_inv = outs
    torch.cuda.synchronize()
    assert np.array_equal(g_counts.cpu().numpy(), counts)
    assert np.array_equal(g_off.cpu().numpy(), offsets)
    assert np.array_equal(g_tid.cpu().numpy(), p.token_id)
    assert np.array_equal(g_ex.cpu().numpy(), p.expert)
    assert np.array_equal(g_inv.cpu().numpy(), p.inv)
    assert torch.equal(bits(g_px), bits(p.packed_X))
    # same bits as the unfused dispatch on the kernel's own gates
    plain = ext.dispatch_tokens(X.cuda(), g, i, E)
    for a, b in zip(outs, plain):
        assert torch.equal(bits(a), bits(b))


@pytest.mark.parametrize("cfg_id,T", [(1, 4096), (2, 30720), (3, 30720), (5, 65536), (5, 777)])
def test_route_count_dispatch_config_routing(ext, cfg_id, T):
    """Router gate fused with the count, at the configs' logits: the per-block
    counts equal numpy's bincount and the dispatch from them equals the oracle."""
    d = O.make_inputs(cfg_id, T=T, with_weights=False)
    c = d["cfg"]
    X = d["X"]
    if cfg_id == 5:
        X = X[:, :256].contiguous()
    check_route_count(ext, d["logits"], c.k, X, c.E)


@pytest.mark.parametrize("T,E,k,d,dtype", [(1, 1, 1, 8, torch.float32), (7, 3, 3, 5, torch.float16),
                                           (1000, 16, 4, 1024, torch.float32),
                                           (513, 1024, 32, 16, torch.bfloat16),
                                           (2049, 128, 8, 4096, torch.bfloat16),
                                           (300, 9, 1, 2048, torch.bfloat16)])
def test_route_count_random(ext, T, E, k, d, dtype):
    """Ragged block tails, E from 1 to 1024, k up to 32, every row-size plan."""
    g_ = torch.Generator().manual_seed(T * 3 + E)
    logits = torch.randn(T, E, generator=g_)
    logits[::5] = torch.round(logits[::5])  # exact ties
    X = torch.randn(T, d, generator=g_).to(dtype)
    check_route_count(ext, logits, k, X, E)


def test_route_count_empty(ext):
    logits = torch.empty(0, 8, device="cuda")
    X = torch.empty(0, 16, device="cuda", dtype=torch.bfloat16)
    g, i, ws = ext.route_topk_count(logits, 2, X)
    assert g.shape == (0, 2) and i.shape == (0, 2)
    counts, offsets, px, *_ = ext.dispatch_tokens_counted(X, g, i, 8, ws)
    assert counts.tolist() == [0] * 8 and offsets.tolist() == [0] * 9 and px.shape == (0, 16)


def test_route_count_rejects_small_workspace(ext):
    logits = torch.randn(64, 8, device="cuda")
    X = torch.randn(64, 16, device="cuda")
    g, i, ws = ext.route_topk_count(logits, 2, X)
    with pytest.raises(RuntimeError):
        ext.dispatch_tokens_counted(X, g, i, 8, ws[:4])
    with pytest.raises(RuntimeError):
        ext.route_topk_count(logits, 2, X[:10])


@pytest.mark.parametrize("cfg_id,T,d", [(3, 30720, 512), (5, 65536, 2048), (2, 30720, 512)])
def test_counted_dispatch_keeps_the_counts(ext, cfg_id, T, d):
    """dispatch_tokens_counted only reads the per-block counts at the start
    of its workspace: they are unchanged after a call, and a second call on
    the same workspace gives the same bits. C3 and C5 routing take the
    separate scan launch (E x blocks above the in-pack fold limit), which
    writes the workspace's scratch after the counts; C2 the fold."""
    from nanotitan_amd import capi

    dd = O.make_inputs(cfg_id, T=T, with_weights=False)
    c = dd["cfg"]
    X = dd["X"][:, :d].contiguous().cuda()
    g, i, ws = ext.route_topk_count(dd["logits"].cuda(), c.k, X)
    TB = capi.load().nt_dispatch_block_tokens(T, c.k, d, capi.dtype_code(X.dtype))
    nb = -(-T // TB)
    counts_bytes = c.E * nb * 4
    before = ws[:counts_bytes].clone()
    first = ext.dispatch_tokens_counted(X, g, i, c.E, ws)
    torch.cuda.synchronize()
    assert torch.equal(ws[:counts_bytes], before)
    second = ext.dispatch_tokens_counted(X, g, i, c.E, ws)
    torch.cuda.synchronize()
    assert torch.equal(ws[:counts_bytes], before)
    for a, b in zip(first, second):
        assert torch.equal(bits(a), bits(b))
    want = np.bincount(O.route(dd["logits"], c.k)[1].numpy().ravel(), minlength=c.E)
    assert np.array_equal(first[0].cpu().numpy(), want)
    assert (c.E * nb > 8192) == (cfg_id in (3, 5))  # the separate scan path at C3 / C5


def test_counted_dispatch_opcheck_on_gpu(ext):
    """torch.library.opcheck on device tensors: the schema (workspace
    marked mutable) and the fake kernel agree with what the HIP op does."""
    from nanotitan_amd.extension import load_op_library

    load_op_library()
    dd = O.make_inputs(3, T=16384, with_weights=False)  # 64 experts x 256 blocks: the scan launch
    c = dd["cfg"]
    X = dd["X"][:, :64].contiguous().cuda()
    g, i, ws = torch.ops.nanotitan.route_topk_count(dd["logits"].cuda(), c.k, X)
    torch.library.opcheck(torch.ops.nanotitan.dispatch_tokens_counted.default,
                          (X, g, i, c.E, ws), test_utils=("test_schema", "test_faketensor"))
