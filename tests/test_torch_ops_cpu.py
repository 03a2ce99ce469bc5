"""torch.ops.nanotitan on CPU tensors: the op library's CPU kernels against the
oracle (bit-exact for the integer work and the ordered fp32 sums, the GPU
tests' tolerances for dot products and GEMMs), every op's Meta kernel
against the CPU kernel's output shapes, and torch.library.opcheck of the
schemas. No GPU is needed: these run in the build container."""

import json

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from tests.conftest import GOLDEN

REFERENCE_OPS = ["count_expert_kernel", "pack_tokens_kernel", "combine_tokens_kernel",
                 "combine_kernel_backward", "pack_kernel_backward", "grouped_gemm_kernel",
                 "bwd_grouped_gemm_dW_kernel", "bwd_grouped_gemm_dX_kernel"]
LAYER_OPS = ["grouped_gemm_gelu", "bwd_grouped_gemm_dX_gelu", "grouped_gemm_swiglu",
             "bwd_grouped_gemm_dX_swiglu", "bwd_grouped_gemm_dX2", "bwd_grouped_gemm_dW_dX",
             "bwd_grouped_gemm_dW_dX_gelu", "bwd_grouped_gemm_dW_dX_swiglu",
             "bwd_grouped_gemm_dW_dX2", "route_topk", "route_topk_count", "route_topk_backward",
             "dispatch_tokens", "dispatch_tokens_counted", "pack_tokens_inv", "combine_inv",
             "combine_backward_inv", "pack_backward_inv", "pack_backward_inv_route"]
DTYPES = [torch.float32, torch.float16, torch.bfloat16, torch.float64]


@pytest.fixture(scope="module")
def ops():
    from nanotitan_amd.extension import load_op_library

    return load_op_library()


def bits(t):
    t = t.detach().cpu()
    return t.view({2: torch.int16, 4: torch.int32, 8: torch.int64}[t.element_size()])


@pytest.mark.parametrize("name", REFERENCE_OPS + LAYER_OPS)
def test_every_op_has_gpu_cpu_and_meta_kernels(ops, name):
    qual = f"nanotitan::{name}"
    for key in ("CUDA", "CPU", "Meta"):
        assert torch._C._dispatch_has_kernel_for_dispatch_key(qual, key), (name, key)


def test_reference_pack_kat(ops):
    """reference tests/test_packing.py:14-76 (golden vectors): counts, canonical
    order, packed rows and gates, inverse map, cursor post-state, and the
    pack backward of the same fixture."""
    kat = json.loads((GOLDEN / "pack_kat.json").read_text())
    inp, want, bwd = kat["inputs"], kat["expected"], kat["backward"]
    topk = torch.tensor(inp["topk_experts"], dtype=torch.int32)
    X = torch.tensor(inp["X"], dtype=torch.float32)
    w = torch.tensor(inp["topk_weights"], dtype=torch.float32)
    E = len(want["counts"])
    mask = torch.ones(topk.shape[0], dtype=torch.int32)
    counts = ops.count_expert_kernel(topk, mask, E, topk.shape[1])
    assert counts.tolist() == want["counts"]
    cursor = torch.tensor(inp["expert_offset_cpy"], dtype=torch.int32)
    packed_X, tid, ex, pw, inv = ops.pack_tokens_inv(X, w, topk, cursor)
    assert tid.tolist() == want["packed_tokenId"]
    assert ex.tolist() == want["packed_expert"]
    assert inv.tolist() == want["inv"]
    assert cursor.tolist() == want["cursor_after"]
    assert torch.equal(packed_X, torch.tensor(want["packed_X"], dtype=torch.float32))
    assert torch.equal(pw, torch.tensor(want["packed_topk_weights"], dtype=torch.float32))
    dX, dw = ops.pack_kernel_backward(torch.tensor(bwd["packed_X_grad"], dtype=torch.float32),
                                      torch.tensor(bwd["packed_topk_weights_grad"]), tid, ex, topk)
    assert dX.tolist() == bwd["X_grad"]
    assert dw.tolist() == bwd["topk_weights_grad"]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("T,k,E,d", [(1, 1, 1, 1), (37, 3, 5, 7), (500, 8, 64, 24)])
def test_count_and_pack_vs_oracle(ops, dtype, T, k, E, d):
    g = torch.Generator().manual_seed(T * k + E)
    X = torch.randn(T, d, generator=g).to(dtype)
    w = torch.rand(T, k, generator=g)
    topk = torch.randint(-1, E + 1, (T, k), generator=g, dtype=torch.int32)  # incl. out of range
    mask = (torch.rand(T, generator=g) < 0.8).to(torch.int32)
    counts = ops.count_expert_kernel(topk, mask, E, k)
    assert np.array_equal(counts.numpy(), O.count_experts(topk, mask, E))
    cursor = torch.from_numpy(O.offsets_from_counts(O.count_experts(topk, None, E)))
    want = O.pack_tokens(X, w, topk, cursor)
    got = ops.pack_tokens_inv(X, w, topk, cursor)
    ok = torch.from_numpy(want.written)
    assert np.array_equal(got[4].numpy(), want.inv)
    assert np.array_equal(got[1].numpy()[want.written], want.token_id[want.written])
    assert np.array_equal(got[2].numpy()[want.written], want.expert[want.written])
    assert torch.equal(bits(got[0][ok]), bits(want.packed_X[ok]))
    assert torch.equal(bits(got[3][ok]), bits(torch.from_numpy(want.packed_w)[ok]))
    assert np.array_equal(cursor.numpy(), want.cursor_after)


@pytest.mark.parametrize("cfg_id", [2, 3, 5])
def test_dispatch_tokens_config_routing(ops, cfg_id):
    d = O.make_inputs(cfg_id, T=2048, with_weights=False)
    c = d["cfg"]
    gates, idx, _ = O.route(d["logits"], c.k)
    X = d["X"][:, :40].contiguous()
    counts, offsets, p = O.dispatch(X, gates, idx, c.E)
    got = ops.dispatch_tokens(X, gates, idx, c.E)
    assert np.array_equal(got[0].numpy(), counts)
    assert np.array_equal(got[1].numpy(), offsets)
    assert torch.equal(bits(got[2]), bits(p.packed_X))
    assert np.array_equal(got[3].numpy(), p.token_id)
    assert np.array_equal(got[4].numpy(), p.expert)
    assert np.array_equal(got[5].numpy(), p.packed_w)
    assert np.array_equal(got[6].numpy(), p.inv)
    # the router + counted dispatch gives the same pack
    g2, i2, ws = ops.route_topk_count(d["logits"].contiguous(), c.k, X)
    assert np.array_equal(i2.numpy(), idx.numpy())
    got2 = ops.dispatch_tokens_counted(X, g2, i2, c.E, ws)
    assert np.array_equal(got2[6].numpy(), p.inv)


@pytest.mark.parametrize("case", ["top1", "top2"])
def test_combine_reference_kat(ops, case):
    """reference tests/test_combine.py:12-90 (golden vectors)."""
    kat = json.loads((GOLDEN / "combine_kat.json").read_text())[case]
    y = torch.tensor(kat["expert_outputs"], dtype=torch.float32)
    tid = torch.tensor(kat["packed_tokenId"], dtype=torch.int32)
    w = torch.tensor(kat["packed_topk_weights"], dtype=torch.float32)
    out = ops.combine_tokens_kernel(y, tid, w, kat["num_tokens"], 2)
    torch.testing.assert_close(out, torch.tensor(kat["expected"]), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("T,A,d", [(3, 6, 8), (5, 11, 7), (64, 64 * 300, 24), (50, 0, 16)])
def test_combine_and_backward_vs_oracle(ops, dtype, T, A, d):
    g = torch.Generator().manual_seed(T + A + d)
    y = torch.randn(A, d, generator=g).to(dtype)
    w = torch.randn(A, generator=g)
    tid = torch.randint(-1, T + 1, (A,), generator=g, dtype=torch.int32)
    out = ops.combine_tokens_kernel(y, tid, w, T, d)
    assert torch.equal(bits(out), bits(torch.from_numpy(O.combine_tokens(y, tid, w, T))))
    dY = torch.randn(T, d, generator=g)
    dy, dw = ops.combine_kernel_backward(y, tid, w, dY, d)
    want_dy, want_dw = O.combine_backward(y, tid, w, dY, out_dtype=dtype)
    assert torch.equal(bits(dy), bits(want_dy))
    np.testing.assert_allclose(dw.numpy(), want_dw, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("T,k,E,d", [(3, 2, 3, 8), (5, 3, 3, 7), (300, 8, 64, 40), (77, 1, 4, 5)])
def test_inverse_map_ops_and_pack_backward(ops, dtype, T, k, E, d):
    g = torch.Generator().manual_seed(T * k)
    X = torch.randn(T, d, generator=g).to(dtype)
    w = torch.rand(T, k, generator=g)
    topk = torch.argsort(torch.rand(T, E, generator=g), dim=1)[:, :k].to(torch.int32)
    counts, offsets, p = O.dispatch(X, w, topk, E)
    A = T * k
    tid, inv, pw = (torch.from_numpy(a) for a in (p.token_id, p.inv, p.packed_w))
    y = torch.randn(A, d, generator=g).to(dtype)
    want = torch.from_numpy(O.combine_tokens(y, tid, pw, T))
    assert torch.equal(bits(ops.combine_inv(y, inv, pw, torch.float32)), bits(want))
    assert torch.equal(bits(ops.combine_inv(y, inv, pw, dtype)), bits(want.to(dtype)))
    dY = torch.randn(T, d, generator=g)
    dy, dw = ops.combine_backward_inv(y, inv, pw, dY)
    want_dy, want_dw = O.combine_backward(y, tid, pw, dY, out_dtype=dtype)
    assert torch.equal(bits(dy), bits(want_dy))
    np.testing.assert_allclose(dw.numpy(), want_dw, rtol=1e-5, atol=1e-5)
    dpX = torch.randn(A, d, generator=g).to(dtype)
    dpw = torch.randn(A, generator=g)
    want_dX, want_dw2 = O.pack_backward(dpX, dpw, p.token_id, p.expert, topk, out_dtype=dtype)
    dX, dw2 = ops.pack_kernel_backward(dpX, dpw, tid, torch.from_numpy(p.expert), topk)
    assert torch.equal(bits(dX), bits(want_dX)) and torch.equal(bits(dw2), bits(torch.from_numpy(want_dw2)))
    dX2, dw3 = ops.pack_backward_inv(dpX, dpw, inv)
    assert torch.equal(bits(dX2), bits(want_dX)) and torch.equal(bits(dw3), bits(torch.from_numpy(want_dw2)))
    # the router's backward on that dw, fused (route_topk_backward is pinned
    # against torch autograd in test_route_topk_vs_oracle)
    dX3, dl = ops.pack_backward_inv_route(dpX, dpw, inv, w, topk, E)
    assert torch.equal(bits(dX3), bits(want_dX))
    assert torch.equal(bits(dl), bits(ops.route_topk_backward(w, topk, dw3, E)))


def test_pack_backward_first_match_rule(ops):
    """Duplicate experts in a row: the reference's first-match rule (backward_pack_kernel.cu:35-42)."""
    topk = torch.tensor([[2, 2], [0, 1]], dtype=torch.int32)
    tid = torch.tensor([0, 0, 1, 1], dtype=torch.int32)
    ex = torch.tensor([2, 2, 0, 1], dtype=torch.int32)
    dpw = torch.tensor([1.0, 2.0, 3.0, 4.0])
    _, dw = ops.pack_kernel_backward(torch.zeros(4, 3), dpw, tid, ex, topk)
    assert dw.tolist() == [[3.0, 0.0], [3.0, 4.0]]


TOL = {torch.float32: dict(rtol=1e-4, atol=5e-4), torch.float64: dict(rtol=1e-9, atol=1e-9),
       torch.float16: dict(rtol=2e-2, atol=2e-2), torch.bfloat16: dict(rtol=2e-2, atol=2e-2)}


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("counts,K,N", [([3, 1, 4], 16, 24), ([0, 40, 0, 7, 1], 32, 8)])
def test_grouped_gemm_family_vs_oracle(ops, dtype, counts, K, N):
    g = torch.Generator().manual_seed(sum(counts) + K)
    off = torch.tensor(np.concatenate([[0], np.cumsum(counts)]), dtype=torch.int32)
    A, E = int(off[-1]), len(counts)
    X = torch.randn(A, K, generator=g).to(dtype)
    W = (torch.randn(E, K, N, generator=g) / 4).to(dtype)
    G = torch.randn(A, N, generator=g).to(dtype)
    tol = TOL[dtype]
    torch.testing.assert_close(ops.grouped_gemm_kernel(X, off, W).double(),
                               O.grouped_gemm(X, off, W).to(dtype).double(), **tol)
    torch.testing.assert_close(ops.bwd_grouped_gemm_dX_kernel(W, off, G).double(),
                               O.grouped_gemm_dx(W, off, G).to(dtype).double(), **tol)
    dW = ops.bwd_grouped_gemm_dW_kernel(X, off, G)
    torch.testing.assert_close(dW.double(), O.grouped_gemm_dw(X, off, G).to(dtype).double(),
                               rtol=tol["rtol"], atol=tol["atol"] * 8)
    dW2, dX2 = ops.bwd_grouped_gemm_dW_dX(X, W, off, G)
    assert torch.equal(bits(dW2), bits(dW))
    assert torch.equal(bits(dX2), bits(ops.bwd_grouped_gemm_dX_kernel(W, off, G)))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_fused_ffn_ops_vs_torch_graph(ops, dtype):
    """The fused GELU / SwiGLU ops on CPU equal the unfused torch graph with
    the same roundings (reference src/model/feed_fwd.py:102-112)."""
    g = torch.Generator().manual_seed(3)
    counts = [5, 0, 9, 2]
    off = torch.tensor(np.concatenate([[0], np.cumsum(counts)]), dtype=torch.int32)
    A, E, d, f = int(off[-1]), len(counts), 16, 32
    X = torch.randn(A, d, generator=g).to(dtype)
    Wu = (torch.randn(E, d, f, generator=g) / 3).to(dtype)
    Wv = (torch.randn(E, d, f, generator=g) / 3).to(dtype)
    Wd = (torch.randn(E, f, d, generator=g) / 3).to(dtype)
    dy = torch.randn(A, d, generator=g).to(dtype)
    h = O.grouped_gemm(X, off, Wu).to(dtype)
    act, act_grad = ops.grouped_gemm_gelu(X, off, Wu)
    hd = h.double().requires_grad_(True)
    ref = torch.nn.functional.gelu(hd)
    (ref_grad,) = torch.autograd.grad(ref.sum(), hd)
    tol = TOL[dtype]
    torch.testing.assert_close(act.double(), ref.detach().to(dtype).double(), **tol)
    torch.testing.assert_close(act_grad.double(), ref_grad.to(dtype).double(), **tol)
    dH = ops.bwd_grouped_gemm_dX_gelu(Wd, off, dy, act_grad)
    want = (O.grouped_gemm_dx(Wd, off, dy).to(dtype).float() * act_grad.float()).to(dtype)
    torch.testing.assert_close(dH.double(), want.double(), **tol)
    hidden, gate, value = ops.grouped_gemm_swiglu(X, off, Wu, Wv)
    torch.testing.assert_close(gate.double(), h.double(), **tol)
    torch.testing.assert_close(
        hidden.double(),
        (torch.nn.functional.silu(gate.float()).to(dtype).float() * value.float()).to(dtype).double(),
        **tol)
    dg, dv = ops.bwd_grouped_gemm_dX_swiglu(Wd, off, dy, gate, value)
    gq, vq = gate.double().requires_grad_(True), value.double().requires_grad_(True)
    dhid = O.grouped_gemm_dx(Wd, off, dy).to(dtype).double()
    want_g, want_v = torch.autograd.grad(torch.nn.functional.silu(gq) * vq, (gq, vq), dhid)
    torch.testing.assert_close(dg.double(), want_g.to(dtype).double(), rtol=4e-2, atol=4e-2)
    torch.testing.assert_close(dv.double(), want_v.to(dtype).double(), rtol=4e-2, atol=4e-2)
    dX = ops.bwd_grouped_gemm_dX2(Wu, Wv, off, dg, dv)
    want_dX = O.grouped_gemm_dx(Wu, off, dg) + O.grouped_gemm_dx(Wv, off, dv)
    torch.testing.assert_close(dX.double(), want_dX.to(dtype).double(), **tol)


@pytest.mark.parametrize("cfg_id", [2, 3, 5])
def test_route_topk_vs_oracle(ops, cfg_id):
    d = O.make_inputs(cfg_id, T=1500, with_weights=False)
    k = d["cfg"].k
    logits = d["logits"].contiguous()
    gates, idx = ops.route_topk(logits, k)
    want_g, want_i, _ = O.route(logits, k)
    assert np.array_equal(idx.numpy(), want_i.numpy())
    torch.testing.assert_close(gates, want_g, rtol=2e-6, atol=2e-7)
    dg = torch.randn(gates.shape, generator=torch.Generator().manual_seed(1))
    dl = ops.route_topk_backward(gates, idx, dg, logits.shape[1])
    lz = logits.double().clone().requires_grad_(True)
    sel = torch.gather(lz, 1, idx.long())
    (want_dl,) = torch.autograd.grad(sel.softmax(-1), lz, dg.double())
    torch.testing.assert_close(dl.double(), want_dl, rtol=1e-5, atol=1e-6)


def test_route_topk_special_values(ops):
    """Ties go to the lower id, -0 ties +0, NaN ranks below -inf."""
    z = torch.tensor([[1.0, 1.0, 0.5, 1.0], [-0.0, 0.0, float("nan"), float("-inf")],
                      [float("nan"), float("-inf"), float("nan"), -3.0]])
    _, idx = ops.route_topk(z, 2)
    assert idx.tolist() == [[0, 1], [0, 1], [3, 1]]


def _meta(t):
    return t.to("meta") if isinstance(t, torch.Tensor) else t


def _cases():
    g = torch.Generator().manual_seed(0)
    T, k, E, d, f = 24, 2, 4, 8, 16
    A = T * k
    X = torch.randn(T, d, generator=g)
    w = torch.rand(T, k, generator=g)
    topk = torch.argsort(torch.rand(T, E, generator=g), 1)[:, :k].to(torch.int32).contiguous()
    off = torch.tensor([0, 10, 10, 30, A], dtype=torch.int32)
    inv = torch.randperm(A, generator=g).to(torch.int32).view(T, k)
    tid = torch.randint(0, T, (A,), generator=g, dtype=torch.int32)
    ex = torch.randint(0, E, (A,), generator=g, dtype=torch.int32)
    pX = torch.randn(A, d, generator=g)
    pw = torch.rand(A, generator=g)
    Wu, Wv = torch.randn(E, d, f, generator=g), torch.randn(E, d, f, generator=g)
    Wd = torch.randn(E, f, d, generator=g)
    H, H2, H3 = (torch.randn(A, f, generator=g) for _ in range(3))
    dy, dYt, dgt = torch.randn(A, d, generator=g), torch.randn(T, d, generator=g), torch.randn(T, k, generator=g)
    logits = torch.randn(T, E, generator=g)
    # the expert offsets of these ids, so every packed slot is written
    cursor = torch.zeros(E + 1, dtype=torch.int32)
    cursor[1:] = torch.cumsum(torch.bincount(topk.flatten().long(), minlength=E), 0)
    return {
        "count_expert_kernel": (topk, torch.ones(T, dtype=torch.int32), E, k),
        "pack_tokens_kernel": (X, w, topk, cursor.clone()),
        "pack_tokens_inv": (X, w, topk, cursor.clone()),
        "combine_tokens_kernel": (pX, tid, pw, T, d),
        "combine_kernel_backward": (pX, tid, pw, dYt, d),
        "pack_kernel_backward": (pX, pw, tid, ex, topk),
        "grouped_gemm_kernel": (pX, off, Wu),
        "bwd_grouped_gemm_dW_kernel": (pX, off, H),
        "bwd_grouped_gemm_dX_kernel": (Wu, off, H),
        "grouped_gemm_gelu": (pX, off, Wu),
        "bwd_grouped_gemm_dX_gelu": (Wd, off, dy, H),
        "grouped_gemm_swiglu": (pX, off, Wu, Wv),
        "bwd_grouped_gemm_dX_swiglu": (Wd, off, dy, H, H2),
        "bwd_grouped_gemm_dX2": (Wu, Wv, off, H, H2),
        "bwd_grouped_gemm_dW_dX": (pX, Wu, off, H),
        "bwd_grouped_gemm_dW_dX_gelu": (H, Wd, off, dy, H2),
        "bwd_grouped_gemm_dW_dX_swiglu": (H, Wd, off, dy, H2, H3),
        "bwd_grouped_gemm_dW_dX2": (pX, Wu, Wv, off, H, H2),
        "route_topk": (logits, k),
        "route_topk_count": (logits, k, X),
        "route_topk_backward": (w, topk, dgt, E),
        "dispatch_tokens": (X, w, topk, E),
        "combine_inv": (pX, inv, pw, torch.bfloat16),
        "combine_backward_inv": (pX, inv, pw, dYt),
        "pack_backward_inv": (pX, pw, inv),
        "pack_backward_inv_route": (pX, pw, inv, w, topk, E),
    }


@pytest.mark.parametrize("name", sorted(_cases()))
def test_meta_kernels_match_cpu_shapes(ops, name):
    args = _cases()[name]
    cpu = getattr(ops, name)(*args)
    meta = getattr(ops, name)(*[_meta(a) for a in _cases()[name]])
    cpu = cpu if isinstance(cpu, tuple) else (cpu,)
    meta = meta if isinstance(meta, tuple) else (meta,)
    assert len(cpu) == len(meta)
    for c, m in zip(cpu, meta):
        assert m.device.type == "meta"
        assert c.shape == m.shape and c.dtype == m.dtype, name


@pytest.mark.parametrize("name", ["count_expert_kernel", "pack_tokens_kernel", "dispatch_tokens",
                                  "combine_tokens_kernel", "grouped_gemm_kernel", "combine_inv",
                                  "route_topk", "bwd_grouped_gemm_dW_dX"])
def test_opcheck(ops, name):
    """Schema, fake-tensor and mutation checks of torch.library.opcheck."""
    op = getattr(torch.ops.nanotitan, name).default
    torch.library.opcheck(op, _cases()[name],
                          test_utils=("test_schema", "test_faketensor"))


def test_opcheck_counted_dispatch(ops):
    """The counted dispatch's schema marks its workspace mutable (the HIP
    kernel writes scratch after the router's counts); opcheck's schema and
    fake-tensor checks agree with the CPU kernel."""
    a = _cases()
    X, w, topk, E = a["dispatch_tokens"]
    logits, k = a["route_topk"]
    g, i, ws = ops.route_topk_count(logits, k, X)
    torch.library.opcheck(torch.ops.nanotitan.dispatch_tokens_counted.default, (X, g, i, E, ws),
                          test_utils=("test_schema", "test_faketensor"))
    sch = torch.ops.nanotitan.dispatch_tokens_counted.default._schema
    assert sch.arguments[4].alias_info is not None and sch.arguments[4].alias_info.is_write


def test_cpu_ops_check_arguments_like_the_gpu_ops(ops):
    """Same TORCH_CHECK conditions (and messages) as the HIP surface."""
    T, k, d = 16, 2, 8
    inv = torch.arange(T * k, dtype=torch.int32).view(T, k)
    y, w = torch.randn(T * k, d), torch.rand(T * k)
    with pytest.raises(RuntimeError, match=r"inv\.numel\(\)"):
        ops.combine_inv(y[:-1].contiguous(), inv, w, torch.float32)
    with pytest.raises(RuntimeError, match=r"inv\.numel\(\)"):
        ops.pack_backward_inv(y, w[:-1].contiguous(), inv)
    with pytest.raises(RuntimeError, match="float32"):
        ops.combine_kernel_backward(y, torch.zeros(T * k, dtype=torch.int32), w,
                                    torch.zeros(T, d, dtype=torch.float16), d)
    with pytest.raises(RuntimeError, match="contiguous"):
        ops.combine_tokens_kernel(y.t(), torch.zeros(d, dtype=torch.int32), torch.ones(d), T, T * k)
    with pytest.raises(RuntimeError, match="top_k"):
        ops.route_topk(torch.randn(4, 3), 4)
