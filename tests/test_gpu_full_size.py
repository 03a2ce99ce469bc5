"""GPU parity at the configs' full sizes (C1-C5), where the CPU oracle cannot
run the whole problem in seconds. Every check rests on a property that holds
at any size, so the oracle only ever sees a small part of the problem:

- Integer work (routing, counts, offsets) is compared bit for bit over all
  tokens.
- Row independence of the layer: a token's output, its input gradient and its
  router-logit gradient depend only on that token's x, logits and dY (and the
  weights). The oracle's torch path runs on a seeded sample of tokens (with
  the least-loaded experts' tokens and, at C5, tied-logit tokens included) and
  the full-size GPU results must match at those tokens.
- Row and column independence of a grouped GEMM: forward and dX rows depend
  only on their own input row and expert; a dW column depends on one column of
  dOut over the expert's whole segment. The expert-GEMM chain the layer runs
  (fused GELU up-projection, down-projection, paired dW + GELU-backward dX,
  paired dW + dX) is checked stage by stage on sampled rows of every live
  expert and on sampled dW columns (full reductions), in float64, each stage
  fed the GPU's own output of the stage before.

Tolerances are the other GPU tests': fp32 1e-4, fp16 1e-2, bf16 2e-2
(absolute scaled by the square root of the reduction where values grow
with it).
"""

import pytest
import torch

from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu

TOL = {
    torch.float32: dict(rtol=1e-4, atol=1e-4),
    torch.float16: dict(rtol=1e-2, atol=1e-2),
    torch.bfloat16: dict(rtol=2e-2, atol=2e-2),
}


def _close(got, want, dtype, scale=1.0):
    """got (a dtype tensor) vs the float64 value rounded to dtype."""
    tol = dict(TOL[dtype])
    tol["atol"] *= scale
    torch.testing.assert_close(got.double(), want.to(dtype).double(), **tol)


def _gelu_grad(x):
    x = x.double()
    return 0.5 * (1 + torch.erf(x / 2 ** 0.5)) + x * torch.exp(-0.5 * x * x) / (2 * torch.pi) ** 0.5


def _cuda_weights(c, seed, n=2):
    """n = 2: W_up [E,d,f], W_down [E,f,d]; n = 3: W_gate, W_val [E,d,f], W_out [E,f,d]."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    shapes = [(c.E, c.d, c.f)] * (n - 1) + [(c.E, c.f, c.d)]
    return [(torch.randn(*s, generator=g, device="cuda") * c.w_std).to(c.dtype) for s in shapes]


def _sample_tokens(idx, logits, E, seed, n=32):
    """Seeded random tokens, the first and last, one token of each of the 8
    least-loaded live experts, and up to 8 tokens whose finite logits are tied."""
    T = idx.shape[0]
    g = torch.Generator().manual_seed(seed)
    pick = set(torch.randperm(T, generator=g)[:n].tolist()) | {0, T - 1}
    counts = torch.bincount(idx.reshape(-1).long(), minlength=E)
    live = [e for e in range(E) if counts[e] > 0]
    for e in sorted(live, key=lambda e: int(counts[e]))[:8]:
        pick.add(int((idx == e).any(dim=1).nonzero()[0, 0]))
    fin = torch.where(torch.isfinite(logits), logits, torch.nan)
    tied = (fin.nan_to_num(float("inf")).amin(1) == fin.nan_to_num(float("-inf")).amax(1))
    pick |= set(tied.nonzero().reshape(-1)[:8].tolist())
    return torch.tensor(sorted(pick), dtype=torch.long)


@pytest.mark.parametrize("cfg_id,ffn", [(1, "gelu"), (2, "gelu"), (3, "gelu"), (4, "gelu"),
                                        (5, "gelu"), (2, "swiglu"), (3, "swiglu"), (4, "swiglu"),
                                        (5, "swiglu")])
def test_layer_full_size_sampled_tokens(ext, cfg_id, ffn):
    """The layer forward + backward at the config's full token count (the
    benchmark's path: router with fused count, dispatch, fused expert FFN,
    combine), vs the oracle's torch path on a sample of tokens. GELU is the
    configs' FFN; SwiGLU is the reference's ExpertFFN at the configs' widths."""
    from nanotitan_amd.layer import moe_forward_from_logits
    from nanotitan_amd.moe_ops import grouped_gelu_ffn_fn, swiglu_ffn_fn

    d = O.make_inputs(cfg_id, with_weights=False)
    c = d["cfg"]
    names = ["up", "down"] if ffn == "gelu" else ["gate", "val", "out"]
    W = dict(zip(names, _cuda_weights(c, 7000 + cfg_id, len(names))))

    class FFN(torch.nn.Module):
        def forward(self, px, off):
            if ffn == "gelu":
                return grouped_gelu_ffn_fn(px, W["up"], W["down"], off)
            return swiglu_ffn_fn(px, W["gate"], W["val"], W["out"], off)

    x = d["X"].to(c.dtype).cuda().requires_grad_(True)
    logits = d["logits"].cuda().requires_grad_(True)
    out, counts, _ = moe_forward_from_logits(x, logits, FFN(), c.E, c.k)
    out.backward(d["dY"].to(c.dtype).cuda())
    torch.cuda.synchronize()

    # Integer work over every token.
    _, idx, _ = O.route(d["logits"], c.k)
    assert counts.cpu().long().tolist() == O.count_experts(idx, None, c.E).tolist()
    assert int(counts.sum()) == c.T * c.k
    assert bool(torch.isfinite(out).all()) and bool(torch.isfinite(x.grad).all())

    S = _sample_tokens(idx, d["logits"], c.E, seed=cfg_id)
    weights = {n: w.cpu() for n, w in W.items()}
    ref_out, ref = O.moe_layer_torch(d["X"][S].to(c.dtype), d["logits"][S], weights, c.k,
                                     ffn=ffn, dY=d["dY"][S].to(c.dtype))
    tol = dict(rtol=1e-4, atol=1e-4) if c.dtype == torch.float32 else dict(rtol=2e-2, atol=2e-2)
    torch.testing.assert_close(out.detach()[S.cuda()].cpu().float(), ref_out.float(), **tol)
    torch.testing.assert_close(x.grad[S.cuda()].cpu().float(), ref["x"].float(), **tol)
    torch.testing.assert_close(logits.grad[S.cuda()].cpu().float(), ref["logits"].float(),
                               rtol=tol["rtol"], atol=tol["atol"] / 10)


def _sample_rows(off, seed, per=4):
    """(expert, row) pairs: first and last row of every live expert plus
    `per` - 2 seeded rows inside it."""
    g = torch.Generator().manual_seed(seed)
    rows = []
    for e in range(len(off) - 1):
        a, b = int(off[e]), int(off[e + 1])
        if b <= a:
            continue
        r = {a, b - 1} | set((a + torch.randint(0, b - a, (per - 2,), generator=g)).tolist())
        rows += [(e, x) for x in sorted(r)]
    return rows


def _rows_times(rows, L, W, transpose=False):
    """float64 L[row] @ W[e] (or W[e]^T) for the sampled (expert, row) pairs."""
    out = []
    for e in sorted({e for e, _ in rows}):
        rs = [r for ee, r in rows if ee == e]
        w = W[e].double()
        out.append(L[rs].double() @ (w.T if transpose else w))
    return torch.cat(out)


def _dw_cols(L, R, off, cols, E):
    """float64 dW[:, :, cols] = L_e^T R_e[:, cols] over each expert's full segment."""
    out = torch.zeros(E, L.shape[1], len(cols), dtype=torch.float64)
    for e in range(E):
        a, b = int(off[e]), int(off[e + 1])
        if b > a:
            out[e] = L[a:b].double().T @ R[a:b, cols].double()
    return out


@pytest.mark.parametrize("cfg_id", [1, 2, 3, 4, 5])
def test_expert_gemm_chain_full_size(ext, cfg_id):
    """The four expert-GEMM calls of the GELU FFN at the config's full routed
    segment sizes, checked stage by stage on sampled rows and dW columns."""
    c = O.CONFIGS[cfg_id]
    d = O.make_inputs(cfg_id, with_weights=False)
    _, idx, _ = O.route(d["logits"], c.k)
    off = O.offsets_from_counts(O.count_experts(idx, None, c.E))
    A = c.T * c.k
    og = torch.from_numpy(off).to(torch.int32).cuda()
    g = torch.Generator(device="cuda").manual_seed(8000 + cfg_id)
    X = torch.randn(A, c.d, generator=g, device="cuda").to(c.dtype)
    dy = torch.randn(A, c.d, generator=g, device="cuda").to(c.dtype)
    W_up, W_down = _cuda_weights(c, 9000 + cfg_id)

    a, gg = ext.grouped_gemm_gelu(X, og, W_up)
    y = ext.grouped_gemm_kernel(a, og, W_down)
    dW_down, dH = ext.bwd_grouped_gemm_dW_dX_gelu(a, W_down, og, dy, gg)
    dW_up, dX = ext.bwd_grouped_gemm_dW_dX(X, W_up, og, dH)
    # The paired calls return exactly what the separate calls return.
    assert torch.equal(dW_down, ext.bwd_grouped_gemm_dW_kernel(a, og, dy))
    assert torch.equal(dH, ext.bwd_grouped_gemm_dX_gelu(W_down, og, dy, gg))
    assert torch.equal(dW_up, ext.bwd_grouped_gemm_dW_kernel(X, og, dH))
    assert torch.equal(dX, ext.bwd_grouped_gemm_dX_kernel(W_up, og, dH))
    torch.cuda.synchronize()

    rows = _sample_rows(off, seed=cfg_id)
    R = torch.tensor([r for _, r in rows], dtype=torch.long)
    Rg = R.cuda()
    Xh, dyh, ah, gh, dHh = (t[Rg].cpu() for t in (X, dy, a, gg, dH))
    Wu, Wd = W_up.cpu(), W_down.cpu()
    dt = c.dtype
    # up-projection with GELU: gelu and gelu' of the rounded h, each rounded once
    Xs = {r: i for i, r in enumerate(R.tolist())}
    h = _rows_times(rows, _Rows(Xh, Xs), Wu).to(dt)
    _close(ah, O.gelu(h.double()), dt)
    _close(gh, _gelu_grad(h), dt)
    # down-projection
    _close(y[Rg].cpu(), _rows_times(rows, _Rows(ah, Xs), Wd), dt, scale=(c.f / 512) ** 0.5)
    # GELU backward dX: round(dy @ W_down^T) * gelu'(h), rounded
    dA = _rows_times(rows, _Rows(dyh, Xs), Wd, transpose=True).to(dt).double()
    _close(dHh, dA * gh.double(), dt)
    # up-projection dX
    _close(dX[Rg].cpu(), _rows_times(rows, _Rows(dHh, Xs), Wu, transpose=True), dt,
           scale=(c.f / 512) ** 0.5)
    # dW columns (full reductions over each expert's segment)
    gen = torch.Generator().manual_seed(cfg_id)
    cols_d = sorted({0, c.d - 1, min(255, c.d - 1)}
                    | set(torch.randint(0, c.d, (5,), generator=gen).tolist()))
    cols_f = sorted({0, c.f - 1, min(256, c.f - 1)}
                    | set(torch.randint(0, c.f, (5,), generator=gen).tolist()))
    cd, cf = torch.tensor(cols_d), torch.tensor(cols_f)
    mmax = max(int(off[e + 1] - off[e]) for e in range(c.E))
    ref_dWd = _dw_cols(a.cpu(), dy[:, cd.cuda()].cpu(), off, list(range(len(cols_d))), c.E)
    _close(dW_down[:, :, cd.cuda()].cpu(), ref_dWd, dt, scale=max(mmax / 512, 1.0) ** 0.5)
    ref_dWu = _dw_cols(X.cpu(), dH[:, cf.cuda()].cpu(), off, list(range(len(cols_f))), c.E)
    _close(dW_up[:, :, cf.cuda()].cpu(), ref_dWu, dt, scale=max(mmax / 512, 1.0) ** 0.5)


class _Rows:
    """Row lookup of a gathered sample by original row index."""

    def __init__(self, data, pos):
        self.data, self.pos = data, pos

    def __getitem__(self, rows):
        return self.data[[self.pos[r] for r in rows]]


def _boundary_ties(logits, k):
    """C5's second tie variant: each row's (k+1)-th largest logit is set to
    its k-th largest (where that is finite), so the top-k boundary is a tie
    that only the lower-expert-id rule resolves."""
    z = logits.clone()
    order = torch.sort(z, dim=1, descending=True, stable=True).indices
    kth = z.gather(1, order[:, k - 1:k])
    ok = torch.isfinite(kth).squeeze(1)
    rows = ok.nonzero().squeeze(1)
    z[rows, order[rows, k]] = kth[rows, 0]
    return z


def test_c5_boundary_ties_full_size_bit_exact_and_repeatable(ext):
    """C5 at full size with the boundary-tie variant: top-k indices bit-exact
    against the stable sort (ties to the lower id) over all 65536 tokens, the
    layer's output and gradients bit-identical across two runs, and the output
    equal to the oracle's torch path on sampled tokens."""
    from nanotitan_amd.layer import moe_forward_from_logits
    from nanotitan_amd.moe_ops import grouped_gelu_ffn_fn, route_fn

    d = O.make_inputs(5, with_weights=False)
    c = d["cfg"]
    logits = _boundary_ties(d["logits"], c.k)
    order = torch.sort(logits, dim=1, descending=True, stable=True).indices
    assert bool((logits.gather(1, order[:, c.k - 1:c.k]) == logits.gather(1, order[:, c.k:c.k + 1]))
                .all())
    _, want_idx, _ = O.route(logits, c.k)
    _, idx = route_fn(logits.cuda(), c.k)
    assert torch.equal(idx.cpu(), want_idx)

    W = _cuda_weights(c, 7105)

    class FFN(torch.nn.Module):
        def forward(self, px, off):
            return grouped_gelu_ffn_fn(px, W[0], W[1], off)

    runs = []
    for _ in range(2):
        x = d["X"].to(c.dtype).cuda().requires_grad_(True)
        lg = logits.cuda().requires_grad_(True)
        out, counts, _ = moe_forward_from_logits(x, lg, FFN(), c.E, c.k)
        out.backward(d["dY"].to(c.dtype).cuda())
        torch.cuda.synchronize()
        runs.append((out.detach().view(torch.int16).cpu(), x.grad.view(torch.int16).cpu(),
                     lg.grad.cpu(), counts.cpu()))
    for a, b in zip(*runs):
        assert torch.equal(a, b)
    assert runs[0][3].long().tolist() == O.count_experts(want_idx, None, c.E).tolist()

    S = _sample_tokens(want_idx, logits, c.E, seed=55)
    weights = {"up": W[0].cpu(), "down": W[1].cpu()}
    ref_out, ref = O.moe_layer_torch(d["X"][S].to(c.dtype), logits[S], weights, c.k, ffn="gelu",
                                     dY=d["dY"][S].to(c.dtype))
    out16 = runs[0][0].view(c.dtype)
    torch.testing.assert_close(out16[S].float(), ref_out.float(), rtol=2e-2, atol=2e-2)
    torch.testing.assert_close(runs[0][1].view(c.dtype)[S].float(), ref["x"].float(), rtol=2e-2,
                               atol=2e-2)


@pytest.mark.parametrize("cfg_id", [4, 5])
def test_dispatch_full_width_bit_exact(ext, cfg_id):
    """The dispatch at C4 and C5 in full: every token at its real row width
    (4096 bf16 / 2048 fp16 columns, the long-row pack kernel), through the
    layer's path (router with fused count, counted dispatch) and the plain
    dispatch. Bit for bit over all rows: counts = bincount, offsets = their
    exclusive scan, token_id / expert / inv = the oracle's stable counting
    sort (the permutation alone: the oracle gets one column), packed rows
    = torch's gather X[token_id] on the GPU, packed gates = w[t, slot], and
    token_id / inv inverse maps of each other."""
    import numpy as np

    d = O.make_inputs(cfg_id, with_weights=False)
    c = d["cfg"]
    X = d["X"].to(c.dtype)
    T, k, E = X.shape[0], c.k, c.E
    print(f"[full-width dispatch] C{cfg_id} T={T} d={X.shape[1]} E={E} k={k}", flush=True)
    want_g, want_i, _ = O.route(d["logits"], k)
    counts, offsets, p = O.dispatch(X[:, :1].contiguous(), want_g, want_i, E)
    Xg = X.cuda()
    g, i, ws = ext.route_topk_count(d["logits"].cuda(), k, Xg)
    assert torch.equal(i.cpu(), want_i)
    runs = {"counted": ext.dispatch_tokens_counted(Xg, g, i, E, ws),
            "plain": ext.dispatch_tokens(Xg, g, i, E)}
    for name, (g_counts, g_off, g_px, g_tid, g_ex, g_pw, g_inv) in runs.items():
        torch.cuda.synchronize()
        assert np.array_equal(g_counts.cpu().numpy(), counts), name
        assert np.array_equal(g_off.cpu().numpy(), offsets), name
        assert np.array_equal(g_tid.cpu().numpy(), p.token_id), name
        assert np.array_equal(g_ex.cpu().numpy(), p.expert), name
        assert np.array_equal(g_inv.cpu().numpy(), p.inv), name
        A = T * k
        assert g_px.shape == (A, X.shape[1])
        gathered = Xg.index_select(0, g_tid.long())
        assert torch.equal(g_px.view(torch.int16), gathered.view(torch.int16)), name
        del gathered
        flat_inv = g_inv.reshape(-1).long()
        assert torch.equal(g_pw[flat_inv], g.reshape(-1)), name  # gate of assignment (t, j)
        t_of = torch.arange(T, device="cuda").repeat_interleave(k)
        assert torch.equal(g_tid[flat_inv].long(), t_of), name  # token_id o inv = identity
        assert torch.equal(g_ex[flat_inv], i.reshape(-1)), name
        assert torch.equal(torch.sort(flat_inv).values, torch.arange(A, device="cuda")), name
    del runs
    torch.cuda.empty_cache()
