"""CPU oracle for the nanoTitan MoE expert path — TEST INFRASTRUCTURE ONLY.

This module restates, on the CPU, what the reference computes on the hot
path. Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import it, and only as the checker (or, for the CPU
baseline, as the timed reference path). The product (``nanotitan_amd``)
never imports it and has no CPU fallback.

Integer and byte work (counts, offsets, packed order, gathers) is numpy;
floating-point sums whose order matters are written as explicit ordered
numpy operations; dtype casts use torch's CPU casts (round to nearest even).

Every function cites the reference file:line it follows (paths relative to
the nanoTitan tree). Pinning — what checks each function against something
other than itself — is listed in PINNING below and exercised by
tests/test_oracle.py:

* count_experts / offsets_from_counts / pack_tokens: reference known-answer
  test (tests/test_packing.py:14-76, as tests/golden/pack_kat.json), the
  reference pack invariants (benchmarks/bench_pack_tokens.py:176-223),
  brute-force Python loops on small inputs, numpy bincount closed form.
* combine_tokens: reference KATs (tests/test_combine.py:12-90, as
  tests/golden/combine_kat.json), torch.index_add_ (a library scatter-add,
  tests/test_combine_bwd.py:48-53), float64 sum bound.
* combine_backward / pack_backward: torch.autograd of the reference test
  formulas (tests/test_combine_bwd.py:48-53, tests/test_pack_bwd.py:41-44).
* grouped_gemm / _dx / _dw: torch.autograd of the reference test formula
  (tests/test_grouped_gemm.py:42-48), float64.
* moe_layer: a token-by-token dense restatement (every token runs its own
  k experts) with torch.autograd gradients.
* route: the stable top-k rule checked against brute-force sorting.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

PINNING = {
    "count_experts": "golden pack_kat + bincount closed form + brute force",
    "offsets_from_counts": "golden pack_kat + closed form",
    "pack_tokens": "golden pack_kat + reference invariants + brute force",
    "combine_tokens": "golden combine_kat + torch.index_add_ + float64 bound",
    "combine_backward": "torch.autograd of reference test formula",
    "pack_backward": "torch.autograd of reference test formula + brute force first-match",
    "grouped_gemm": "torch.autograd of reference test formula (float64)",
    "grouped_gemm_dx": "torch.autograd of reference test formula (float64)",
    "grouped_gemm_dw": "torch.autograd of reference test formula (float64)",
    "route": "brute-force sort with explicit tie rule + torch softmax/renorm",
    "moe_layer": "token-by-token dense restatement + torch.autograd",
}


def _np(t) -> np.ndarray:
    if isinstance(t, np.ndarray):
        return t
    if not isinstance(t, torch.Tensor):
        return np.asarray(t)
    t = t.detach().cpu()
    if t.dtype in (torch.bfloat16, torch.float16):
        t = t.float()
    return t.numpy()


# ----------------------------------------------------------------- dispatch


def count_experts(topk, mask, num_experts: int) -> np.ndarray:
    """count[e] = #{(t,j): mask[t] != 0 and topk[t,j] == e}; ids outside [0,E) ignored.

    Reference: csrc/kernels/count_experts.cu:8-29 (one thread per token,
    atomicAdd per slot, mask honoured at :20).
    """
    topk = _np(topk).astype(np.int64)
    T = topk.shape[0]
    keep = np.ones(T, dtype=bool) if mask is None else (_np(mask) != 0)
    ids = topk[keep].reshape(-1)
    ids = ids[(ids >= 0) & (ids < num_experts)]
    return np.bincount(ids, minlength=num_experts).astype(np.int32)


def offsets_from_counts(counts) -> np.ndarray:
    """offsets[0] = 0, offsets[1:] = cumsum(counts) (reference src/model/cuda_backend.py:54-58)."""
    counts = _np(counts).astype(np.int64)
    return np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)


@dataclass
class Packed:
    packed_X: torch.Tensor  # [A, d] in X's dtype
    token_id: np.ndarray  # [A] int32
    expert: np.ndarray  # [A] int32
    packed_w: np.ndarray  # [A] float32
    inv: np.ndarray  # [T, k] int32 (-1 for dropped assignments)
    cursor_after: np.ndarray  # [E+1] int32
    written: np.ndarray  # [A] bool: slot written by some assignment


def pack_tokens(X: torch.Tensor, topk_weights, topk_experts, cursor) -> Packed:
    """Canonical pack: slot(f) = cursor[e] + #{f' < f : topk.flat[f'] == e}.

    Reference: csrc/kernels/pack_tokens.cu:8-48 (scatter each (token, slot)
    to a slot claimed from the per-expert cursor, copy the row; cursor ends
    at cursor[e] + count[e]) with the in-segment order of the torch backend,
    src/model/torch_backend.py:58-66 (argwhere enumerates (t, j) row-major per
    expert). Assignments whose id is outside [0, E) or whose slot falls
    outside [0, A) are dropped.
    """
    topk = _np(topk_experts).astype(np.int64)
    w = _np(topk_weights).astype(np.float32)
    cur = _np(cursor).astype(np.int64).copy()
    T, k = topk.shape
    A = T * k
    E = cur.shape[0] - 1
    flat = topk.reshape(-1)
    valid = (flat >= 0) & (flat < E)
    order = np.argsort(np.where(valid, flat, E), kind="stable")
    order = order[valid[order]]
    e_sorted = flat[order]
    # rank of each assignment among same-expert assignments, in flat order
    seg_start = np.searchsorted(e_sorted, e_sorted, side="left")
    rank = np.arange(order.size) - seg_start
    slot = cur[e_sorted] + rank
    ok = (slot >= 0) & (slot < A)
    inv = np.full(A, -1, dtype=np.int64)
    inv[order[ok]] = slot[ok]
    counts = np.bincount(e_sorted, minlength=E)
    cur_after = cur.copy()
    cur_after[:E] += counts

    token_id = np.zeros(A, dtype=np.int32)
    expert = np.zeros(A, dtype=np.int32)
    packed_w = np.zeros(A, dtype=np.float32)
    written = np.zeros(A, dtype=bool)
    f_ok = order[ok]
    s_ok = slot[ok]
    token_id[s_ok] = (f_ok // k).astype(np.int32)
    expert[s_ok] = flat[f_ok].astype(np.int32)
    packed_w[s_ok] = w.reshape(-1)[f_ok]
    written[s_ok] = True
    Xc = X.detach().cpu()
    packed_X = torch.zeros((A, Xc.shape[1]), dtype=Xc.dtype)
    packed_X[torch.from_numpy(s_ok)] = Xc[torch.from_numpy(f_ok // k)]
    return Packed(packed_X, token_id, expert, packed_w, inv.reshape(T, k).astype(np.int32),
                  cur_after.astype(np.int32), written)


def dispatch(X: torch.Tensor, topk_weights, topk_experts, num_experts: int):
    """Fused count + offsets + pack (reference src/model/cuda_backend.py:46-67)."""
    counts = count_experts(topk_experts, None, num_experts)
    offsets = offsets_from_counts(counts)
    packed = pack_tokens(X, topk_weights, topk_experts, offsets)
    return counts, offsets, packed


# ------------------------------------------------------------------ combine


def combine_tokens(y, token_id, w, num_tokens: int) -> np.ndarray:
    """out[t] = sum over p with token_id[p] == t, ascending p, of fl32(w[p] * y[p]).

    Reference: csrc/kernels/combine_kernels.cu:8-34 (fp32 accumulation of
    weight * float(value)); the fixed ascending order is the order of a
    sequential index_add_ (tests/test_combine_bwd.py:48-53). np.add.at
    applies its updates one index at a time in order, in float32.
    """
    y = _np(y).astype(np.float32)
    tid = _np(token_id).astype(np.int64)
    w = _np(w).astype(np.float32)
    out = np.zeros((num_tokens, y.shape[1]), dtype=np.float32)
    ok = (tid >= 0) & (tid < num_tokens)
    prod = (w[:, None] * y).astype(np.float32)
    np.add.at(out, tid[ok], prod[ok])
    return out


def combine_backward(y, token_id, w, dY, out_dtype=torch.float32):
    """dy[p] = cast(fl32(dY[t] * w[p])), dw[p] = sum_h dY[t,h] * y[p,h] (float64 sum).

    Reference: csrc/kernels/backward_combine_kernel.cu:8-40.
    """
    yf = _np(y).astype(np.float32)
    tid = _np(token_id).astype(np.int64)
    w = _np(w).astype(np.float32)
    g = _np(dY).astype(np.float32)
    T = g.shape[0]
    ok = (tid >= 0) & (tid < T)
    rows = np.zeros_like(yf)
    rows[ok] = g[tid[ok]]
    dy32 = (rows * w[:, None]).astype(np.float32)
    dw = (rows.astype(np.float64) * yf.astype(np.float64)).sum(axis=1).astype(np.float32)
    return torch.from_numpy(dy32).to(out_dtype), dw


def pack_backward(dpX, dpw, token_id, expert, topk, out_dtype=torch.float32):
    """dX[t] = cast(sum over rows p of token t, ascending p, of dpX[p]) (float32 adds);
    dw[t, j] += dpw[p] for the first slot j with topk[t, j] == expert[p].

    Reference: csrc/kernels/backward_pack_kernel.cu:10-44 (the reference adds
    into dX with dtype atomics in arbitrary order; this is the fp32 ordered
    sum it approximates).
    """
    x = _np(dpX).astype(np.float32)
    dpw = _np(dpw).astype(np.float32)
    tid = _np(token_id).astype(np.int64)
    ex = _np(expert).astype(np.int64)
    tk = _np(topk).astype(np.int64)
    T, k = tk.shape
    dX = np.zeros((T, x.shape[1]), dtype=np.float32)
    ok = (tid >= 0) & (tid < T)
    np.add.at(dX, tid[ok], x[ok])
    dw = np.zeros((T, k), dtype=np.float32)
    p_ok = np.nonzero(ok)[0]
    if p_ok.size:
        t_p = tid[p_ok]
        match = tk[t_p] == ex[p_ok][:, None]  # [n, k]
        has = match.any(axis=1)
        first = match.argmax(axis=1)
        sel = p_ok[has]
        np.add.at(dw, (t_p[has], first[has]), dpw[sel])
    return torch.from_numpy(dX).to(out_dtype), dw


# ------------------------------------------------------------- grouped GEMM


def _segments(offsets, A):
    off = _np(offsets).astype(np.int64)
    E = off.shape[0] - 1
    for e in range(E):
        a = min(max(int(off[e]), 0), A)
        b = min(max(int(off[e + 1]), a), A)
        yield e, a, b


def grouped_gemm(X, offsets, W) -> torch.Tensor:
    """out[a] = X[a] @ W[e] for rows a of expert e, float64 (rows past offsets[E]: 0).

    Reference: csrc/kernels/grouped_gemm.cu:12-40.
    """
    X64 = X.detach().cpu().double()
    W64 = W.detach().cpu().double()
    A = X64.shape[0]
    out = torch.zeros((A, W64.shape[2]), dtype=torch.float64)
    for e, a, b in _segments(offsets, A):
        if b > a:
            out[a:b] = X64[a:b] @ W64[e]
    return out


def grouped_gemm_dx(W, offsets, dOut) -> torch.Tensor:
    """dX[a] = dOut[a] @ W[e]^T, float64. Reference: csrc/kernels/bwd_grouped_gemm_dX.cu:13-44."""
    W64 = W.detach().cpu().double()
    G = dOut.detach().cpu().double()
    A = G.shape[0]
    out = torch.zeros((A, W64.shape[1]), dtype=torch.float64)
    for e, a, b in _segments(offsets, A):
        if b > a:
            out[a:b] = G[a:b] @ W64[e].T
    return out


def grouped_gemm_dw(X, offsets, dOut) -> torch.Tensor:
    """dW[e] = X_e^T @ dOut_e (zero for an empty expert), float64.

    Reference: csrc/kernels/bwd_grouped_gemm_dW.cu:11-40.
    """
    X64 = X.detach().cpu().double()
    G = dOut.detach().cpu().double()
    A = X64.shape[0]
    E = _np(offsets).shape[0] - 1
    out = torch.zeros((E, X64.shape[1], G.shape[1]), dtype=torch.float64)
    for e, a, b in _segments(offsets, A):
        if b > a:
            out[e] = X64[a:b].T @ G[a:b]
    return out


# ------------------------------------------------------------------ routing


def select_topk(logits: torch.Tensor, top_k: int) -> torch.Tensor:
    """Indices of the k largest logits per row, ties to the lower expert id.

    The k largest logits are the k largest softmax probabilities (softmax is
    monotonic); comparing logits avoids ties created by rounding the
    probabilities. torch.topk, used by the reference
    (src/model/cuda_backend.py:34), leaves the order of ties unspecified.
    """
    _, idx = torch.sort(logits.float(), dim=-1, descending=True, stable=True)
    return idx[:, :top_k]


def route(logits: torch.Tensor, top_k: int):
    """(gates f32 [T,k], ids int32 [T,k], probs f32 [T,E]).

    Reference: src/model/cuda_backend.py:30-37 (fp32 softmax, top-k,
    gates = p_topk / sum p_topk). The renormalised gates equal the softmax of
    the selected logits; computed here in float64 and rounded.
    """
    probs = logits.float().softmax(dim=-1)
    idx = select_topk(logits, top_k)
    sel = torch.gather(logits.double(), 1, idx)
    gates = sel.softmax(dim=-1).float()
    return gates, idx.to(torch.int32), probs


# ------------------------------------------------------------- MoE layer


def gelu(x):
    return torch.nn.functional.gelu(x)  # erf form


def moe_layer_torch(x, logits, weights, top_k, ffn="gelu", dY=None):
    """torch-CPU restatement of the reference's torch MoE path with ep_size=1.

    Reference: src/model/torch_backend.py:24-71 (argwhere pack per expert),
    :149-151 (index_add_ combine; accumulated here in float32 per the
    CUDA backend, csrc/kernels/combine_kernels.cu:32), and
    src/model/feed_fwd.py:80-100 (per-expert matmuls; SwiGLU) or the
    configs' GELU FFN (up, GELU, down). Runs forward and, when dY is given,
    backward through autograd. Returns (out, grads dict).

    ``weights`` is a dict: gelu -> {"up": [E,d,f], "down": [E,f,d]};
    swiglu -> {"gate": [E,d,f], "val": [E,d,f], "out": [E,f,d]}.
    """
    x = x.detach().clone().requires_grad_(True)
    logits = logits.detach().clone().requires_grad_(True)
    params = {n: w.detach().clone().requires_grad_(True) for n, w in weights.items()}
    T, d = x.shape
    E = logits.shape[1]
    probs = logits.float().softmax(dim=-1)
    idx = select_topk(logits, top_k)
    vals = torch.gather(probs, 1, idx)
    gates = vals / vals.sum(dim=-1, keepdim=True)
    counts = torch.bincount(idx.reshape(-1), minlength=E)
    offsets = torch.zeros(E + 1, dtype=torch.long)
    offsets[1:] = torch.cumsum(counts, 0)
    A = T * top_k
    packed_X = torch.empty((A, d), dtype=x.dtype)
    token_ids = torch.empty(A, dtype=torch.long)
    packed_w = torch.empty(A, dtype=torch.float32)
    for e in range(E):
        ind = torch.argwhere(idx == e)
        if ind.numel() == 0:
            continue
        s, t = int(offsets[e]), int(offsets[e + 1])
        packed_X[s:t] = x[ind[:, 0]]
        token_ids[s:t] = ind[:, 0]
        packed_w[s:t] = gates[ind[:, 0], ind[:, 1]]
    out_rows = torch.empty((A, d), dtype=x.dtype)
    for e in range(E):
        s, t = int(offsets[e]), int(offsets[e + 1])
        if t == s:
            continue
        xe = packed_X[s:t]
        if ffn == "gelu":
            h = gelu(xe @ params["up"][e])
            out_rows[s:t] = h @ params["down"][e]
        else:
            h = torch.nn.functional.silu(xe @ params["gate"][e]) * (xe @ params["val"][e])
            out_rows[s:t] = h @ params["out"][e]
    pool = torch.zeros((T, d), dtype=torch.float32)
    pool = pool.index_add(0, token_ids, out_rows.float() * packed_w[:, None])
    out = pool.to(x.dtype)
    grads = {}
    if dY is not None:
        out.backward(dY.to(out.dtype))
        grads = {"x": x.grad, "logits": logits.grad}
        grads.update({n: p.grad for n, p in params.items()})
    return out.detach(), grads


def moe_layer_dense(x, logits, weights, top_k, ffn="gelu"):
    """Token-by-token restatement in float64: out[t] = sum_j gate[t,j] FFN_{e_tj}(x[t]).

    An independent formulation (no packing, no segments) used to pin
    moe_layer_torch; differentiable through torch.autograd.
    """
    probs = logits.double().softmax(dim=-1)
    idx = select_topk(logits.detach(), top_k)
    vals = torch.gather(probs, 1, idx)
    gates = vals / vals.sum(dim=-1, keepdim=True)
    xd = x.double()
    rows = []
    for t in range(x.shape[0]):
        acc = torch.zeros(x.shape[1], dtype=torch.float64)
        for j in range(top_k):
            e = int(idx[t, j])
            if ffn == "gelu":
                h = gelu(xd[t] @ weights["up"][e].double()) @ weights["down"][e].double()
            else:
                gt = torch.nn.functional.silu(xd[t] @ weights["gate"][e].double())
                h = (gt * (xd[t] @ weights["val"][e].double())) @ weights["out"][e].double()
            acc = acc + gates[t, j] * h
        rows.append(acc)
    return torch.stack(rows)


# --------------------------------------------------------- synthetic inputs

CONFIG_SEEDS = {1: 1001, 2: 1002, 3: 1003, 4: 1004, 5: 1005}


@dataclass
class MoEConfigShape:
    name: str
    dtype: torch.dtype
    T: int
    d: int
    E: int
    k: int
    f: int
    w_std: float
    logit_std: float = 1.0


CONFIGS = {
    1: MoEConfigShape("C1", torch.float32, 4096, 512, 8, 2, 2048, 0.02),
    2: MoEConfigShape("C2", torch.bfloat16, 30720, 512, 8, 2, 2048, 0.02),
    3: MoEConfigShape("C3", torch.bfloat16, 30720, 512, 64, 8, 256, 0.02),
    4: MoEConfigShape("C4", torch.bfloat16, 16384, 4096, 8, 2, 14336, 0.01),
    5: MoEConfigShape("C5", torch.float16, 65536, 2048, 128, 8, 768, 0.02, 2.0),
}


def _gen(cfg_id: int, stream: int) -> torch.Generator:
    return torch.Generator().manual_seed(CONFIG_SEEDS[cfg_id] * 100 + stream)


def make_inputs(cfg_id: int, T: int | None = None, with_weights: bool = True, ffn="gelu"):
    """Seeded synthetic inputs for config C<cfg_id>, drawn on the CPU in fp32.

    Each tensor has its own generator (seed = config seed * 100 + stream):
    0: X ~ N(0,1) [T,d]; 1: logits ~ N(0, s^2) [T,E] plus the config edits
    (C3: log-Zipf(1.2) bias over a seeded expert permutation; C5: 16 dead
    experts at -inf and 1% of tokens with all live logits tied at 0);
    2..4: expert weights ~ N(0, w_std^2) (up, down or gate, val, out);
    9: dY ~ N(0,1) [T,d]. ``T`` truncates the token count (same draws).
    """
    c = CONFIGS[cfg_id]
    Tn = c.T if T is None else T
    X = torch.randn(c.T, c.d, generator=_gen(cfg_id, 0))[:Tn]
    g = _gen(cfg_id, 1)
    logits = torch.randn(c.T, c.E, generator=g)[:Tn] * c.logit_std
    if cfg_id == 3:
        z = torch.tensor([(i + 1) ** -1.2 for i in range(c.E)], dtype=torch.float64)
        perm = torch.randperm(c.E, generator=g)
        bias = torch.log(z[perm] / z.sum()).float()
        logits = logits + bias
    if cfg_id == 5:
        dead = torch.randperm(c.E, generator=g)[:16]
        ties = torch.randperm(c.T, generator=g)[: math.ceil(c.T / 100)]
        ties = ties[ties < Tn]
        live = torch.ones(c.E, dtype=torch.bool)
        live[dead] = False
        logits[ties.unsqueeze(1), live.nonzero().squeeze(1).unsqueeze(0)] = 0.0
        logits[:, dead] = float("-inf")
    weights = {}
    if with_weights:
        names = ["up", "down"] if ffn == "gelu" else ["gate", "val", "out"]
        for i, n in enumerate(names):
            shape = (c.E, c.d, c.f) if n in ("up", "gate", "val") else (c.E, c.f, c.d)
            weights[n] = (torch.randn(*shape, generator=_gen(cfg_id, 2 + i)) * c.w_std).to(c.dtype)
    dY = torch.randn(c.T, c.d, generator=_gen(cfg_id, 9))[:Tn]
    return {
        "cfg": c,
        "X": X.to(c.dtype),
        "logits": logits,
        "weights": weights,
        "dY": dY.to(c.dtype),
    }
