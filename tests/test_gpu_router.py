"""GPU parity: fused router gate (softmax -> top-k -> renorm) vs the oracle.

Indices are bit-exact (top-k by logit, ties to the lower expert id); gates
within rel 2e-6 of the float64 renormalised softmax; dlogits within rel 1e-5
of torch.autograd through the reference formula (softmax, gather, renorm).
"""

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu


def reference_grad(logits, idx, dg):
    """torch.autograd of gates = p[idx] / sum(p[idx]), p = softmax(logits) (float64)."""
    z = logits.double().clone().requires_grad_(True)
    p = z.softmax(dim=-1)
    sel = torch.gather(p, 1, idx.long())
    g = sel / sel.sum(dim=-1, keepdim=True)
    g.backward(dg.double())
    return z.grad


@pytest.mark.parametrize("cfg_id,T", [(1, 4096), (2, 30720), (3, 30720), (5, 65536)])
def test_route_config_logits(ext, cfg_id, T):
    d = O.make_inputs(cfg_id, T=T, with_weights=False)
    k = d["cfg"].k
    logits = d["logits"]
    want_g, want_i, _ = O.route(logits, k)
    g, i = ext.route_topk(logits.cuda(), k)
    torch.cuda.synchronize()
    assert np.array_equal(i.cpu().numpy(), want_i.numpy())
    torch.testing.assert_close(g.cpu(), want_g, rtol=2e-6, atol=1e-7)
    if cfg_id == 5:  # dead experts are never chosen; tied rows get the 8 lowest live ids at 1/8
        dead = torch.isinf(logits[0]).nonzero().squeeze(1)
        assert not torch.isin(i.cpu().long(), dead).any()


@pytest.mark.parametrize("T,E,k", [(1, 1, 1), (7, 3, 3), (1000, 16, 4), (513, 1024, 32),
                                   (2048, 128, 8), (300, 9, 1)])
def test_route_random_and_backward(ext, T, E, k):
    g_ = torch.Generator().manual_seed(T + E + k)
    logits = torch.randn(T, E, generator=g_)
    logits[::7] = torch.round(logits[::7])  # plenty of exact ties
    want_g, want_i, _ = O.route(logits, k)
    g, i = ext.route_topk(logits.cuda(), k)
    assert np.array_equal(i.cpu().numpy(), want_i.numpy())
    torch.testing.assert_close(g.cpu(), want_g, rtol=2e-6, atol=1e-7)
    dg = torch.randn(T, k, generator=g_)
    dz = ext.route_topk_backward(g, i, dg.cuda(), E)
    torch.testing.assert_close(dz.cpu().double(), reference_grad(logits, want_i, dg),
                               rtol=1e-5, atol=1e-6)


def test_route_autograd_function(ext):
    from nanotitan_amd.moe_ops import route_fn

    g_ = torch.Generator().manual_seed(5)
    logits = torch.randn(777, 64, generator=g_)
    z = logits.cuda().requires_grad_(True)
    gates, idx = route_fn(z, 6)
    dg = torch.randn(777, 6, generator=g_)
    gates.backward(dg.cuda())
    torch.testing.assert_close(z.grad.cpu().double(), reference_grad(logits, idx.cpu(), dg),
                               rtol=1e-5, atol=1e-6)


def test_route_rejects_bad_k(ext):
    with pytest.raises(RuntimeError):
        ext.route_topk(torch.zeros(4, 8, device="cuda"), 9)
    with pytest.raises(RuntimeError):
        ext.route_topk(torch.zeros(4, 64, device="cuda"), 33)


def test_route_special_values(ext):
    """Signed zeros tie (lower id first), denormals keep their order, +-FLT_MAX
    and +-inf rank at the ends: indices equal the oracle's stable descending
    sort; gates compared where the selected logits are finite."""
    tiny = 1e-45  # smallest fp32 denormal
    big = 3.4028234663852886e38
    rows = [
        [0.0, -0.0, -1.0, 1.0, -0.0, 0.0, 2.0, -2.0],
        [-0.0, 0.0, 0.0, -0.0, -0.0, 0.0, -0.0, 0.0],
        [tiny, 2 * tiny, -tiny, 0.0, -2 * tiny, 3 * tiny, -0.0, tiny],
        [big, -big, 1.0, big, -big, 0.0, -1.0, 5.0],
        [float("-inf"), -1.0, float("-inf"), 0.5, float("-inf"), -3.0, float("-inf"), 0.25],
        [float("inf"), 1.0, float("-inf"), 0.0, 2.0, float("inf"), -1.0, 3.0],
    ]
    logits = torch.tensor(rows, dtype=torch.float32).repeat(50, 1)  # several per wave
    for k in (1, 3, 5, 8):
        want_g, want_i, _ = O.route(logits, k)
        g, i = ext.route_topk(logits.cuda(), k)
        torch.cuda.synchronize()
        assert np.array_equal(i.cpu().numpy(), want_i.numpy()), k
        fin = torch.isfinite(want_g).all(dim=1)  # rows with +inf selected have NaN gates
        assert fin.sum() >= 4 * 50
        torch.testing.assert_close(g.cpu()[fin], want_g[fin], rtol=2e-6, atol=1e-7)
