"""CPU: the generated bf16 GELU table that the fused GEMM epilogue reads.

Every entry is checked against torch's own bf16 GELU (torch.nn.functional.gelu
and aten.gelu_backward, evaluated in fp32 and rounded once, which is what the
reference's unfused FFN computes) and against scipy's double-precision normal
CDF rounded to bf16. The table is rounded from double precision, so it may
differ from torch's fp32 evaluation where fp32 cancellation in 1 + erf(x/sqrt2)
costs torch its accuracy (x < -3); above that they agree bit for bit.
"""

import importlib.util
import math
from pathlib import Path

import numpy as np
import pytest
import torch

GEN = Path(__file__).resolve().parents[1] / "nanotitan_amd" / "csrc" / "gen_gelu_table.py"


def _gen():
    spec = importlib.util.spec_from_file_location("gen_gelu_table", GEN)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="module")
def table():
    g = _gen()
    words = np.array(g.table(), dtype=np.uint32)
    u = np.arange(g.N, dtype=np.uint32)
    bits = np.empty(2 * g.N, dtype=np.uint16)
    bits[0::2] = g.LO + u
    bits[1::2] = (g.LO + u) | 0x8000
    x = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16)
    return g, words, x


def _bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def test_layout_and_range(table):
    g, words, x = table
    assert g.LO == 0x3780 and g.HI == 0x4100  # 2^-16 and 8.0
    xf = x.float()
    assert xf[0].item() == 2.0**-16 and xf[1].item() == -(2.0**-16)
    assert xf.abs().max().item() < 8.0
    assert len(words) == 2 * (g.HI - g.LO)


def test_matches_torch_bf16_gelu(table):
    _, words, x = table
    want = _bits(torch.nn.functional.gelu(x.float()).to(torch.bfloat16))
    got = (words & 0xFFFF).astype(np.uint16)
    diff = np.abs(got.astype(np.int32) - want.astype(np.int32))
    # torch evaluates 0.5 * (1 + erf(x / sqrt2)) in fp32, which cancels for
    # x < -3 (and flushes to zero below about -5.5): bit-equal above -3, within
    # one ulp above -4, and the scipy test covers the tail.
    xf = x.float().numpy()
    assert diff[xf > -3.0].max() == 0
    assert diff[xf > -4.0].max() <= 1


def test_matches_torch_bf16_gelu_grad(table):
    _, words, x = table
    xf = x.float()
    want = _bits(torch.ops.aten.gelu_backward(torch.ones_like(xf), xf).to(torch.bfloat16))
    got = (words >> 16).astype(np.uint16)
    diff = np.abs(got.astype(np.int32) - want.astype(np.int32))
    xn = xf.numpy()
    assert diff[xn > -3.0].max() == 0
    assert diff[xn > -4.0].max() <= 1


def test_matches_scipy_double(table):
    """Independent double-precision evaluation (scipy.special.ndtr), rounded
    to bf16 by torch: equal everywhere, including the far negative tail."""
    from scipy.special import ndtr

    _, words, x = table
    xd = x.double().numpy()
    cdf = ndtr(xd)
    pdf = np.exp(-0.5 * xd * xd) / math.sqrt(2 * math.pi)
    g = torch.from_numpy(xd * cdf).to(torch.bfloat16)
    gp = torch.from_numpy(cdf + xd * pdf).to(torch.bfloat16)
    assert np.array_equal((words & 0xFFFF).astype(np.uint16), _bits(g))
    assert np.array_equal((words >> 16).astype(np.uint16), _bits(gp))


def test_special_values(table):
    g, words, x = table
    xf = x.float().numpy()
    lo = (words & 0xFFFF).astype(np.uint16)
    hi = (words >> 16).astype(np.uint16)
    vals = torch.from_numpy(lo.view(np.int16).copy()).view(torch.bfloat16).float().numpy()
    grads = torch.from_numpy(hi.view(np.int16).copy()).view(torch.bfloat16).float().numpy()
    # gelu(x) ~ x/2 and gelu'(x) ~ 1/2 near zero; gelu(x) = x, gelu'(x) = 1 near 8
    tiny = np.abs(xf) <= 2.0**-12
    assert np.all(vals[tiny] == xf[tiny] / 2)
    assert np.all(grads[tiny] == 0.5)
    big = xf >= 4.0
    assert np.all(vals[big] == xf[big])
    assert np.all(grads[big] == 1.0)
    # gelu has its minimum -0.16997 at x = -0.7518; gelu' = phi(x) (2 - x^2)
    # vanishes at x = -sqrt2, where gelu' takes its minimum -0.12899
    assert abs(vals.min() + 0.16997) < 1e-3 and abs(xf[vals.argmin()] + 0.7518) < 0.1
    assert abs(grads.min() + 0.12899) < 1e-3 and abs(xf[grads.argmin()] + math.sqrt(2)) < 0.1
