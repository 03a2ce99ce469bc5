"""torch.ops.nanotitan on GPU tensors: the dispatcher runs the HIP kernels
(CUDA dispatch key), and their results equal the op library's CPU kernels on
the same inputs: bit for bit for the integer work, the packed rows and the
ordered fp32 sums; within the GPU tests' tolerances for GEMMs, dot products
and the router's exponentials."""

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from tests.test_torch_ops_cpu import _cases, bits

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops(ext):
    from nanotitan_amd.extension import load_op_library

    return load_op_library()


def _gpu(a):
    return a.cuda() if isinstance(a, torch.Tensor) else a


EXACT = {"count_expert_kernel", "pack_tokens_kernel", "pack_tokens_inv", "dispatch_tokens",
         "combine_tokens_kernel", "pack_kernel_backward", "combine_inv", "pack_backward_inv"}


@pytest.mark.parametrize("name", sorted(_cases()))
def test_gpu_op_matches_cpu_op(ops, name):
    args = _cases()[name]
    cpu = getattr(ops, name)(*args)
    gpu = getattr(ops, name)(*[_gpu(a) for a in _cases()[name]])
    torch.cuda.synchronize()
    cpu = cpu if isinstance(cpu, tuple) else (cpu,)
    gpu = gpu if isinstance(gpu, tuple) else (gpu,)
    assert len(cpu) == len(gpu)
    if name == "route_topk_count":
        cpu, gpu = cpu[:2], gpu[:2]  # the workspace holds counts in the dispatch's layout
    for i, (c, g) in enumerate(zip(cpu, gpu)):
        assert g.is_cuda and g.shape == c.shape and g.dtype == c.dtype, (name, i)
        if name in EXACT or c.dtype == torch.int32:
            assert torch.equal(bits(g), bits(c)), (name, i)
        else:
            torch.testing.assert_close(g.cpu().double(), c.double(), rtol=2e-4, atol=2e-4,
                                       msg=f"{name} output {i}")


def test_gpu_ops_pack_mutates_cursor_like_the_cpu_op(ops):
    d = O.make_inputs(3, T=4096, with_weights=False)
    c = d["cfg"]
    gates, idx, _ = O.route(d["logits"], c.k)
    X = d["X"][:, :128].contiguous()
    counts = O.count_experts(idx, None, c.E)
    cur_cpu = torch.from_numpy(O.offsets_from_counts(counts))
    cur_gpu = cur_cpu.cuda()
    want = ops.pack_tokens_kernel(X, gates, idx, cur_cpu)
    got = ops.pack_tokens_kernel(X.cuda(), gates.cuda(), idx.cuda(), cur_gpu)
    torch.cuda.synchronize()
    assert torch.equal(cur_gpu.cpu(), cur_cpu)
    for g, w in zip(got, want):
        assert torch.equal(bits(g), bits(w))


def test_gpu_ops_layer_sequence_bf16(ops):
    """The layer's op sequence through torch.ops on device tensors at C2
    widths: route+count, counted dispatch, fused GELU FFN, combine into bf16,
    equal to the pybind module's outputs (same kernels) bit for bit."""
    from nanotitan_amd.extension import get_hip_extension

    ext = get_hip_extension()
    d = O.make_inputs(2, T=2048)
    c = d["cfg"]
    x, logits = d["X"].cuda(), d["logits"].cuda()
    W_up, W_down = d["weights"]["up"].cuda(), d["weights"]["down"].cuda()
    runs = []
    for lib in (ops, ext):
        g, i, ws = lib.route_topk_count(logits, c.k, x)
        counts, offsets, px, tid, ex, pw, inv = lib.dispatch_tokens_counted(x, g, i, c.E, ws)
        a, gg = lib.grouped_gemm_gelu(px, offsets, W_up)
        y = lib.grouped_gemm_kernel(a, offsets, W_down)
        out = lib.combine_inv(y, inv, pw, torch.bfloat16)
        runs.append((counts, offsets, inv, a, gg, y, out))
    torch.cuda.synchronize()
    for u, v in zip(*runs):
        assert torch.equal(bits(u), bits(v))
    want_counts = np.bincount(O.route(d["logits"], c.k)[1].numpy().ravel(), minlength=c.E)
    assert np.array_equal(runs[0][0].cpu().numpy(), want_counts)
