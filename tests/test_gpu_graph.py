"""The MoE layer step captured into one HIP graph.

Router, dispatch, the fused GELU experts, combine and all their backwards
are captured with torch.cuda.graph and replayed on new inputs copied into
the captured buffers. Every replay must equal an eager step on the same
inputs bit for bit: the output, the counts, the gates and the gradients of
the tokens, the router logits and both expert weights. Eager steps run on
the same device between the replays. This holds only if nothing in the path
synchronises with the host, allocates outside the graph's pool, or keeps
state from one launch to the next that a replay would not reset (the paired
dW + dX kernels' claim counters are cleared inside the graph by a fill
kernel when the stream is capturing).
"""

import pytest
import torch

from tests.test_gpu_dispatch import bits

pytestmark = pytest.mark.gpu

T, D, E, K, F = 4096, 512, 8, 2, 1024
DTYPE = torch.bfloat16
NAMES = ("out", "counts", "gates", "dX", "dlogits", "dW_up", "dW_down")


def _inputs(seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    X = torch.randn(T, D, generator=g, device="cuda").to(DTYPE)
    logits = torch.randn(T, E, generator=g, device="cuda")
    dY = torch.randn(T, D, generator=g, device="cuda").to(DTYPE)
    return X, logits, dY


# The weights' gradient-accumulation nodes are created by the warm-up steps on
# the side stream, which torch reports as a stream mismatch at capture; every
# gradient of every replay is checked bit for bit below.
@pytest.mark.filterwarnings("ignore:The AccumulateGrad node's stream")
def test_layer_step_under_graph_replay(ext):
    from nanotitan_amd.layer import moe_forward_from_logits
    from nanotitan_amd.moe_ops import grouped_gelu_ffn_fn

    g = torch.Generator(device="cuda").manual_seed(1)
    W_up = (torch.randn(E, D, F, generator=g, device="cuda") * 0.02).to(DTYPE).requires_grad_(True)
    W_down = (torch.randn(E, F, D, generator=g, device="cuda") * 0.02).to(DTYPE).requires_grad_(True)

    def ffn(packed_X, offsets):
        return grouped_gelu_ffn_fn(packed_X, W_up, W_down, offsets)

    def run(X, logits, dY):
        X.grad = logits.grad = W_up.grad = W_down.grad = None
        out, counts, gates = moe_forward_from_logits(X, logits, ffn, E, K)
        out.backward(dY)
        return out, counts, gates, X.grad, logits.grad, W_up.grad, W_down.grad

    def eager(seed):
        X, logits, dY = _inputs(seed)
        X.requires_grad_(True)
        logits.requires_grad_(True)
        return [t.detach().clone() for t in run(X, logits, dY)]

    sX, slog, sdY = _inputs(0)
    sX.requires_grad_(True)
    slog.requires_grad_(True)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm up outside the capture
        for _ in range(3):
            run(sX, slog, sdY)
    torch.cuda.current_stream().wait_stream(side)
    sX.grad = slog.grad = W_up.grad = W_down.grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = run(sX, slog, sdY)
    torch.cuda.synchronize()

    for seed in (11, 12, 13, 14):
        X, logits, dY = _inputs(seed)
        with torch.no_grad():
            sX.copy_(X)
            slog.copy_(logits)
            sdY.copy_(dY)
        print(f"[graph] layer step replay, inputs of seed {seed}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        got = [t.detach().clone() for t in captured]
        want = eager(seed)
        torch.cuda.synchronize()
        for name, a, b in zip(NAMES, got, want):
            assert torch.equal(bits(a), bits(b)), (seed, name)
