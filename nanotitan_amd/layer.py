"""MoE layer on the HIP expert path: the drop-in for the reference's CUDA backend.

* ``HIPMoEBackend(cfg, experts, router, spec)`` — the dataflow of the
  reference's ``CUDAMoEBackend.forward`` (src/model/cuda_backend.py:17-81):
  router in ``cfg.moe_router_dtype``, fp32 softmax / top-k / renorm, count,
  offsets, pack, experts, combine, cast, and ``MoELayerStats``. It takes the
  four-argument constructor that ``MoE.__init__`` uses
  (src/model/feed_fwd.py:142; the reference class only accepts three).
  The router kernel emits the per-block expert counts, offsets + pack run as
  one native call after it, and the combine writes
  the activation dtype directly (same values as combine-to-fp32-then-cast).
* ``ExpertFFN(cfg, spec)`` — SwiGLU experts with ``[E,d,f]`` / ``[E,f,d]``
  weights (src/model/feed_fwd.py:39-122), three grouped GEMMs.
* ``GeluExpertFFN(cfg, spec)`` — the 2-GEMM up -> GELU -> down FFN the
  benchmark configs specify, with the activation fused into the GEMMs.
* ``MoE(cfg, spec)`` — router + experts + backend (src/model/feed_fwd.py:128-152).
* ``route(logits, top_k)`` — fp32 softmax, top-k with ties to the lower
  expert id, renormalised gates, int32 ids.

Only the HIP path exists here; any other ``moe_backend`` raises.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch
import torch.nn as nn
from torch.profiler import record_function

from nanotitan_amd.moe_ops import (
    combine_inv_fn,
    grouped_gelu_ffn_fn,
    route_dispatch_fn,
    route_fn,
    swiglu_ffn_fn,
)

HIP_BACKENDS = ("hip", "cuda")  # "cuda" is accepted so reference configs select this path


@dataclass
class ModelShardSpec:
    """Expert range of this rank (reference src/model/utils.py:10-20); ep_size is 1 here."""

    layer_start: int = 0
    layer_end: int = 1
    has_token_embed: bool = False
    has_pos_embed: bool = False
    has_unembed_head: bool = False
    per_rank_expert: int = 1
    start_expert_id: int = 0
    end_expert_id: int = 1
    ep_size: int = 1
    ep_group: object | None = None


@dataclass
class MoELayerStats:
    """Routing statistics and the load-balancing loss (reference src/model/utils.py:70-93)."""

    tokens_per_expert: torch.Tensor
    probs_per_expert: torch.Tensor
    cfg: object
    aux_loss: torch.Tensor | None = field(default=None)

    def __post_init__(self):
        self.num_tokens = self.probs_per_expert.shape[0]
        self.total_assignments = self.tokens_per_expert.sum()
        self.ass_frac_per_expert = self.tokens_per_expert.float() / self.total_assignments
        self.probs_per_expert = self.probs_per_expert.mean(dim=0)
        self.aux_loss = (
            self.cfg.router_alpha
            * self.cfg.num_experts
            * torch.sum(self.ass_frac_per_expert * self.probs_per_expert)
        )


def route(logits: torch.Tensor, top_k: int):
    """(gates f32 [T,k], ids int32 [T,k]) from the fused router kernel.

    Reference src/model/cuda_backend.py:30-37: fp32 softmax, torch.topk,
    renormalise. The kernel selects the k largest logits (the same set as the
    k largest probabilities; ties go to the lower expert id, where torch.topk
    leaves the order unspecified) and returns the selected probabilities
    renormalised to sum 1.
    """
    return route_fn(logits.float().contiguous(), top_k)


def _check_backend(cfg):
    backend = getattr(cfg, "moe_backend", "hip")
    if backend not in HIP_BACKENDS:
        raise ValueError(f"moe_backend={backend!r}: this package implements only the HIP path")


class ExpertFFN(nn.Module):
    """SwiGLU experts: silu(X W_gate) * (X W_val), then W_out (reference feed_fwd.py:39-122)."""

    def __init__(self, cfg, spec):
        super().__init__()
        _check_backend(cfg)
        self.cfg = cfg
        self.spec = spec
        E, d, f = spec.per_rank_expert, cfg.d_model, cfg.ffn_in
        self.W_gate = nn.Parameter(torch.empty(E, d, f, dtype=cfg.dtype))
        self.W_val = nn.Parameter(torch.empty(E, d, f, dtype=cfg.dtype))
        self.W_out = nn.Parameter(torch.empty(E, f, d, dtype=cfg.dtype))
        for p in (self.W_gate, self.W_val, self.W_out):
            nn.init.kaiming_normal_(p, mode="fan_in", nonlinearity="relu")

    def forward(self, packed_X, expert_offset):
        # Gate and value GEMMs in one kernel with silu(gate) * value in its
        # epilogue; the backward fuses the activation's gradient likewise.
        return swiglu_ffn_fn(packed_X, self.W_gate, self.W_val, self.W_out, expert_offset)

    def parameter_count(self) -> int:
        return sum(p.numel() for p in self.parameters())


class GeluExpertFFN(nn.Module):
    """Up -> GELU (erf) -> down experts, the FFN of the benchmark configs."""

    def __init__(self, cfg, spec, std: float = 0.02):
        super().__init__()
        _check_backend(cfg)
        self.cfg = cfg
        self.spec = spec
        E, d, f = spec.per_rank_expert, cfg.d_model, cfg.ffn_in
        self.W_up = nn.Parameter(torch.randn(E, d, f).mul_(std).to(cfg.dtype))
        self.W_down = nn.Parameter(torch.randn(E, f, d).mul_(std).to(cfg.dtype))

    def forward(self, packed_X, expert_offset):
        return grouped_gelu_ffn_fn(packed_X, self.W_up, self.W_down, expert_offset)


def moe_forward_from_logits(x_flat, logits, experts, num_experts, top_k):
    """Hot path from router logits: route, dispatch, experts, combine (output in x's dtype).

    Returns (out [T,d], counts [E], gates [T,k]).
    """
    # The router kernel also counts the tokens per expert and per dispatch
    # block, so the dispatch starts at its scan; in the backward, the pack
    # backward also writes the router's gradient.
    with record_function("moe/topK_pack_tokens"):
        gates, idx, packed_X, packed_w, counts, offsets, _token_id, inv = route_dispatch_fn(
            logits.float().contiguous(), top_k, x_flat, num_experts
        )
    with record_function("moe/expert_compute"):
        y = experts(packed_X, offsets)
    with record_function("moe/combine_tokens"):
        out = combine_inv_fn(y, inv, packed_w, x_flat.dtype)
    return out, counts, gates


class HIPMoEBackend:
    """Reference CUDAMoEBackend dataflow (src/model/cuda_backend.py:11-81) on the HIP path."""

    def __init__(self, cfg, experts: nn.Module, router: nn.Linear, spec=None):
        _check_backend(cfg)
        self.cfg = cfg
        self.router = router
        self.experts = experts
        self.spec = spec

    def forward(self, x: torch.Tensor):
        batch, seq_len, d_model = x.shape
        flat = x.reshape(-1, d_model)
        router_dtype = self.router.weight.dtype
        with record_function("moe/router"):
            logits = self.router(flat.to(router_dtype))
        # Aux-loss probabilities from a second router pass on detached tokens
        # (src/model/cuda_backend.py:40-41), so the aux grad reaches only the router.
        aux_probs = self.router(flat.detach().to(router_dtype)).softmax(dim=-1)
        out, counts, _ = moe_forward_from_logits(
            flat, logits, self.experts, self.cfg.num_experts, self.cfg.top_k
        )
        stats = MoELayerStats(tokens_per_expert=counts.detach(), probs_per_expert=aux_probs,
                              cfg=self.cfg)
        return out.reshape(batch, seq_len, d_model), stats


class MoE(nn.Module):
    """Router + experts + HIP backend (reference src/model/feed_fwd.py:128-152)."""

    def __init__(self, cfg, spec=None, ffn: str = "swiglu"):
        super().__init__()
        _check_backend(cfg)
        if spec is None:
            spec = ModelShardSpec(per_rank_expert=cfg.num_experts, end_expert_id=cfg.num_experts)
        self.cfg = cfg
        self.spec = spec
        self.experts = ExpertFFN(cfg, spec) if ffn == "swiglu" else GeluExpertFFN(cfg, spec)
        router_dtype = getattr(cfg, "moe_router_dtype", torch.float32)
        self.router = nn.Linear(cfg.d_model, cfg.num_experts, bias=False, dtype=router_dtype)
        self.moe_backend = HIPMoEBackend(cfg, self.experts, self.router, spec)

    def forward(self, x):
        return self.moe_backend.forward(x)
