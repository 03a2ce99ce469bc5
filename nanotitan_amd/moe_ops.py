"""Autograd surface of the MoE expert path.

Same function names, argument orders and gradient contracts as the
reference's ``src/model/moe_ops.py:10-125``:

* ``pack_tokens_fn(X, topk_weights, topk_experts, expert_offset_cpy)``
  -> (packed_X, packed_tokenId, packed_expert, packed_topk_weights);
  backward returns (X_grad, topk_weights_grad, None, None).
* ``combine_tokens_fn(packed_expert_outputs, packed_tokenId,
  packed_topk_weights, num_tokens, hidden_dim)`` -> float32 [T, d];
  backward casts the incoming grad to float32 contiguous and returns
  (expert_output_grad, None, packed_topk_weights_grad, None, None).
* ``grouped_gemm_fn(X, weight, expert_offset)`` applies
  ``GroupedGEMM_FN.apply(X, expert_offset, weight)``; backward returns
  (dX, None, dW).

Every op runs the HIP kernels through ``get_hip_extension()``; a missing
extension raises RuntimeError, never a silent fallback.

The layer uses additional Functions built on the inverse map the pack
writes: ``RouteCountFN`` (router gate that also counts the tokens per expert
and dispatch block), ``DispatchFN`` (count + offsets + pack, or offsets + pack
from RouteCountFN's counts) and ``CombineInvFN`` (combine whose backward reads
each token's grad row once). They compute the same values as pack_tokens_fn /
combine_tokens_fn on the same inputs.
"""

from __future__ import annotations

from typing import Any

import torch

from nanotitan_amd.extension import get_hip_extension


def combine_tokens_fn(
    packed_expert_outputs, packed_tokenId, packed_topk_weights, num_tokens, hidden_dim
):
    return CombineTokensFN.apply(
        packed_expert_outputs, packed_tokenId, packed_topk_weights, num_tokens, hidden_dim
    )


def pack_tokens_fn(X, topk_weights, topk_experts, expert_offset_cpy):
    return PackTokensFN.apply(X, topk_weights, topk_experts, expert_offset_cpy)


def grouped_gemm_fn(X, weight, expert_offset):
    return GroupedGEMM_FN.apply(X, expert_offset, weight)


class PackTokensFN(torch.autograd.Function):
    """Reference: src/model/moe_ops.py:40-73."""

    @staticmethod
    def forward(ctx, X, topk_weights, topk_experts, expert_offset_cpy) -> tuple:
        ext = get_hip_extension()
        packed_X, packed_tokenId, packed_expert, packed_topk_weights = ext.pack_tokens_kernel(
            X, topk_weights, topk_experts, expert_offset_cpy
        )
        ctx.save_for_backward(packed_tokenId, packed_expert, topk_experts)
        ctx.mark_non_differentiable(packed_tokenId, packed_expert)
        return packed_X, packed_tokenId, packed_expert, packed_topk_weights

    @staticmethod
    def backward(ctx, packed_X_grad, packed_tokenId_grad, packed_expert_grad,
                 packed_topk_weights_grad) -> Any:
        ext = get_hip_extension()
        packed_tokenId, packed_expert, topk_experts = ctx.saved_tensors
        if packed_topk_weights_grad is None:
            packed_topk_weights_grad = torch.zeros(
                packed_tokenId.shape, dtype=torch.float32, device=packed_tokenId.device
            )
        if packed_X_grad is None:
            raise RuntimeError("pack_tokens_fn backward needs a gradient for packed_X")
        X_grad, topk_weights_grad = ext.pack_kernel_backward(
            packed_X_grad.contiguous(),
            packed_topk_weights_grad.contiguous(),
            packed_tokenId,
            packed_expert,
            topk_experts,
        )
        return X_grad, topk_weights_grad, None, None


class CombineTokensFN(torch.autograd.Function):
    """Reference: src/model/moe_ops.py:76-104."""

    @staticmethod
    def forward(ctx, packed_expert_outputs, packed_tokenId, packed_topk_weights, num_tokens,
                hidden_dim) -> torch.Tensor:
        ext = get_hip_extension()
        pool = ext.combine_tokens_kernel(
            packed_expert_outputs, packed_tokenId, packed_topk_weights, num_tokens, hidden_dim
        )
        ctx.save_for_backward(packed_expert_outputs, packed_tokenId, packed_topk_weights)
        ctx.hidden_dim = hidden_dim
        return pool

    @staticmethod
    def backward(ctx, d_resid_stream) -> tuple:
        ext = get_hip_extension()
        packed_expert_outputs, packed_tokenId, packed_topk_weights = ctx.saved_tensors
        expert_output_grad, packed_topk_weights_grad = ext.combine_kernel_backward(
            packed_expert_outputs,
            packed_tokenId,
            packed_topk_weights,
            d_resid_stream.to(torch.float32).contiguous(),
            ctx.hidden_dim,
        )
        return expert_output_grad, None, packed_topk_weights_grad, None, None


class GroupedGEMM_FN(torch.autograd.Function):
    """Reference: src/model/moe_ops.py:107-125."""

    @staticmethod
    def forward(ctx, X, expert_offset, weight) -> torch.Tensor:
        ext = get_hip_extension()
        ctx.save_for_backward(X, expert_offset, weight)
        return ext.grouped_gemm_kernel(X, expert_offset, weight)

    @staticmethod
    def backward(ctx, out_grad) -> tuple:
        ext = get_hip_extension()
        X, expert_offset, weight = ctx.saved_tensors
        out_grad = out_grad.contiguous()
        dX = dW = None
        if ctx.needs_input_grad[0] and ctx.needs_input_grad[2]:
            # one call: the dW may run beside the dX (same values as the two calls)
            dW, dX = ext.bwd_grouped_gemm_dW_dX(X, weight, expert_offset, out_grad)
        elif ctx.needs_input_grad[0]:
            dX = ext.bwd_grouped_gemm_dX_kernel(weight, expert_offset, out_grad)
        elif ctx.needs_input_grad[2]:
            dW = ext.bwd_grouped_gemm_dW_kernel(X, expert_offset, out_grad)
        return dX, None, dW


class GroupedGeluFFN_FN(torch.autograd.Function):
    """Expert FFN up -> GELU (erf) -> down on the grouped GEMM, activation fused.

    Forward: (a, g) = grouped_gemm_gelu(X, W_up) — a = gelu(h) and
    g = gelu'(h) for h = X W_up, from one kernel — then y = a W_down.
    Backward: dH = (dy W_down^T) * g from one kernel, then the three
    remaining grouped GEMMs. The values of grouped_gemm_fn +
    torch.nn.functional.gelu + grouped_gemm_fn (the reference's ExpertFFN
    dataflow, src/model/feed_fwd.py:102-112, with the configs' GELU), except
    that gelu'(h) is rounded to the activation dtype before the multiply;
    backward returns (dX, None, dW_up, dW_down).
    """

    @staticmethod
    def forward(ctx, X, expert_offset, W_up, W_down):
        ext = get_hip_extension()
        a, g = ext.grouped_gemm_gelu(X, expert_offset, W_up)
        y = ext.grouped_gemm_kernel(a, expert_offset, W_down)
        ctx.save_for_backward(X, expert_offset, W_up, W_down, a, g)
        return y

    @staticmethod
    def backward(ctx, dy):
        ext = get_hip_extension()
        X, expert_offset, W_up, W_down, a, g = ctx.saved_tensors
        dy = dy.contiguous()
        dX = dW_up = dW_down = None
        need_dH = ctx.needs_input_grad[0] or ctx.needs_input_grad[2]
        # Each projection's dW and dX in one call: a dW with few 256x256
        # tiles runs beside its dX in one kernel launch (same values).
        if ctx.needs_input_grad[3] and need_dH:
            dW_down, dH = ext.bwd_grouped_gemm_dW_dX_gelu(a, W_down, expert_offset, dy, g)
        elif ctx.needs_input_grad[3]:
            dW_down = ext.bwd_grouped_gemm_dW_kernel(a, expert_offset, dy)
        elif need_dH:
            dH = ext.bwd_grouped_gemm_dX_gelu(W_down, expert_offset, dy, g)
        if ctx.needs_input_grad[0] and ctx.needs_input_grad[2]:
            dW_up, dX = ext.bwd_grouped_gemm_dW_dX(X, W_up, expert_offset, dH)
        elif ctx.needs_input_grad[0]:
            dX = ext.bwd_grouped_gemm_dX_kernel(W_up, expert_offset, dH)
        elif ctx.needs_input_grad[2]:
            dW_up = ext.bwd_grouped_gemm_dW_kernel(X, expert_offset, dH)
        return dX, None, dW_up, dW_down


def grouped_gelu_ffn_fn(X, W_up, W_down, expert_offset):
    return GroupedGeluFFN_FN.apply(X, expert_offset, W_up, W_down)


class SwiGLUFFN_FN(torch.autograd.Function):
    """The reference's SwiGLU ExpertFFN on fused grouped GEMMs.

    Forward: (h, g, v) = grouped_gemm_swiglu(X, W_gate, W_val) — the gate and
    value GEMMs in one kernel whose epilogue writes gate, value and
    hidden = silu(gate) * value — then y = h W_out. Backward:
    (dgate, dvalue) from one kernel (dhidden = dy W_out^T and the SwiGLU
    backward in its epilogue), dX = dgate W_gate^T + dvalue W_val^T as one
    GEMM over the concatenated reduction, and the three weight gradients.
    The values of the reference's _forward_cuda (src/model/feed_fwd.py:102-112:
    grouped_gemm_fn, grouped_gemm_fn, silu(gate) * value, grouped_gemm_fn),
    rounded where it rounds, except that the two dX products are summed
    before the one rounding; backward returns
    (dX, None, dW_gate, dW_val, dW_out).
    """

    @staticmethod
    def forward(ctx, X, expert_offset, W_gate, W_val, W_out):
        ext = get_hip_extension()
        h, g, v = ext.grouped_gemm_swiglu(X, expert_offset, W_gate, W_val)
        y = ext.grouped_gemm_kernel(h, expert_offset, W_out)
        ctx.save_for_backward(X, expert_offset, W_gate, W_val, W_out, h, g, v)
        return y

    @staticmethod
    def backward(ctx, dy):
        ext = get_hip_extension()
        X, expert_offset, W_gate, W_val, W_out, h, g, v = ctx.saved_tensors
        dy = dy.contiguous()
        dX = dW_gate = dW_val = dW_out = None
        need_d = any(ctx.needs_input_grad[i] for i in (0, 2, 3))
        # Paired calls (a dW with few tiles runs beside its dX in one launch).
        if ctx.needs_input_grad[4] and need_d:
            dW_out, dg, dv = ext.bwd_grouped_gemm_dW_dX_swiglu(h, W_out, expert_offset, dy, g, v)
        elif ctx.needs_input_grad[4]:
            dW_out = ext.bwd_grouped_gemm_dW_kernel(h, expert_offset, dy)
        elif need_d:
            dg, dv = ext.bwd_grouped_gemm_dX_swiglu(W_out, expert_offset, dy, g, v)
        if ctx.needs_input_grad[0] and ctx.needs_input_grad[2]:
            dW_gate, dX = ext.bwd_grouped_gemm_dW_dX2(X, W_gate, W_val, expert_offset, dg, dv)
        elif ctx.needs_input_grad[0]:
            dX = ext.bwd_grouped_gemm_dX2(W_gate, W_val, expert_offset, dg, dv)
        elif ctx.needs_input_grad[2]:
            dW_gate = ext.bwd_grouped_gemm_dW_kernel(X, expert_offset, dg)
        if ctx.needs_input_grad[3]:
            dW_val = ext.bwd_grouped_gemm_dW_kernel(X, expert_offset, dv)
        return dX, None, dW_gate, dW_val, dW_out


def swiglu_ffn_fn(X, W_gate, W_val, W_out, expert_offset):
    return SwiGLUFFN_FN.apply(X, expert_offset, W_gate, W_val, W_out)


# --------------------------------------------------------------- layer ops


class DispatchFN(torch.autograd.Function):
    """Fused count + offsets + pack for the layer.

    Forward returns (packed_X, packed_topk_weights, counts, offsets, token_id,
    inv); the integer outputs are non-differentiable. Backward is the pack
    backward driven by the inverse map.
    """

    @staticmethod
    def forward(ctx, X, topk_weights, topk_experts, num_experts, counted_ws=None):
        # counted_ws: the workspace route_count_fn returned for these tokens,
        # already holding the per-block expert counts (the counting pass is
        # then skipped).
        ext = get_hip_extension()
        if counted_ws is None:
            outs = ext.dispatch_tokens(X, topk_weights, topk_experts, num_experts)
        else:
            outs = ext.dispatch_tokens_counted(X, topk_weights, topk_experts, num_experts,
                                               counted_ws)
        counts, offsets, packed_X, token_id, _expert, packed_w, inv = outs
        ctx.save_for_backward(inv)
        ctx.mark_non_differentiable(counts, offsets, token_id, inv)
        # No zero-filled grads for the integer outputs (or an unused packed_w).
        ctx.set_materialize_grads(False)
        return packed_X, packed_w, counts, offsets, token_id, inv

    @staticmethod
    def backward(ctx, packed_X_grad, packed_w_grad, *_):
        ext = get_hip_extension()
        (inv,) = ctx.saved_tensors
        if packed_X_grad is None:
            raise RuntimeError("dispatch_fn backward needs a gradient for packed_X")
        if packed_w_grad is None:
            packed_w_grad = torch.zeros(inv.numel(), dtype=torch.float32, device=inv.device)
        X_grad, w_grad = ext.pack_backward_inv(
            packed_X_grad.contiguous(), packed_w_grad.contiguous(), inv
        )
        return X_grad, w_grad, None, None, None


class CombineInvFN(torch.autograd.Function):
    """Combine by inverse map; output in ``out_dtype`` (float32 on the reference surface).

    Backward accepts the grad in float32 or the activation dtype without a cast
    pass and returns (expert_output_grad, None, packed_topk_weights_grad, None).
    """

    @staticmethod
    def forward(ctx, packed_expert_outputs, inv, packed_topk_weights, out_dtype):
        ext = get_hip_extension()
        out = ext.combine_inv(packed_expert_outputs, inv, packed_topk_weights, out_dtype)
        ctx.save_for_backward(packed_expert_outputs, inv, packed_topk_weights)
        return out

    @staticmethod
    def backward(ctx, grad):
        ext = get_hip_extension()
        y, inv, w = ctx.saved_tensors
        if grad.dtype not in (torch.float32, y.dtype):
            grad = grad.to(torch.float32)
        dy, dw = ext.combine_backward_inv(y, inv, w, grad.contiguous())
        return dy, None, dw, None


class RouteFN(torch.autograd.Function):
    """Fused router gate: logits [T,E] f32 -> (gates [T,k] f32, topk [T,k] int32).

    Top-k by logit with ties to the lower expert id (the top-k of the
    softmax probabilities), gates = the selected probabilities renormalised
    (reference src/model/cuda_backend.py:30-37). Backward returns dlogits.
    """

    @staticmethod
    def forward(ctx, logits, top_k):
        ext = get_hip_extension()
        gates, topk = ext.route_topk(logits.contiguous(), top_k)
        ctx.save_for_backward(gates, topk)
        ctx.num_experts = logits.shape[1]
        ctx.mark_non_differentiable(topk)
        ctx.set_materialize_grads(False)  # no zero-filled grad for the int32 ids
        return gates, topk

    @staticmethod
    def backward(ctx, dgates, _dtopk):
        ext = get_hip_extension()
        gates, topk = ctx.saved_tensors
        if dgates is None:
            return None, None
        return ext.route_topk_backward(gates, topk, dgates.contiguous().float(),
                                       ctx.num_experts), None


class RouteCountFN(torch.autograd.Function):
    """RouteFN with the dispatch's expert count fused into the router kernel.

    Returns (gates, topk, dispatch_ws): dispatch_ws holds the per-block
    expert counts for the tokens X (X fixes the block size and device) and
    goes to dispatch_fn(..., counted_ws=dispatch_ws). Same gates, ids and
    backward as RouteFN.
    """

    @staticmethod
    def forward(ctx, logits, top_k, X):
        ext = get_hip_extension()
        gates, topk, ws = ext.route_topk_count(logits.contiguous(), top_k, X)
        ctx.save_for_backward(gates, topk)
        ctx.num_experts = logits.shape[1]
        ctx.mark_non_differentiable(topk, ws)
        ctx.set_materialize_grads(False)
        return gates, topk, ws

    @staticmethod
    def backward(ctx, dgates, _dtopk, _dws):
        ext = get_hip_extension()
        gates, topk = ctx.saved_tensors
        if dgates is None:
            return None, None, None
        return ext.route_topk_backward(gates, topk, dgates.contiguous().float(),
                                       ctx.num_experts), None, None


class RouteDispatchFN(torch.autograd.Function):
    """Router gate (with the dispatch's count) and dispatch in one Function.

    Forward: route_topk_count on logits [T,E] f32, then dispatch_tokens_counted
    of X with those gates. Returns (gates, topk, packed_X, packed_w, counts,
    offsets, token_id, inv), the outputs of RouteCountFN and DispatchFN.
    Backward: when the gates get no gradient of their own (they feed only the
    dispatch), one launch writes dX and dlogits (pack_backward_inv_route);
    otherwise the pack backward's gate gradient is added to theirs before the
    router's backward. Either way the result equals RouteCountFN followed by
    DispatchFN.
    """

    @staticmethod
    def forward(ctx, logits, top_k, X, num_experts):
        ext = get_hip_extension()
        gates, topk, ws = ext.route_topk_count(logits.contiguous(), top_k, X)
        outs = ext.dispatch_tokens_counted(X, gates, topk, num_experts, ws)
        counts, offsets, packed_X, token_id, _expert, packed_w, inv = outs
        ctx.save_for_backward(gates, topk, inv)
        ctx.num_experts = logits.shape[1]
        ctx.mark_non_differentiable(topk, counts, offsets, token_id, inv)
        ctx.set_materialize_grads(False)
        return gates, topk, packed_X, packed_w, counts, offsets, token_id, inv

    @staticmethod
    def backward(ctx, dgates, _dtopk, packed_X_grad, packed_w_grad, *_):
        ext = get_hip_extension()
        gates, topk, inv = ctx.saved_tensors
        if packed_X_grad is None:
            raise RuntimeError("route_dispatch_fn backward needs a gradient for packed_X")
        if packed_w_grad is None:
            packed_w_grad = torch.zeros(inv.numel(), dtype=torch.float32, device=inv.device)
        dpX, dpw = packed_X_grad.contiguous(), packed_w_grad.contiguous()
        if dgates is None:
            X_grad, dlogits = ext.pack_backward_inv_route(dpX, dpw, inv, gates, topk,
                                                          ctx.num_experts)
        else:
            X_grad, w_grad = ext.pack_backward_inv(dpX, dpw, inv)
            dlogits = ext.route_topk_backward(gates, topk, (w_grad + dgates.float()).contiguous(),
                                              ctx.num_experts)
        return dlogits, None, X_grad, None


def route_fn(logits, top_k):
    return RouteFN.apply(logits, top_k)


def route_count_fn(logits, top_k, X):
    return RouteCountFN.apply(logits, top_k, X)


def route_dispatch_fn(logits, top_k, X, num_experts):
    return RouteDispatchFN.apply(logits, top_k, X, num_experts)


def dispatch_fn(X, topk_weights, topk_experts, num_experts, counted_ws=None):
    return DispatchFN.apply(X, topk_weights, topk_experts, num_experts, counted_ws)


def combine_inv_fn(packed_expert_outputs, inv, packed_topk_weights, out_dtype=torch.float32):
    return CombineInvFN.apply(packed_expert_outputs, inv, packed_topk_weights, out_dtype)
