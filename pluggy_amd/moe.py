"""Operator level of the MoE block: router and dropless expert FFN on HIP.

Mirrors the reference operator surface:

* ``moe_expert_ffn`` replaces ``pluggy.kernels.moe.moe_expert_ffn``
  (pluggy/kernels/moe.py:127-168): same arguments, same shapes, same errors
  (AssertionError on rank/shape), a freshly allocated output, inputs never
  mutated. It always runs the HIP grouped path; ``use_grouped_mm`` is accepted
  for signature compatibility.
* ``router_topk`` is the arithmetic of ``Qwen3MoeTopKRouter.forward``
  (pluggy/models/qwen3_moe/qwen3_moe.py:168-178) with fp32 logits and the
  "ties -> lower expert id" selection rule.

Both are ``torch.autograd.Function``s whose forward and backward each call one
C-ABI entry point of ``libpmoe.so``.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib
from ._lib import call, dtype_code, ptr, require_gpu, size, stream_of, workspace


@dataclass
class RouterStats:
    """Additive per-layer routing statistics emitted by the fused router."""

    expert_counts: torch.Tensor   # (E,) int32: picks per expert over all slots
    prob_sum: torch.Tensor        # (E,) fp32: sum over tokens of softmax(logits)
    lse_sq_sum: torch.Tensor      # (1,) fp32: sum over tokens of logsumexp(logits)^2
    tokens: int


class _RouterFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, top_k, norm_topk_prob, logit_bias, out_dtype):
        T, H = x.shape
        E = weight.shape[0]
        dev = x.device
        logits = torch.empty(T, E, dtype=torch.float32, device=dev)
        top_w = torch.empty(T, top_k, dtype=out_dtype, device=dev)
        top_i = torch.empty(T, top_k, dtype=torch.int64, device=dev)
        top_w32 = torch.empty(T, top_k, dtype=torch.float32, device=dev)
        counts = torch.empty(E, dtype=torch.int32, device=dev)
        psum = torch.empty(E, dtype=torch.float32, device=dev)
        lse2 = torch.empty(1, dtype=torch.float32, device=dev)
        nbytes = size("pmoe_router_forward_workspace_size", T, E)
        ws = workspace(nbytes, dev)
        call("pmoe_router_forward", ptr(x), dtype_code(x.dtype), ptr(weight), dtype_code(weight.dtype),
             ptr(logit_bias), T, H, E, top_k, int(norm_topk_prob), ptr(logits), ptr(top_w), dtype_code(out_dtype),
             ptr(top_i), ptr(top_w32), ptr(counts), ptr(psum), ptr(lse2), ptr(ws), ws.numel(), stream_of(x))
        ctx.save_for_backward(x, weight, logits, top_i, top_w32)
        ctx.norm_topk_prob = bool(norm_topk_prob)
        ctx.mark_non_differentiable(top_i, top_w32, counts, psum, lse2)
        return logits, top_w, top_i, top_w32, counts, psum, lse2

    @staticmethod
    def backward(ctx, g_logits, g_w, _gi, _gw32, _gc, _gp, _gl):
        x, weight, logits, top_i, top_w32 = ctx.saved_tensors
        T, H = x.shape
        E, K = weight.shape[0], top_i.shape[1]
        need_x, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        if not (need_x or need_w) or (g_logits is None and g_w is None):
            return None, None, None, None, None, None
        gx = torch.empty_like(x) if need_x else None
        gW = torch.empty_like(weight) if need_w else None
        if g_logits is not None:
            g_logits = g_logits.float().contiguous()
        gw_code = _lib.PMOE_F32
        if g_w is not None:
            g_w = g_w.contiguous()
            gw_code = dtype_code(g_w.dtype)
        ws = workspace(size("pmoe_router_backward_workspace_size", T, H, E), x.device)
        call("pmoe_router_backward", ptr(x), dtype_code(x.dtype), ptr(weight), dtype_code(weight.dtype),
             ptr(logits), ptr(top_i), ptr(top_w32), ptr(g_w), gw_code, ptr(g_logits), T, H, E, K,
             int(ctx.norm_topk_prob), ptr(gx), ptr(gW), ptr(ws), ws.numel(), stream_of(x))
        return gx, gW, None, None, None, None


def router_topk(hidden: torch.Tensor, weight: torch.Tensor, top_k: int, norm_topk_prob: bool = True,
                logit_bias: torch.Tensor | None = None, return_stats: bool = False):
    """Fused router: fp32 logits, softmax, top-k (ties -> lower id), renormalise.

    Returns ``(router_logits (T,E) fp32, top_weights (T,K) hidden.dtype,
    top_indices (T,K) int64)`` and, with ``return_stats``, a ``RouterStats``.
    Gradients flow to ``hidden`` and ``weight`` through both the logits (for
    aux losses) and the top weights.
    """
    assert hidden.dim() == 2, "router expects (T, H) hidden states"
    assert weight.dim() == 2 and weight.shape[1] == hidden.shape[1]
    assert 1 <= top_k <= weight.shape[0]
    require_gpu(hidden, weight, logit_bias)
    x = hidden.contiguous()
    w = weight.contiguous()
    if w.dtype not in (torch.float32, torch.bfloat16):
        w = w.float()
    if logit_bias is not None:
        logit_bias = logit_bias.float().contiguous()
    logits, top_w, top_i, _w32, counts, psum, lse2 = _RouterFunction.apply(
        x, w, int(top_k), bool(norm_topk_prob), logit_bias, x.dtype)
    if return_stats:
        return logits, top_w, top_i, RouterStats(counts, psum, lse2, x.shape[0])
    return logits, top_w, top_i


class _ExpertFFNFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, hidden, top_indices, top_weights, gate_up_proj, down_proj):
        T, H = hidden.shape
        K = top_indices.shape[1]
        E, two_i, _ = gate_up_proj.shape
        I = two_i // 2
        P = T * K
        dev, dt = hidden.device, hidden.dtype
        out = torch.empty(T, H, dtype=dt, device=dev)
        counts = torch.empty(E, dtype=torch.int32, device=dev)
        offs = torch.empty(E, dtype=torch.int32, device=dev)
        sorted_pair = torch.empty(P, dtype=torch.int32, device=dev)
        inv_pos = torch.empty(P, dtype=torch.int32, device=dev)
        x_perm = torch.empty(P, H, dtype=dt, device=dev)
        gu = torch.empty(P, 2 * I, dtype=dt, device=dev)
        mid = torch.empty(P, I, dtype=dt, device=dev)
        y = torch.empty(P, H, dtype=dt, device=dev)
        ws = workspace(size("pmoe_expert_ffn_forward_workspace_size", T, K, E), dev)
        call("pmoe_expert_ffn_forward", ptr(hidden), ptr(top_indices), ptr(top_weights),
             dtype_code(top_weights.dtype), ptr(gate_up_proj), ptr(down_proj), dtype_code(dt), T, K, E, H, I,
             ptr(out), ptr(counts), ptr(offs), ptr(sorted_pair), ptr(inv_pos), ptr(x_perm), ptr(gu), ptr(mid),
             ptr(y), ptr(ws), ws.numel(), stream_of(hidden))
        ctx.save_for_backward(top_weights, gate_up_proj, down_proj, offs, sorted_pair, inv_pos, x_perm, gu, mid, y)
        ctx.dims = (T, K, E, H, I)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        top_w, gate_up, down, offs, sorted_pair, inv_pos, x_perm, gu, mid, y = ctx.saved_tensors
        T, K, E, H, I = ctx.dims
        need = ctx.needs_input_grad
        grad_out = grad_out.contiguous()
        if grad_out.dtype != x_perm.dtype:
            grad_out = grad_out.to(x_perm.dtype)
        dev = grad_out.device
        g_hidden = torch.empty(T, H, dtype=x_perm.dtype, device=dev) if need[0] else None
        g_w = torch.empty_like(top_w) if need[2] else None
        g_gu = torch.empty_like(gate_up) if need[3] else None
        g_dn = torch.empty_like(down) if need[4] else None
        ws = workspace(size("pmoe_expert_ffn_backward_workspace_size", T, K, H, I, dtype_code(x_perm.dtype)), dev)
        call("pmoe_expert_ffn_backward", ptr(grad_out), ptr(top_w), dtype_code(top_w.dtype), ptr(gate_up),
             ptr(down), dtype_code(x_perm.dtype), T, K, E, H, I, ptr(offs), ptr(sorted_pair), ptr(inv_pos),
             ptr(x_perm), ptr(gu), ptr(mid), ptr(y), ptr(g_hidden), ptr(g_w), ptr(g_gu), ptr(g_dn), ptr(ws),
             ws.numel(), stream_of(grad_out))
        return g_hidden, None, g_w, g_gu, g_dn


def moe_expert_ffn(
    hidden: torch.Tensor,        # (T, H)
    top_indices: torch.Tensor,   # (T, K) int64
    top_weights: torch.Tensor,   # (T, K)
    gate_up_proj: torch.Tensor,  # (E, 2I, H)
    down_proj: torch.Tensor,     # (E, H, I)
    *,
    use_grouped_mm: bool | None = None,
) -> torch.Tensor:
    """Dropless top-k expert FFN on MI355X (drop-in for moe.py:127-168).

    ``out[t] = sum_k w[t,k] * down[e](silu(gate[e] x_t) * up[e] x_t)`` with
    e = top_indices[t,k]. Weights are cast to ``hidden.dtype`` first, as the
    reference does (moe.py:110-112). The permutation, both grouped GEMMs and
    the fp32-accumulating combine run as HIP kernels; there is no CPU path.
    """
    assert hidden.dim() == 2
    assert top_indices.shape == top_weights.shape
    assert top_indices.shape[0] == hidden.shape[0]
    assert gate_up_proj.dim() == 3 and down_proj.dim() == 3
    del use_grouped_mm  # one code path: the HIP grouped kernels
    require_gpu(hidden, top_indices, top_weights, gate_up_proj, down_proj)
    dt = hidden.dtype
    gu = gate_up_proj.to(dtype=dt).contiguous()
    dn = down_proj.to(dtype=dt).contiguous()
    tw = top_weights if top_weights.dtype in (torch.float32, torch.bfloat16) else top_weights.float()
    return _ExpertFFNFunction.apply(hidden.contiguous(), top_indices.to(torch.int64).contiguous(), tw.contiguous(),
                                    gu, dn)

