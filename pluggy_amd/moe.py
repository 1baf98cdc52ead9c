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

Both are ``torch.autograd.Function``s. Each stage (router, permutation, row
gather, each grouped GEMM, combine, and their backward) is one C-ABI call on
the current stream; ``stage_timer()`` brackets the stages with HIP events.
"""

from __future__ import annotations

import contextlib
from collections import defaultdict
from dataclasses import dataclass

import torch

from . import ops
from ._lib import require_gpu


@dataclass
class RouterStats:
    """Additive per-layer routing statistics emitted by the fused router."""

    expert_counts: torch.Tensor   # (E,) int32: picks per expert over all slots
    prob_sum: torch.Tensor        # (E,) fp32: sum over tokens of softmax(logits)
    lse_sq_sum: torch.Tensor      # (1,) fp32: sum over tokens of logsumexp(logits)^2
    tokens: int


# ------------------------------------------------------------ stage timing


class StageTimer:
    """HIP-event timing of each named stage on the stream it runs on."""

    def __init__(self):
        self.records: dict[str, list] = defaultdict(list)

    @contextlib.contextmanager
    def mark(self, name: str):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        try:
            yield
        finally:
            end.record()
            self.records[name].append((start, end))

    def summary(self) -> dict[str, dict[str, float]]:
        """name -> {"calls", "total_ms", "mean_ms"} (synchronises)."""
        torch.cuda.synchronize()
        out = {}
        for name, evs in self.records.items():
            ms = [s.elapsed_time(e) for s, e in evs]
            out[name] = {"calls": len(ms), "total_ms": sum(ms), "mean_ms": sum(ms) / len(ms)}
        return out


_timer: StageTimer | None = None


@contextlib.contextmanager
def stage_timer():
    """Collect per-stage HIP-event timings of every MoE call made inside the block."""
    global _timer
    prev, _timer = _timer, StageTimer()
    try:
        yield _timer
    finally:
        _timer = prev


def _stage(name: str):
    return _timer.mark(name) if _timer is not None else contextlib.nullcontext()


# ------------------------------------------------------------------ router


class _RouterFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, top_k, norm_topk_prob, logit_bias):
        with _stage("router_fwd"):
            logits, top_w, top_i, top_w32, counts, psum, lse2 = ops.router_forward(
                x, weight, top_k, norm_topk_prob, logit_bias)
        ctx.save_for_backward(x, weight, logits, top_i, top_w32)
        ctx.norm_topk_prob = bool(norm_topk_prob)
        ctx.mark_non_differentiable(top_i, top_w32, counts, psum, lse2)
        ctx.set_materialize_grads(False)  # absent gradients stay None (no zero-filled tensors)
        return logits, top_w, top_i, top_w32, counts, psum, lse2

    @staticmethod
    def backward(ctx, g_logits, g_w, _gi, _gw32, _gc, _gp, _gl):
        x, weight, logits, top_i, top_w32 = ctx.saved_tensors
        if not (ctx.needs_input_grad[0] or ctx.needs_input_grad[1]) or (g_logits is None and g_w is None):
            return None, None, None, None, None
        if g_logits is not None:
            g_logits = g_logits.float().contiguous()
        if g_w is not None:
            g_w = g_w.contiguous()
        with _stage("router_bwd"):
            gx, gW = ops.router_backward(x, weight, logits, top_i, top_w32, g_w, g_logits, ctx.norm_topk_prob)
        return (gx if ctx.needs_input_grad[0] else None), (gW if ctx.needs_input_grad[1] else None), None, None, None


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
        x, w, int(top_k), bool(norm_topk_prob), logit_bias)
    if return_stats:
        return logits, top_w, top_i, RouterStats(counts, psum, lse2, x.shape[0])
    return logits, top_w, top_i


# -------------------------------------------------------------- expert FFN


class _ExpertFFNFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, hidden, top_indices, top_weights, gate_up_proj, down_proj):
        E = gate_up_proj.shape[0]
        K = top_indices.shape[1]
        with _stage("permute"):
            counts, offs, sorted_pair, inv_pos = ops.permute(top_indices, E)
        with _stage("dispatch"):
            x_perm = ops.dispatch(hidden, inv_pos, K)
        with _stage("gate_up_fwd"):
            gu, mid = ops.gate_up_swiglu(x_perm, gate_up_proj, offs)
        with _stage("down_fwd"):
            y = ops.down_proj(mid, down_proj, offs)
        with _stage("combine"):
            out = ops.combine(y, top_weights, inv_pos)
        ctx.save_for_backward(top_weights, gate_up_proj, down_proj, offs, inv_pos, x_perm, gu, mid, y)
        ctx.dims = (hidden.shape[0], K, E)
        ctx.set_materialize_grads(False)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        if grad_out is None:
            return None, None, None, None, None
        top_w, gate_up, down, offs, inv_pos, x_perm, gu, mid, y = ctx.saved_tensors
        T, K, E = ctx.dims
        need = ctx.needs_input_grad
        grad_out = grad_out.contiguous()
        if grad_out.dtype != x_perm.dtype:
            grad_out = grad_out.to(x_perm.dtype)
        with _stage("combine_bwd"):
            g_y, g_w = ops.combine_backward(grad_out, y, top_w, inv_pos)
        g_hidden = g_gu_w = g_dn_w = None
        g_gu = None
        if need[0] or need[3]:
            with _stage("down_dgrad"):
                g_gu = ops.down_proj_dgrad(g_y, gu, down, offs)
        if need[4]:
            with _stage("down_wgrad"):
                g_dn_w = ops.down_proj_wgrad(g_y, mid, offs, E)
        del g_y
        if need[0]:
            with _stage("gate_up_dgrad"):
                g_xp = ops.gate_up_dgrad(g_gu, gate_up, offs)
            with _stage("dispatch_bwd"):
                g_hidden = ops.dispatch_backward(g_xp, inv_pos, T, K)
            del g_xp
        if need[3]:
            with _stage("gate_up_wgrad"):
                g_gu_w = ops.gate_up_wgrad(g_gu, x_perm, offs, E)
        return g_hidden, None, (g_w if need[2] else None), g_gu_w, g_dn_w


# ------------------------------------------------- whole sparse MLP block


class _SparseMoEFunction(torch.autograd.Function):
    """Router + dropless experts as one autograd node (Qwen3MoeSparseMLP.forward).

    Outputs ``(out, router_logits)``: the logits stay graph-connected for the
    aux losses. In the backward the router's share of the input gradient is
    computed first and folded into the dispatch-backward sum, so the two input
    gradients are never added by a separate pass.
    """

    @staticmethod
    def forward(ctx, x, router_weight, gate_up_proj, down_proj, top_k, norm_topk_prob, logit_bias):
        E = gate_up_proj.shape[0]
        K = int(top_k)
        with _stage("router_fwd"):
            logits, top_w, top_i, top_w32, counts, psum, lse2 = ops.router_forward(
                x, router_weight, K, norm_topk_prob, logit_bias)
        with _stage("permute"):
            _, offs, _, inv_pos = ops.permute(top_i, E)
        with _stage("dispatch"):
            x_perm = ops.dispatch(x, inv_pos, K)
        with _stage("gate_up_fwd"):
            gu, mid = ops.gate_up_swiglu(x_perm, gate_up_proj, offs)
        with _stage("down_fwd"):
            y = ops.down_proj(mid, down_proj, offs)
        with _stage("combine"):
            out = ops.combine(y, top_w, inv_pos)
        ctx.save_for_backward(x, router_weight, logits, top_i, top_w32, top_w, gate_up_proj, down_proj, offs, inv_pos,
                              x_perm, gu, mid, y)
        ctx.norm_topk_prob = bool(norm_topk_prob)
        ctx.dims = (x.shape[0], K, E)
        ctx.mark_non_differentiable(counts, psum, lse2)
        ctx.set_materialize_grads(False)
        return out, logits, counts, psum, lse2

    @staticmethod
    def backward(ctx, g_out, g_logits, _gc, _gp, _gl):
        (x, rw, logits, top_i, top_w32, top_w, gate_up, down, offs, inv_pos, x_perm, gu, mid,
         y) = ctx.saved_tensors
        T, K, E = ctx.dims
        need = ctx.needs_input_grad
        if g_out is None and g_logits is None:
            return None, None, None, None, None, None, None
        if g_logits is not None:
            g_logits = g_logits.float().contiguous()
        g_x = g_rw = g_gu_w = g_dn_w = None
        g_tw = None
        g_y = None
        if g_out is not None:
            g_out = g_out.contiguous()
            if g_out.dtype != x_perm.dtype:
                g_out = g_out.to(x_perm.dtype)
            with _stage("combine_bwd"):
                g_y, g_tw = ops.combine_backward(g_out, y, top_w, inv_pos)
        gx_router = None
        if need[0] or need[1]:
            with _stage("router_bwd"):
                gx_router, g_rw = ops.router_backward(x, rw, logits, top_i, top_w32, g_tw, g_logits,
                                                      ctx.norm_topk_prob)
        if g_y is not None:
            g_gu = None
            if need[0] or need[2]:
                with _stage("down_dgrad"):
                    g_gu = ops.down_proj_dgrad(g_y, gu, down, offs)
            if need[3]:
                with _stage("down_wgrad"):
                    g_dn_w = ops.down_proj_wgrad(g_y, mid, offs, E)
            del g_y
            if need[0]:
                with _stage("gate_up_dgrad"):
                    g_xp = ops.gate_up_dgrad(g_gu, gate_up, offs)
                with _stage("dispatch_bwd"):
                    g_x = ops.dispatch_backward(g_xp, inv_pos, T, K, add=gx_router)
                del g_xp
            if need[2]:
                with _stage("gate_up_wgrad"):
                    g_gu_w = ops.gate_up_wgrad(g_gu, x_perm, offs, E)
        elif need[0]:
            g_x = gx_router
        return (g_x if need[0] else None), (g_rw if need[1] else None), g_gu_w, g_dn_w, None, None, None


def sparse_moe_block(hidden: torch.Tensor, router_weight: torch.Tensor, gate_up_proj: torch.Tensor,
                     down_proj: torch.Tensor, top_k: int, norm_topk_prob: bool = True,
                     logit_bias: torch.Tensor | None = None):
    """Router + experts of ``Qwen3MoeSparseMLP.forward`` (qwen3_moe.py:233-239) on HIP.

    ``hidden`` (T, H). Returns ``(out (T,H), router_logits (T,E) fp32,
    RouterStats)``; the logits carry the gradient of any aux loss. Same
    arithmetic as ``router_topk`` followed by ``moe_expert_ffn``.
    """
    assert hidden.dim() == 2 and router_weight.dim() == 2 and router_weight.shape[1] == hidden.shape[1]
    assert gate_up_proj.dim() == 3 and down_proj.dim() == 3
    assert 1 <= top_k <= router_weight.shape[0]
    require_gpu(hidden, router_weight, gate_up_proj, down_proj, logit_bias)
    dt = hidden.dtype
    x = hidden.contiguous()
    rw = router_weight.contiguous()
    if rw.dtype not in (torch.float32, torch.bfloat16):
        rw = rw.float()
    gu = gate_up_proj.to(dtype=dt).contiguous()
    dn = down_proj.to(dtype=dt).contiguous()
    if logit_bias is not None:
        logit_bias = logit_bias.float().contiguous()
    out, logits, counts, psum, lse2 = _SparseMoEFunction.apply(x, rw, gu, dn, int(top_k), bool(norm_topk_prob),
                                                                logit_bias)
    return out, logits, RouterStats(counts, psum, lse2, x.shape[0])


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
