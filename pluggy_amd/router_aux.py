"""Router aux losses and expert counts that follow the kernels' own routing.

The reference computes its load-balance loss and its per-expert counts by
selecting experts again with ``torch.topk`` on the probabilities
(pluggy/models/qwen3_moe/qwen3_moe.py:299-303, :417-426). The fused router
selects by fp32 logit with ties going to the lower expert id, and it already
counts its picks (``RouterStats.expert_counts``). At a tie the two selections
can differ, and the reference zero-initialises the router (:165-166, :399), so
at step 0 every token is a full tie: there the reference's loss would push down
experts the kernels never routed to. The functions here use the kernels'
selection instead:

* ``load_balancing_loss_from_stats`` - the value and the logits gradient of
  ``load_balancing_loss`` with ``f_e`` taken from the fused router's counts;
  the value comes from the additive statistics (no pass over the logits) and
  the backward is one fused pass per layer.
* ``load_balancing_loss`` - the reference's signature over a list of logits,
  selecting with the kernels' rule (a stable descending sort of the fp32
  logits), for callers that only hold the logits.
* ``router_z_loss_from_stats`` / ``expert_counts_from_stats`` - the z-loss value
  and the counts of ``_update_expert_counts`` from the same statistics.
* ``install_stats_aux(model)`` - points a reference ``Qwen3Moe``'s
  ``_update_expert_counts`` and ``aux_loss`` at the functions above.
"""

from __future__ import annotations

import types

import torch
import torch.nn.functional as F

from .moe import RouterStats


def _totals(stats: list[RouterStats]) -> tuple[int, torch.Tensor, torch.Tensor]:
    n = sum(int(s.tokens) for s in stats)
    counts = torch.stack([s.expert_counts for s in stats]).sum(0).to(torch.float32)
    psum = torch.stack([s.prob_sum for s in stats]).sum(0).to(torch.float32)
    return n, counts, psum


class _LoadBalanceFromStats(torch.autograd.Function):
    """LB = E * sum_e (c_e / N) * (psum_e / N), c the kernels' pick counts.

    dLB/dl_tj = (E / N) * p_tj * (f_j - sum_e f_e p_te) with f = c / N and
    p = softmax(l_t) (the counts carry no gradient, as the reference's one-hot
    mask does not)."""

    @staticmethod
    def forward(ctx, f, psum, n, num_experts, *logits):
        ctx.save_for_backward(f, *logits)
        ctx.scale = num_experts / n
        return (f * psum).sum() * (num_experts / n)

    @staticmethod
    def backward(ctx, g):
        f, *logits = ctx.saved_tensors
        grads = []
        for lg in logits:
            if lg is None or not ctx.needs_input_grad[4 + len(grads)]:
                grads.append(None)
                continue
            p = torch.softmax(lg.float(), dim=-1)
            d = p * (f - (p * f).sum(-1, keepdim=True)) * (g * ctx.scale)
            grads.append(d.to(lg.dtype))
        return (None, None, None, None, *grads)


def load_balancing_loss_from_stats(router_logits: list[torch.Tensor], stats: list[RouterStats],
                                   num_experts: int) -> torch.Tensor:
    """``load_balancing_loss`` (qwen3_moe.py:285-308) with the kernels' selection.

    ``router_logits`` are the layers' ``last_router_logits`` (graph-connected)
    and ``stats`` their routers' ``last_stats``, in any layer order as long as
    both lists hold the same layers. Returns the scalar (fp32) loss; its
    gradient reaches every layer's logits. The value is ``E * sum_e f_e P_e``
    with ``f_e`` = picks of e / N over all K slots and ``P_e`` the mean router
    probability, as in the reference.
    """
    if not router_logits:
        return torch.tensor(0.0)
    assert len(router_logits) == len(stats), "one RouterStats per layer's logits"
    n, counts, psum = _totals(stats)
    assert n == sum(int(lg.shape[0]) for lg in router_logits), "stats and logits cover different rows"
    f = counts / n
    return _LoadBalanceFromStats.apply(f, psum, n, num_experts, *router_logits)


def select_lower_id(logits: torch.Tensor, top_k: int) -> torch.Tensor:
    """Top-k expert ids of fp32 logits with ties going to the lower id (the
    fused router's rule): a stable descending sort keeps equal logits in id
    order."""
    return torch.sort(logits.float(), dim=-1, descending=True, stable=True).indices[:, :top_k]


def load_balancing_loss(router_logits: list[torch.Tensor], num_experts: int, top_k: int) -> torch.Tensor:
    """Drop-in for ``load_balancing_loss`` (qwen3_moe.py:285-308): same
    arguments and value, with the experts selected by the fused router's rule
    (``select_lower_id``) instead of ``torch.topk``; differentiable through the
    probabilities as the reference."""
    if not router_logits:
        return torch.tensor(0.0)
    logits = torch.cat([g.float() for g in router_logits], dim=0)
    probs = F.softmax(logits, dim=-1)
    idx = select_lower_id(logits, top_k)
    counts = torch.zeros(num_experts, device=logits.device, dtype=torch.float32)
    counts.scatter_add_(0, idx.reshape(-1), torch.ones(idx.numel(), device=logits.device))
    return (counts / logits.shape[0] * probs.mean(dim=0)).sum() * num_experts


def router_z_loss_from_stats(stats: list[RouterStats]) -> torch.Tensor:
    """Value of ``router_z_loss`` (qwen3_moe.py:311-316): mean_t logsumexp(logits_t)^2
    (no gradient: the logits-based ``router_z_loss`` carries it)."""
    n = sum(int(s.tokens) for s in stats)
    return torch.stack([s.lse_sq_sum.to(torch.float32).reshape(()) for s in stats]).sum() / n


def expert_counts_from_stats(stats: list[RouterStats]) -> torch.Tensor | None:
    """What ``Qwen3Moe._update_expert_counts`` (qwen3_moe.py:417-426) stores in
    ``last_tokens_per_expert``: picks per expert over all layers and slots,
    as a detached fp32 (E,) tensor, here from the kernels' own counts."""
    if not stats:
        return None
    return torch.stack([s.expert_counts for s in stats]).sum(0).to(torch.float32).detach()


def _sparse_routers(model):
    from .qwen3_moe import Qwen3MoeSparseMLP

    return [b.ffn for b in model.blocks
            if isinstance(b.ffn, Qwen3MoeSparseMLP) and b.ffn.last_router_logits is not None]


def install_stats_aux(model) -> None:
    """Make a reference ``Qwen3Moe`` (qwen3_moe.py:319-489) take its expert
    counts and load-balance loss from the kernels' routing.

    Replaces, on this instance only, ``_update_expert_counts`` (:417-426) by
    ``expert_counts_from_stats`` and ``aux_loss`` (:428-444) by the same
    combination ``router_aux_loss_coef * LB + router_z_loss_coef * Z`` with LB
    from ``load_balancing_loss_from_stats``. The z-loss keeps the reference's
    logits-based formula (it does not depend on the selection). The model's
    sparse blocks must be ``pluggy_amd.Qwen3MoeSparseMLP`` (installed as in the
    module-level integration), whose routers keep ``last_stats``.
    """
    def _update_expert_counts(self, router_logits):
        mlps = _sparse_routers(self)
        self.last_tokens_per_expert = expert_counts_from_stats([m.router.last_stats for m in mlps]) if mlps else None

    def aux_loss(self):
        logits = getattr(self, "_router_logits", None)
        if not logits:
            return None
        mlps = _sparse_routers(self)
        loss = torch.zeros((), device=logits[0].device)
        if self.router_aux_loss_coef != 0.0:
            loss = loss + self.router_aux_loss_coef * load_balancing_loss_from_stats(
                [m.last_router_logits for m in mlps], [m.router.last_stats for m in mlps], self.num_experts)
        if self.router_z_loss_coef != 0.0:
            z_logits = torch.cat([g.float() for g in logits], dim=0)
            loss = loss + self.router_z_loss_coef * torch.square(torch.logsumexp(z_logits, dim=-1)).mean()
        return loss

    model._update_expert_counts = types.MethodType(_update_expert_counts, model)
    model.aux_loss = types.MethodType(aux_loss, model)
