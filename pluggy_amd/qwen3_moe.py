"""Module level of the MoE block: drop-ins for pluggy's Qwen3-MoE sparse FFN.

Same class names, constructor arguments, parameter names and shapes as
pluggy/models/qwen3_moe/qwen3_moe.py:152-239, so state_dicts interchange
(``router.weight`` (E,H), ``experts.gate_up_proj`` (E,2I,H),
``experts.down_proj`` (E,H,I)) and ``forward`` has the same contract:

* ``Qwen3MoeTopKRouter.forward(hidden (T,H)) -> (router_logits (T,E),
  top_weights (T,K) hidden.dtype, top_indices (T,K) int64)`` (:168-178)
* ``Qwen3MoeExperts.forward(hidden, top_indices, top_weights) -> (T,H)`` (:201-213)
* ``Qwen3MoeSparseMLP.forward(x (B,S,H)) -> (B,S,H)``, stashing
  ``last_router_logits`` (T,E) with its graph for the aux losses (:233-239)

Differences, both deliberate: router logits are fp32 whatever the autocast
state (the reference's are bf16 under the trainer's autocast), and top-k ties
go to the lower expert id. The routers also keep the fused per-layer
statistics of the last forward in ``last_stats``.
"""

from __future__ import annotations

import torch
from torch import nn

from .moe import RouterStats, moe_expert_ffn, router_topk, sparse_moe_block


class Qwen3MoeTopKRouter(nn.Module):
    def __init__(self, emb_dim: int, num_experts: int, top_k: int, norm_topk_prob: bool = True):
        super().__init__()
        assert 1 <= top_k <= num_experts
        self.top_k = top_k
        self.num_experts = num_experts
        self.norm_topk_prob = norm_topk_prob
        # zeros -> uniform softmax at init, as the reference (qwen3_moe.py:165-166)
        self.weight = nn.Parameter(torch.zeros(num_experts, emb_dim))
        # optional additive logit bias (E,) for routing stress tests; not a parameter
        self.logit_bias: torch.Tensor | None = None
        self.last_stats: RouterStats | None = None

    def forward(self, hidden_states: torch.Tensor):
        logits, w, idx, stats = router_topk(hidden_states, self.weight, self.top_k, self.norm_topk_prob,
                                            logit_bias=self.logit_bias, return_stats=True)
        self.last_stats = stats
        return logits, w, idx


class Qwen3MoeExperts(nn.Module):
    """Packed expert weights (E, ...); dropless top-k FFN on the HIP grouped kernels."""

    def __init__(self, emb_dim: int, moe_ffn_dim: int, num_experts: int):
        super().__init__()
        self.num_experts = num_experts
        self.emb_dim = emb_dim
        self.moe_ffn_dim = moe_ffn_dim
        self.gate_up_proj = nn.Parameter(torch.empty(num_experts, 2 * moe_ffn_dim, emb_dim))
        self.down_proj = nn.Parameter(torch.empty(num_experts, emb_dim, moe_ffn_dim))

    def forward(self, hidden_states: torch.Tensor, top_indices: torch.Tensor,
                top_weights: torch.Tensor) -> torch.Tensor:
        return moe_expert_ffn(hidden_states, top_indices, top_weights, self.gate_up_proj, self.down_proj)


class Qwen3MoeSparseMLP(nn.Module):
    def __init__(self, emb_dim: int, moe_ffn_dim: int, num_experts: int, top_k: int, norm_topk_prob: bool = True):
        super().__init__()
        self.router = Qwen3MoeTopKRouter(emb_dim, num_experts, top_k, norm_topk_prob)
        self.experts = Qwen3MoeExperts(emb_dim, moe_ffn_dim, num_experts)
        self.last_router_logits: torch.Tensor | None = None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        B, S, H = x.shape
        flat = x.reshape(B * S, H)
        r = self.router
        # router + experts as one autograd node (same arithmetic as calling
        # self.router then self.experts, which remain usable on their own)
        y, logits, stats = sparse_moe_block(flat, r.weight, self.experts.gate_up_proj, self.experts.down_proj,
                                            r.top_k, r.norm_topk_prob, logit_bias=r.logit_bias)
        r.last_stats = stats
        self.last_router_logits = logits
        return y.reshape(B, S, H)

