"""pluggy_amd: MI355X-native (gfx950) Qwen3-MoE sparse FFN block for pluggy.

Drop-in replacements for the reference block (pluggy/models/qwen3_moe/qwen3_moe.py:152-239)
and operator (pluggy/kernels/moe.py:127-168), backed by hand-written HIP kernels
in ``libpmoe.so`` (C ABI in ``include/pmoe.h``).
"""

from .moe import RouterStats, moe_expert_ffn, moe_sublayer, router_topk, sparse_moe_block, weight_cast_cache
from .qwen3_moe import Qwen3MoeExperts, Qwen3MoeSparseMLP, Qwen3MoeTopKRouter
from .router_aux import (
    expert_counts_from_stats,
    install_stats_aux,
    load_balancing_loss,
    load_balancing_loss_from_stats,
    router_z_loss_from_stats,
    select_lower_id,
)

__all__ = [
    "Qwen3MoeExperts",
    "Qwen3MoeSparseMLP",
    "Qwen3MoeTopKRouter",
    "RouterStats",
    "expert_counts_from_stats",
    "install_stats_aux",
    "load_balancing_loss",
    "load_balancing_loss_from_stats",
    "moe_expert_ffn",
    "moe_sublayer",
    "router_topk",
    "router_z_loss_from_stats",
    "select_lower_id",
    "sparse_moe_block",
    "weight_cast_cache",
]
