"""Synthetic MoE-layer workloads (the five configurations of the benchmark).

Every tensor is drawn on the CPU from a seeded ``torch.Generator`` in fp32 and
then cast, so a CPU run and a GPU run see bit-identical inputs. Draw order is
fixed: x, router weight, gate_up_proj, down_proj (seed 0), upstream grad
(seed 1), skew bias (seed 2).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch


@dataclass(frozen=True)
class MoEConfig:
    name: str
    tokens: int            # T = batch * seq
    hidden: int            # H (emb_dim)
    experts: int           # E (num_experts)
    top_k: int             # K
    inter: int             # I (moe_ffn_dim)
    dtype: torch.dtype     # activation / expert-weight dtype
    backward: bool         # fwd+bwd or forward only
    skew: float = 0.0      # Zipf exponent of the additive router-logit bias (0 = none)
    batch: int = 1
    norm_topk_prob: bool = True
    notes: str = field(default="", compare=False)

    @property
    def pairs(self) -> int:
        return self.tokens * self.top_k

    def gemm_flops(self) -> float:
        """Algorithmic expert-GEMM FLOPs: 2*P*H*2I + 2*P*I*H forward, x3 with backward."""
        f = 2.0 * self.pairs * self.hidden * 2 * self.inter + 2.0 * self.pairs * self.inter * self.hidden
        return 3.0 * f if self.backward else f

    def router_flops(self) -> float:
        f = 2.0 * self.tokens * self.hidden * self.experts
        return 3.0 * f if self.backward else f


CONFIGS = {
    1: MoEConfig("small-fp32-fwd", 2048, 512, 8, 2, 1024, torch.float32, False,
                 notes="reference CPU-runnable case; bit-exact routing"),
    2: MoEConfig("qwen3-30b-a3b", 8192, 2048, 128, 8, 768, torch.bfloat16, True, batch=4,
                 notes="headline: batch 4 x seq 2048"),
    3: MoEConfig("qwen3-235b-a22b", 16384, 4096, 128, 8, 1536, torch.bfloat16, True),
    4: MoEConfig("skewed-zipf1.2", 8192, 2048, 128, 8, 768, torch.bfloat16, True, skew=1.2, batch=4),
    5: MoEConfig("decode-t64", 64, 2048, 128, 8, 768, torch.bfloat16, False),
}


# Not a BASELINE.json configuration: the MoE layer of pluggy's own MoE training
# config (configs/qwen3_moe_climbmix.json:4-19; micro batch 2 x seq 4096).
CLIMBMIX = MoEConfig("qwen3-moe-climbmix", 8192, 1024, 32, 4, 512, torch.bfloat16, True, batch=2,
                     notes="pluggy's qwen3_moe_climbmix training shape")


def zipf_logit_bias(num_experts: int, s: float, seed: int = 2) -> torch.Tensor:
    """b_e = ln q_e - mean(ln q), q_e ~ (r_e + 1)^-s, r a seeded permutation of ids."""
    g = torch.Generator().manual_seed(seed)
    r = torch.randperm(num_experts, generator=g).double()
    lnq = -s * torch.log(r + 1.0)
    return (lnq - lnq.mean()).float()


def make_inputs(cfg: MoEConfig, device="cpu", std: float = 0.02, tokens: int | None = None):
    """Seeded inputs for one configuration.

    Returns a dict with ``x (T,H)``, ``router_weight (E,H) fp32``,
    ``gate_up_proj (E,2I,H)``, ``down_proj (E,H,I)``, ``grad_out (T,H)`` (when
    the config has a backward) and ``logit_bias (E,)`` (when skewed).
    ``tokens`` overrides T (the first ``tokens`` rows of the full draw are NOT
    used; a smaller draw is made so the CPU baseline can run a bounded sample).
    """
    T = cfg.tokens if tokens is None else tokens
    g = torch.Generator().manual_seed(0)
    x = torch.randn(T, cfg.hidden, generator=g)
    wr = torch.randn(cfg.experts, cfg.hidden, generator=g) * std
    gu = torch.randn(cfg.experts, 2 * cfg.inter, cfg.hidden, generator=g) * std
    dn = torch.randn(cfg.experts, cfg.hidden, cfg.inter, generator=g) * std
    out = {
        "x": x.to(cfg.dtype).to(device),
        "router_weight": wr.to(device),
        "gate_up_proj": gu.to(cfg.dtype).to(device),
        "down_proj": dn.to(cfg.dtype).to(device),
    }
    if cfg.backward:
        g1 = torch.Generator().manual_seed(1)
        out["grad_out"] = torch.randn(T, cfg.hidden, generator=g1).to(cfg.dtype).to(device)
    if cfg.skew:
        out["logit_bias"] = zipf_logit_bias(cfg.experts, cfg.skew).to(device)
    return out


def mib(nbytes: float) -> float:
    return nbytes / (1 << 20)


def dispatch_bytes(cfg: MoEConfig) -> float:
    """Compulsory bytes of the row gather: read T*H, write P*H (+ int32 indices)."""
    es = cfg.dtype.itemsize
    return cfg.tokens * cfg.hidden * es + cfg.pairs * cfg.hidden * es + cfg.pairs * 4


def combine_bytes(cfg: MoEConfig) -> float:
    """Compulsory bytes of the combine: read the P weighted rows (P*H) and their
    positions (P int32), write T*H (the routing weight is already in the rows)."""
    es = cfg.dtype.itemsize
    return cfg.pairs * cfg.hidden * es + cfg.pairs * 4 + cfg.tokens * cfg.hidden * es


def log2_ceil(n: int) -> int:
    return max(0, math.ceil(math.log2(max(1, n))))
