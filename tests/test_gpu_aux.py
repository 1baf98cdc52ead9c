"""GPU: the load-balance loss and expert counts follow the kernels' own routing.

Reference: load_balancing_loss / _update_expert_counts / aux_loss
(pluggy/models/qwen3_moe/qwen3_moe.py:285-308, :417-444). The fused router's
counts and probability sums feed ``load_balancing_loss_from_stats``; its value
and logits gradient are compared with the oracle's restatement of the
reference formula under the lower-id tie rule, on the GPU's own fp32 logits:
at config 4 (Zipf-skewed routing, full size) and with the zero-initialised
router, where every token ties (closed form: LB = K, dLB/dl_tj =
(1[j < K] - K/E) / N).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from tests._gpu_helpers import DEV, rel, say

pytestmark = pytest.mark.gpu


def _run(cfg_id: int, zero_router: bool):
    import pluggy_amd
    from pluggy_amd.workloads import CONFIGS, make_inputs

    cfg = CONFIGS[cfg_id]
    inp = make_inputs(cfg, device=DEV)
    T, H, E, K, I = cfg.tokens, cfg.hidden, cfg.experts, cfg.top_k, cfg.inter
    mlp = pluggy_amd.Qwen3MoeSparseMLP(H, I, E, K).to(DEV)
    with torch.no_grad():
        if not zero_router:
            mlp.router.weight.copy_(inp["router_weight"])
        mlp.experts.gate_up_proj.data = inp["gate_up_proj"]
        mlp.experts.down_proj.data = inp["down_proj"]
    mlp.router.logit_bias = inp.get("logit_bias")
    mlp(inp["x"].reshape(1, T, H))
    logits = mlp.last_router_logits
    logits.retain_grad()
    stats = mlp.router.last_stats
    return mlp, logits, stats, E, K, T


@pytest.mark.parametrize("case", ["config4-zipf", "zero-router"])
def test_load_balance_from_stats_follows_kernel_routing(case):
    import pluggy_amd

    mlp, logits, stats, E, K, T = _run(4 if case == "config4-zipf" else 2, case == "zero-router")
    say(f"aux {case}: T={T} E={E} K={K}")
    lb = pluggy_amd.load_balancing_loss_from_stats([logits], [stats], E)
    lb.backward()
    lg_cpu = logits.detach().cpu()
    # the kernels' counts are the oracle selection on the same fp32 logits, bit for bit
    want_counts = np.bincount(O.select_topk(lg_cpu, K).reshape(-1), minlength=E)
    assert np.array_equal(stats.expert_counts.cpu().numpy(), want_counts)
    ref_in = lg_cpu.double().requires_grad_(True)
    ref = O.load_balancing_loss([ref_in], E, K)
    ref.backward()
    r = rel(logits.grad, ref_in.grad)
    mabs = (logits.grad.double().cpu() - ref_in.grad).abs().max().item()
    say(f"  LB {lb.item():.6f} vs oracle {ref.item():.6f}; grad rel {r:.2e} max-abs {mabs:.2e}")
    assert abs(lb.item() - ref.item()) <= 1e-5 * abs(ref.item())
    # fp32 gradients of magnitude <= E/N: rel-L2 1e-5 and max-abs 1e-7 against fp64
    assert r < 1e-5 and mabs < 1e-7
    if case == "zero-router":
        assert abs(lb.item() - K) < 1e-5
        want = ((torch.arange(E) < K).double() - K / E) / T
        assert (logits.grad.double().cpu() - want.expand(T, E)).abs().max().item() < 1e-9
    # the drop-in with the reference's signature agrees on the same logits
    lb2 = pluggy_amd.load_balancing_loss([logits.detach()], E, K)
    assert abs(lb2.item() - ref.item()) <= 1e-5 * abs(ref.item())
    counts = pluggy_amd.expert_counts_from_stats([stats])
    assert np.array_equal(counts.cpu().numpy(), want_counts.astype(np.float32))
