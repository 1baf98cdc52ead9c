"""CPU tests of the aux-loss helpers that follow the kernels' routing (pluggy_amd.router_aux).

Each is checked against the oracle's restatement of the reference formulas
(qwen3_moe.py:285-316, :417-426) with the oracle's lower-id tie rule, against
fp64 autograd for the gradient, and against the closed forms of the all-tie
(zero router) case. RouterStats are built from oracle.router_stats, i.e. what
the fused router emits, so no kernel runs here.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from pluggy_amd import (
    Qwen3MoeSparseMLP,
    RouterStats,
    expert_counts_from_stats,
    install_stats_aux,
    load_balancing_loss,
    load_balancing_loss_from_stats,
    router_z_loss_from_stats,
    select_lower_id,
)


def _stats(logits: torch.Tensor, K: int) -> RouterStats:
    E = logits.shape[1]
    idx = O.select_topk(logits.detach(), K)
    counts, psum, lse2 = O.router_stats(logits.detach(), torch.from_numpy(idx), E)
    return RouterStats(torch.from_numpy(counts).to(torch.int32), psum.float(), lse2.float().reshape(1),
                       logits.shape[0])


def _layers(seed: int, sizes, E: int, ties: bool = False) -> list[torch.Tensor]:
    g = torch.Generator().manual_seed(seed)
    out = []
    for T in sizes:
        lg = torch.randn(T, E, generator=g)
        if ties:  # coarse values: many exact ties across the k-th boundary
            lg = (lg * 2).round() / 2
        out.append(lg)
    return out


@pytest.mark.parametrize("ties", [False, True])
def test_lb_from_stats_matches_oracle_value_and_grad(ties):
    E, K = 16, 4
    layers = _layers(0, (37, 64, 5), E, ties)
    stats = [_stats(lg, K) for lg in layers]
    # oracle: the reference formula with the lower-id selection, fp64 autograd
    ref_in = [lg.double().requires_grad_(True) for lg in layers]
    ref = O.load_balancing_loss(ref_in, E, K)
    ref.backward()
    got_in = [lg.clone().requires_grad_(True) for lg in layers]
    got = load_balancing_loss_from_stats(got_in, stats, E)
    got.backward()
    assert abs(got.item() - ref.item()) <= 1e-5 * abs(ref.item())
    for a, b in zip(got_in, ref_in):
        assert O.rel_l2(a.grad, b.grad) < 1e-5
        assert (a.grad.double() - b.grad).abs().max().item() < 1e-7


def test_lb_uniform_router_closed_form():
    """Zero router: every token ties everywhere, the kernels pick ids 0..K-1.
    LB = K exactly, and dLB/dl_tj = (1[j < K] - K/E) / N."""
    E, K, T = 32, 8, 100
    lg = torch.zeros(T, E, requires_grad=True)
    st = _stats(lg, K)
    assert st.expert_counts.tolist() == [T] * K + [0] * (E - K)
    loss = load_balancing_loss_from_stats([lg], [st], E)
    assert abs(loss.item() - K) < 1e-6
    loss.backward()
    want = (torch.arange(E) < K).double().sub(K / E).div(T).expand(T, E)
    assert (lg.grad.double() - want).abs().max().item() < 1e-9


def test_lb_from_stats_needs_matching_rows():
    E, K = 8, 2
    a, b = _layers(1, (10, 12), E)
    with pytest.raises(AssertionError):
        load_balancing_loss_from_stats([a, b], [_stats(a, K), _stats(a, K)], E)


def test_lb_drop_in_selects_like_the_kernels():
    E, K = 16, 4
    layers = _layers(2, (50, 33), E, ties=True)
    # the stable descending sort reproduces the oracle's selection (pinned by brute force in test_oracle)
    for lg in layers:
        assert np.array_equal(select_lower_id(lg, K).numpy(), O.select_topk(lg, K))
    ref_in = [lg.double().requires_grad_(True) for lg in layers]
    ref = O.load_balancing_loss(ref_in, E, K)
    ref.backward()
    got_in = [lg.clone().requires_grad_(True) for lg in layers]
    got = load_balancing_loss(got_in, E, K)
    got.backward()
    assert abs(got.item() - ref.item()) <= 1e-5 * abs(ref.item())
    for a, b in zip(got_in, ref_in):
        assert O.rel_l2(a.grad, b.grad) < 1e-5
    # the zero router: the lower-id rule gives exactly K as well
    assert abs(load_balancing_loss([torch.zeros(7, E)], E, K).item() - K) < 1e-6


def test_planted_tie_rule_is_caught():
    """A selection that breaks ties toward the higher id changes the value on
    tied logits, so the agreement above is not vacuous."""
    E, K, T = 8, 2, 20
    lg = torch.zeros(T, E)
    hi = O.load_balancing_loss([lg], E, K, select=lambda l, k: torch.arange(E - 1, E - 1 - k, -1).expand(T, k))
    lo = load_balancing_loss([lg], E, K)
    assert abs(hi.item() - lo.item()) < 1e-6  # the value alone cannot tell at uniform probabilities
    lg2 = torch.zeros(T, E, requires_grad=True)
    st = _stats(lg2, K)
    load_balancing_loss_from_stats([lg2], [st], E).backward()
    lg3 = torch.zeros(T, E, dtype=torch.float64, requires_grad=True)
    O.load_balancing_loss([lg3], E, K, select=lambda l, k: torch.arange(E - 1, E - 1 - k, -1).expand(T, k)).backward()
    assert (lg2.grad.double() - lg3.grad).abs().max().item() > 1e-3  # ... but the gradient can


def test_counts_and_z_from_stats():
    E, K = 16, 4
    layers = _layers(3, (40, 24), E)
    stats = [_stats(lg, K) for lg in layers]
    counts = expert_counts_from_stats(stats)
    want = sum(np.bincount(O.select_topk(lg, K).reshape(-1), minlength=E) for lg in layers)
    assert counts.dtype == torch.float32 and counts.tolist() == want.astype(np.float32).tolist()
    assert not counts.requires_grad
    z = router_z_loss_from_stats(stats)
    assert abs(z.item() - O.router_z_loss(layers).item()) < 1e-5 * O.router_z_loss(layers).item()
    assert expert_counts_from_stats([]) is None


class _Block(torch.nn.Module):
    def __init__(self, ffn):
        super().__init__()
        self.ffn = ffn


class _RefModelStandIn(torch.nn.Module):
    """The attributes of a reference Qwen3Moe (qwen3_moe.py:319-344, :409-444)
    that the aux harvest reads; no reference code is imported."""

    def __init__(self, mlps, E, K):
        super().__init__()
        self.blocks = torch.nn.ModuleList(_Block(m) for m in mlps)
        self.num_experts, self.top_k = E, K
        self.router_aux_loss_coef, self.router_z_loss_coef = 1e-3, 1e-3
        self._router_logits = [m.last_router_logits for m in mlps]


def test_install_stats_aux_on_a_model_stand_in():
    H, I, E, K = 8, 4, 16, 4
    layers = [lg.requires_grad_(True) for lg in _layers(4, (30, 30), E, ties=True)]
    mlps = []
    for lg in layers:
        m = Qwen3MoeSparseMLP(H, I, E, K)
        m.last_router_logits = lg
        m.router.last_stats = _stats(lg, K)
        mlps.append(m)
    model = _RefModelStandIn(mlps, E, K)
    install_stats_aux(model)
    model._update_expert_counts(model._router_logits)
    want = sum(np.bincount(O.select_topk(lg.detach(), K).reshape(-1), minlength=E) for lg in layers)
    assert model.last_tokens_per_expert.tolist() == want.astype(np.float32).tolist()
    aux = model.aux_loss()
    ref_in = [lg.detach().double().requires_grad_(True) for lg in layers]
    ref = 1e-3 * O.load_balancing_loss(ref_in, E, K) + 1e-3 * O.router_z_loss(ref_in)
    assert abs(aux.item() - ref.item()) <= 1e-5 * abs(ref.item())
    aux.backward()
    ref.backward()
    for a, b in zip(layers, ref_in):
        assert O.rel_l2(a.grad, b.grad) < 1e-5
