"""Pins the CPU oracle (oracle/moe_oracle.py) before it is trusted as the checker.

Each oracle function is checked against something that does not restate it:
brute force on small inputs, closed forms and invariants, the textbook special
case E = K = 1, torch autograd in fp64, and the reference's own test semantics
(grouped path == loop path, tests/kernels.py:118-163). Planted mistakes in the
oracle (monkeypatched on the CPU) must make at least one of these checks fail.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from hypothesis import given, settings
from hypothesis import strategies as st

from oracle import moe_oracle as O


def _inputs(T, H, E, I, dtype=torch.float32, seed=0, std=0.05):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g)
    wr = torch.randn(E, H, generator=g) * std
    gu = torch.randn(E, 2 * I, H, generator=g) * std
    dn = torch.randn(E, H, I, generator=g) * std
    return x.to(dtype), wr, gu.to(dtype), dn.to(dtype)


# ---------------------------------------------------------------- selection


def test_zero_logits_select_lowest_ids():
    """All-tie rows (the reference's zero-initialised router) pick experts 0..K-1."""
    idx = O.select_topk(np.zeros((5, 128), np.float32), 8)
    assert (idx == np.arange(8)).all()


@settings(max_examples=200, deadline=None)
@given(st.integers(1, 6), st.integers(1, 40), st.data())
def test_select_topk_brute_force(T, E, data):
    K = data.draw(st.integers(1, E))
    # few distinct values -> many ties
    vals = data.draw(st.lists(st.sampled_from([-1.5, 0.0, -0.0, 0.25, 3.0, 1e-30, -np.inf]),
                              min_size=T * E, max_size=T * E))
    logits = np.array(vals, np.float32).reshape(T, E)
    got = O.select_topk(logits, K)
    for t in range(T):
        brute = sorted(range(E), key=lambda e: (-float(logits[t, e]), e))[:K]
        assert list(got[t]) == brute


def test_router_weights_closed_form():
    x, wr, _, _ = _inputs(64, 32, 16, 8, seed=1)
    logits, w, idx, w32 = O.router_forward(x, wr, 4, norm_topk_prob=True)
    lg = (x.double() @ wr.double().t())
    sel = lg.gather(1, idx)
    ref = torch.softmax(sel, -1)          # the full-softmax denominator cancels
    assert torch.allclose(w32.double(), ref, rtol=1e-5, atol=1e-7)
    assert torch.allclose(w32.sum(-1), torch.ones(64), atol=1e-6)
    _, _, _, w32n = O.router_forward(x, wr, 4, norm_topk_prob=False)
    assert torch.allclose(w32n.double(), torch.softmax(lg, -1).gather(1, idx), rtol=1e-5, atol=1e-7)


def test_router_matches_torch_topk_without_ties():
    """Away from ties the tie rule is invisible: same set and order as torch.topk on probs."""
    x, wr, _, _ = _inputs(256, 64, 32, 8, seed=2)
    logits, _, idx, _ = O.router_forward(x, wr, 6)
    _, ti = torch.topk(torch.softmax(logits, -1), 6, dim=-1)
    assert torch.equal(ti, idx)


@pytest.mark.parametrize("norm", [True, False])
def test_router_backward_closed_form_vs_autograd(norm):
    g = torch.Generator().manual_seed(3)
    T, E, K = 50, 12, 4
    logits = torch.randn(T, E, generator=g, dtype=torch.float64, requires_grad=True)
    idx = torch.from_numpy(O.select_topk(logits.detach(), K))
    p = torch.softmax(logits, -1)
    w = p.gather(1, idx)
    if norm:
        w = w / w.sum(-1, keepdim=True)
    G = torch.randn(T, K, generator=g, dtype=torch.float64)
    Gl = torch.randn(T, E, generator=g, dtype=torch.float64)
    ((w * G).sum() + (logits * Gl).sum()).backward()
    dl = O.router_backward_closed_form(logits.detach(), idx, G, norm, grad_logits=Gl)
    assert torch.allclose(dl, logits.grad, rtol=1e-10, atol=1e-12)


# ---------------------------------------------------------------- aux stats


def test_aux_losses_uniform_router():
    E, K, T = 16, 4, 40
    z = [torch.zeros(T, E), torch.zeros(2 * T, E)]
    assert O.load_balancing_loss(z, E, K).item() == pytest.approx(K, rel=1e-6)
    assert O.router_z_loss(z).item() == pytest.approx(math.log(E) ** 2, rel=1e-6)
    # the reference's own selection (torch.topk) gives the same value on a uniform router
    tk = lambda lg, k: torch.topk(torch.softmax(lg, -1), k, dim=-1)[1]
    assert O.load_balancing_loss(z, E, K, select=tk).item() == pytest.approx(K, rel=1e-6)


def test_router_stats_are_additive_and_match_losses():
    g = torch.Generator().manual_seed(4)
    E, K = 16, 4
    layers = [torch.randn(30, E, generator=g), torch.randn(50, E, generator=g)]
    stats = [O.router_stats(lg, torch.from_numpy(O.select_topk(lg, K)), E) for lg in layers]
    N = 80
    counts = sum(s[0] for s in stats)
    psum = sum(s[1] for s in stats)
    lse2 = sum(s[2] for s in stats)
    assert counts.sum() == N * K
    lb = (torch.from_numpy(counts).double() / N * psum / N).sum() * E
    assert lb.item() == pytest.approx(O.load_balancing_loss(layers, E, K).item(), rel=1e-5)
    assert (lse2 / N).item() == pytest.approx(O.router_z_loss(layers).item(), rel=1e-5)


# -------------------------------------------------------------- permutation


@settings(max_examples=100, deadline=None)
@given(st.integers(1, 30), st.integers(1, 6), st.integers(1, 12), st.integers(0, 2**31 - 1))
def test_permute_brute_force(T, K, E, seed):
    K = min(K, E)
    rng = np.random.default_rng(seed)
    idx = np.stack([rng.permutation(E)[:K] for _ in range(T)])
    counts, offs, sp, inv = O.permute(idx, E)
    flat = idx.reshape(-1)
    brute = sorted(range(T * K), key=lambda q: (flat[q], q))
    assert list(sp) == brute
    assert (inv[sp] == np.arange(T * K)).all()
    assert list(counts) == [int((flat == e).sum()) for e in range(E)]
    assert list(offs) == list(np.cumsum([int((flat == e).sum()) for e in range(E)]))
    # within an expert, tokens are increasing (slot order does not matter)
    tok = sp // K
    for e in range(E):
        lo = 0 if e == 0 else offs[e - 1]
        assert (np.diff(tok[lo:offs[e]]) > 0).all()


# ---------------------------------------------------------------- expert FFN


def test_loop_matches_dense_fp64():
    x, wr, gu, dn = _inputs(96, 32, 8, 16, seed=5)
    _, w, idx, _ = O.router_forward(x, wr, 3)
    out = O.expert_ffn_loop(x, idx, w, gu, dn)
    ref = O.expert_ffn_dense_fp64(x, idx, w, gu, dn)
    assert O.rel_l2(out, ref) < 1e-6


def test_grouped_matches_loop_reference_semantics():
    """tests/kernels.py:118-163 at its own shapes and thresholds (bf16 hidden, fp32 weights)."""
    torch.manual_seed(0)
    T, H, I, E, K = 128, 64, 32, 8, 2
    hidden = torch.randn(T, H, dtype=torch.bfloat16)
    probs = F.softmax(torch.randn(T, E), dim=-1)
    top_w, top_i = torch.topk(probs, K, dim=-1)
    top_w = (top_w / top_w.sum(-1, keepdim=True)).to(torch.bfloat16)
    gate_up = torch.randn(E, 2 * I, H) * 0.02
    down = torch.randn(E, H, I) * 0.02
    grads = []
    outs = []
    for fn in (O.expert_ffn_loop, O.expert_ffn_grouped):
        h = hidden.clone().requires_grad_(True)
        a = gate_up.clone().requires_grad_(True)
        b = down.clone().requires_grad_(True)
        out = fn(h, top_i, top_w, a, b)
        out.float().pow(2).mean().backward()
        outs.append(out)
        grads.append((h.grad, a.grad, b.grad))
    assert O.rel_l2(outs[1], outs[0]) < 3e-2
    for g1, g0 in zip(grads[1], grads[0]):
        assert O.rel_l2(g1, g0) < 5e-2


def test_single_expert_is_dense_swiglu_mlp():
    """E = K = 1: the block is the textbook SwiGLU MLP down(silu(gate x) * up x)."""
    x, wr, gu, dn = _inputs(40, 24, 1, 16, seed=6)
    _, w, idx, _ = O.router_forward(x, wr, 1)
    assert (w == 1).all() and (idx == 0).all()
    out = O.expert_ffn_loop(x, idx, w, gu, dn)
    xd = x.double()
    ref = (F.silu(xd @ gu[0, :16].double().t()) * (xd @ gu[0, 16:].double().t())) @ dn[0].double().t()
    assert O.rel_l2(out, ref) < 1e-6


def test_k_equals_e_with_uniform_router_is_expert_average():
    E, I = 5, 8
    x, _, gu, dn = _inputs(30, 16, E, I, seed=7)
    _, w, idx, _ = O.router_forward(x, torch.zeros(E, 16), E)
    assert (idx == torch.arange(E)).all()
    out = O.expert_ffn_loop(x, idx, w, gu, dn)
    xd = x.double()
    ys = [(F.silu(xd @ gu[e, :I].double().t()) * (xd @ gu[e, I:].double().t())) @ dn[e].double().t()
          for e in range(E)]
    assert O.rel_l2(out, sum(ys) / E) < 1e-6


def test_sparse_mlp_shapes_and_logits():
    x, wr, gu, dn = _inputs(2 * 16, 32, 8, 16, seed=8)
    y, logits = O.sparse_mlp_forward(x.reshape(2, 16, 32), wr, gu, dn, 2)
    assert y.shape == (2, 16, 32) and logits.shape == (32, 8) and logits.dtype == torch.float32


# ------------------------------------------------------------ planted mistakes


def _checks_pass() -> bool:
    tests = [test_zero_logits_select_lowest_ids, test_router_weights_closed_form, test_loop_matches_dense_fp64,
             test_single_expert_is_dense_swiglu_mlp, test_k_equals_e_with_uniform_router_is_expert_average]
    try:
        for t in tests:
            t()
    except AssertionError:
        return False
    return True


def test_checks_pass_unplanted():
    assert _checks_pass()


@pytest.mark.parametrize("plant", ["swap_gate_up", "drop_renorm", "reverse_ties", "transpose_down"])
def test_planted_mistakes_are_caught(monkeypatch, plant):
    if plant == "swap_gate_up":
        monkeypatch.setattr(O, "swiglu", lambda g, u: F.silu(u) * g)
    elif plant == "drop_renorm":
        orig = O.router_forward

        def no_renorm(x, w, k, norm_topk_prob=True, logit_bias=None):
            return orig(x, w, k, False, logit_bias)
        monkeypatch.setattr(O, "router_forward", no_renorm)
    elif plant == "reverse_ties":
        def rev(logits, k):
            lg = np.asarray(logits.detach().numpy() if isinstance(logits, torch.Tensor) else logits, np.float32)
            E = lg.shape[1]
            order = np.argsort(-lg[:, ::-1], axis=1, kind="stable")
            return (E - 1 - order[:, :k]).astype(np.int64)
        monkeypatch.setattr(O, "select_topk", rev)
    elif plant == "transpose_down":
        orig_linear = F.linear

        def bad_loop(hidden, top_indices, top_weights, gate_up_proj, down_proj):
            T, H = hidden.shape
            out = torch.zeros(T, H, dtype=hidden.dtype)
            I = gate_up_proj.shape[1] // 2
            for t in range(T):
                for k in range(top_indices.shape[1]):
                    e = int(top_indices[t, k])
                    gu = orig_linear(hidden[t:t + 1], gate_up_proj[e])
                    m = F.silu(gu[:, :I]) * gu[:, I:]
                    # mistake: down_proj used as (I, H) by reshaping instead of transposing
                    y = m @ down_proj[e].reshape(I, H)
                    out[t] += (top_weights[t, k] * y[0]).to(out.dtype)
            return out
        monkeypatch.setattr(O, "expert_ffn_loop", bad_loop)
    assert not _checks_pass(), f"planted mistake {plant} went unnoticed"
