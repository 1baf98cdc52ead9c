"""CPU oracle for pluggy's Qwen3-MoE sparse FFN block: TEST INFRASTRUCTURE ONLY.

This module restates, on the CPU, the arithmetic of the reference block so the
HIP path in ``pluggy_amd`` can be checked against it. Nothing in the product
imports it; ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg are its only users.

Reference files restated (paths relative to the sonnetx/pluggy checkout):

* ``pluggy/models/qwen3_moe/qwen3_moe.py:152-178``  router (linear, fp32 softmax,
  top-k, renormalise, cast)
* ``pluggy/kernels/moe.py:38-65``   per-expert loop path (the reference CPU path)
* ``pluggy/kernels/moe.py:68-124``  sorted/grouped path (stable sort by expert,
  bincount, cumsum offsets, two grouped GEMMs, weighted scatter-add)
* ``pluggy/kernels/swiglu.py:14-16``  silu(gate) * up
* ``pluggy/models/qwen3_moe/qwen3_moe.py:285-316``  load-balance and z losses
* ``pluggy/models/qwen3_moe/qwen3_moe.py:417-426``  per-expert token counts

Two precision choices are made on top of the reference code and are part of the
contract this oracle defines:

1. Router logits are fp32: ``F.linear(x.float(), W.float())``. (Outside the
   trainer's autocast the reference would reject bf16 x with an fp32 weight.)
2. Top-k selection ranks the fp32 *logits* with ties broken by the lower expert
   id (a stable descending sort). ``torch.topk`` on probabilities, which the
   reference calls, leaves tie order unspecified; softmax is monotone, so the
   two agree whenever no two probabilities tie across the k-th boundary.

How each function is pinned (tests/test_oracle.py): brute force on small inputs
(``sorted(range(P), key=(expert, pair))`` for the permutation, an fp64 dense
per-token sum for the FFN), closed forms (uniform router gives load-balance loss
K exactly and z-loss (ln E)^2; zero logits select experts 0..K-1; K == E gives
the average of every expert's output), the textbook special case E = K = 1
(a dense SwiGLU MLP), torch.autograd.gradcheck in fp64 for the closed-form router
backward, and the reference's own test semantics (grouped path == loop path at
rel-L2 3e-2 / 5e-2, tests/kernels.py:118-163). Planted mistakes in this module
(dropped renormalisation, swapped gate/up, tie broken the other way) are shown
to fail those checks.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

__all__ = [
    "select_topk",
    "router_forward",
    "router_backward_closed_form",
    "router_stats",
    "permute",
    "swiglu",
    "expert_ffn_loop",
    "expert_ffn_grouped",
    "expert_ffn_dense_fp64",
    "sparse_mlp_forward",
    "load_balancing_loss",
    "router_z_loss",
    "rel_l2",
]


def rel_l2(a: torch.Tensor, b: torch.Tensor) -> float:
    """||a - b|| / ||b|| in fp64 (tests/kernels.py:22-25 uses the same measure)."""
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    den = b.norm().item()
    num = (a - b).norm().item()
    if den == 0.0:
        return 0.0 if num == 0.0 else float("inf")
    return num / den


# ---------------------------------------------------------------- router ----


def select_topk(logits, k: int) -> np.ndarray:
    """Top-k expert ids per row of fp32 logits, descending, ties -> lower id.

    Follows the selection step of ``qwen3_moe.py:174`` (``torch.topk`` over the
    softmax) with the tie rule stated in the module docstring. ``-x`` is exact
    in fp32, so a stable ascending sort of ``-logits`` is a stable descending
    sort of ``logits``.
    """
    if isinstance(logits, torch.Tensor):
        logits = logits.detach().float().cpu().numpy()
    logits = np.asarray(logits, dtype=np.float32)
    order = np.argsort(-logits, axis=1, kind="stable")
    return order[:, :k].astype(np.int64)


def router_forward(x: torch.Tensor, weight: torch.Tensor, top_k: int,
                   norm_topk_prob: bool = True, logit_bias: torch.Tensor | None = None):
    """Restates ``Qwen3MoeTopKRouter.forward`` (qwen3_moe.py:168-178).

    Returns ``(logits fp32 (T,E), top_weights x.dtype (T,K), top_indices int64
    (T,K), top_weights_fp32 (T,K))``. Differentiable w.r.t. ``x`` and ``weight``
    through logits and top_weights (the indices are integers). ``logit_bias``
    (E,) is the skewed-routing stress bias of the benchmark; the reference
    router has none (None reproduces it exactly).
    """
    logits = F.linear(x.float(), weight.float())                     # :172
    if logit_bias is not None:
        logits = logits + logit_bias.float()
    probs = F.softmax(logits, dim=-1, dtype=torch.float32)           # :173
    idx = torch.from_numpy(select_topk(logits, top_k))               # :174
    w = probs.gather(1, idx)
    if norm_topk_prob:                                               # :175-176
        w = w / w.sum(dim=-1, keepdim=True)
    return logits, w.to(dtype=x.dtype), idx, w                       # :177


def router_backward_closed_form(logits: torch.Tensor, idx: torch.Tensor,
                                grad_w: torch.Tensor, norm_topk_prob: bool,
                                grad_logits: torch.Tensor | None = None):
    """d(loss)/d(logits) of the router given d(loss)/d(top_weights).

    With renormalisation the full softmax denominator cancels and
    ``w = softmax(logits[S])`` over the selected set S, so
    ``dl_k = w_k (G_k - sum_{m in S} w_m G_m)`` on S and 0 elsewhere. Without it
    ``w_k = p_k`` and ``dl_j = p_j (g_j - sum_{k in S} p_k G_k)`` with g the
    scatter of G onto S. Pinned against autograd in tests/test_oracle.py.
    """
    logits = logits.double()
    G = grad_w.double()
    p = torch.softmax(logits, dim=-1)
    if norm_topk_prob:
        ls = logits.gather(1, idx)
        w = torch.softmax(ls, dim=-1)
        inner = (w * G).sum(-1, keepdim=True)
        dl = torch.zeros_like(logits)
        dl.scatter_(1, idx, w * (G - inner))
    else:
        g = torch.zeros_like(logits)
        g.scatter_(1, idx, G)
        inner = (p.gather(1, idx) * G).sum(-1, keepdim=True)
        dl = p * (g - inner)
    if grad_logits is not None:
        dl = dl + grad_logits.double()
    return dl


def router_stats(logits: torch.Tensor, idx: torch.Tensor, num_experts: int):
    """Per-layer additive aux statistics the fused router emits.

    ``counts[e]`` = number of (token, slot) picks of e (qwen3_moe.py:417-426,
    summed over slots), ``prob_sum[e]`` = sum_t softmax(logits)_t,e (the
    numerator of ``router_prob`` at qwen3_moe.py:303) and ``lse_sq_sum`` =
    sum_t logsumexp(logits_t)^2 (qwen3_moe.py:316 before the mean).
    """
    logits = logits.double()
    counts = np.bincount(idx.reshape(-1).numpy(), minlength=num_experts)
    prob_sum = torch.softmax(logits, dim=-1).sum(0)
    lse_sq = torch.logsumexp(logits, dim=-1).square().sum()
    return counts.astype(np.int64), prob_sum, lse_sq


def load_balancing_loss(router_logits: list, num_experts: int, top_k: int,
                        select=None) -> torch.Tensor:
    """Restates ``load_balancing_loss`` (qwen3_moe.py:285-308).

    ``select`` picks the top-k ids from fp32 logits; it defaults to this
    oracle's tie rule (the reference calls ``torch.topk`` on probabilities).
    """
    if not router_logits:
        return torch.tensor(0.0)
    logits = torch.cat([g.float() for g in router_logits], dim=0)
    probs = F.softmax(logits, dim=-1)
    if select is None:
        top_idx = torch.from_numpy(select_topk(logits, top_k))
    else:
        top_idx = select(logits, top_k)
    mask = F.one_hot(top_idx, num_experts).float()                   # (N,K,E)
    tokens_per_expert = mask.mean(dim=0)                             # (K,E)
    router_prob = probs.mean(dim=0)                                  # (E,)
    return (tokens_per_expert * router_prob.unsqueeze(0)).sum() * num_experts


def router_z_loss(router_logits: list) -> torch.Tensor:
    """Restates ``router_z_loss`` (qwen3_moe.py:311-316)."""
    if not router_logits:
        return torch.tensor(0.0)
    logits = torch.cat([g.float() for g in router_logits], dim=0)
    return torch.square(torch.logsumexp(logits, dim=-1)).mean()


# ------------------------------------------------------------ permutation ---


def permute(top_indices, num_experts: int):
    """Stable counting sort of the T*K (token, slot) pairs by expert id.

    Restates ``moe.py:89-108``: flat pair q = t*K + k, ``order =
    argsort(expert, stable)``, ``counts = bincount``, ``offs = cumsum`` (int32,
    inclusive end offsets; an empty expert repeats the previous offset).
    Returns ``counts (E,) int64, offs (E,) int32, sorted_pair (P,) int32,
    inv_pos (P,) int32`` with ``inv_pos[sorted_pair[p]] = p``. The sorted token
    of position p is ``sorted_pair[p] // K``.
    """
    if isinstance(top_indices, torch.Tensor):
        top_indices = top_indices.detach().cpu().numpy()
    flat = np.asarray(top_indices).reshape(-1).astype(np.int64)
    order = np.argsort(flat, kind="stable")
    counts = np.bincount(flat, minlength=num_experts).astype(np.int64)
    offs = np.cumsum(counts).astype(np.int32)
    inv = np.empty(flat.size, dtype=np.int32)
    inv[order] = np.arange(flat.size, dtype=np.int32)
    return counts, offs, order.astype(np.int32), inv


# ----------------------------------------------------------- expert FFN ----


def swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """``silu(gate) * up`` (swiglu.py:14-16)."""
    return F.silu(gate) * up


def expert_ffn_loop(hidden, top_indices, top_weights, gate_up_proj, down_proj):
    """Restates the per-expert loop path ``_expert_ffn_loop`` (moe.py:38-65).

    This is the path the reference takes whenever CUDA is absent
    (``_has_grouped_mm``, moe.py:34-35), i.e. the reference CPU path.
    For each hit expert e in ascending order, tokens are taken in (slot, token)
    order as ``torch.where`` over the (K, T) mask yields them; the SwiGLU output
    is scaled by the routing weight in activation dtype and scatter-added.
    """
    T, H = hidden.shape
    E = gate_up_proj.shape[0]
    out = torch.zeros(T, H, dtype=hidden.dtype)
    mask = F.one_hot(top_indices, num_classes=E).permute(2, 1, 0)   # (E,K,T)
    hit = mask.sum(dim=(-1, -2)).nonzero(as_tuple=False).flatten()
    gu = gate_up_proj.to(dtype=hidden.dtype)
    dn = down_proj.to(dtype=hidden.dtype)
    for e in hit.tolist():
        k_pos, tok = torch.where(mask[e])
        if tok.numel() == 0:
            continue
        gate, up = F.linear(hidden[tok], gu[e]).chunk(2, dim=-1)
        y = F.linear(swiglu(gate, up), dn[e])
        y = y * top_weights[tok, k_pos, None]
        out = out.index_add(0, tok, y.to(dtype=out.dtype))
    return out


def expert_ffn_grouped(hidden, top_indices, top_weights, gate_up_proj, down_proj):
    """Restates the sorted/grouped path ``_expert_ffn_grouped`` (moe.py:68-124).

    Each expert's rows are contiguous after the stable sort; the grouped GEMM
    over ``offs`` is evaluated one segment at a time with ``F.linear``.
    """
    T, H = hidden.shape
    E = gate_up_proj.shape[0]
    K = top_indices.shape[1]
    dtype = hidden.dtype
    counts, offs, order, _ = permute(top_indices, E)
    order_t = torch.from_numpy(order.astype(np.int64))
    sorted_token = order_t // K
    sorted_w = top_weights.reshape(-1)[order_t]
    sorted_h = hidden[sorted_token]
    gu = gate_up_proj.to(dtype=dtype)
    dn = down_proj.to(dtype=dtype)
    pieces = []
    start = 0
    for e in range(E):
        end = int(offs[e])
        if end > start:
            gate, up = F.linear(sorted_h[start:end], gu[e]).chunk(2, dim=-1)
            pieces.append(F.linear(swiglu(gate, up), dn[e]))
        start = end
    down = torch.cat(pieces, 0) if pieces else sorted_h.new_zeros(0, H)
    down = down * sorted_w.unsqueeze(1).to(dtype=dtype)
    out = torch.zeros(T, H, dtype=dtype)
    return out.index_add(0, sorted_token, down)


def expert_ffn_dense_fp64(hidden, top_indices, top_weights, gate_up_proj, down_proj):
    """Brute-force fp64 truth: y_t = sum_k w_tk * Wd[e](silu(Wg[e] x_t) * Wu[e] x_t)."""
    x = hidden.double()
    gu = gate_up_proj.double()
    dn = down_proj.double()
    w = top_weights.double()
    T, H = x.shape
    K = top_indices.shape[1]
    I = gu.shape[1] // 2
    out = torch.zeros(T, H, dtype=torch.float64)
    for k in range(K):
        e = top_indices[:, k]
        g = torch.einsum("th,tih->ti", x, gu[e, :I, :])
        u = torch.einsum("th,tih->ti", x, gu[e, I:, :])
        y = torch.einsum("ti,thi->th", F.silu(g) * u, dn[e])
        out = out + w[:, k:k + 1] * y
    return out


def sparse_mlp_forward(x, router_weight, gate_up_proj, down_proj, top_k: int,
                       norm_topk_prob: bool = True, ffn=expert_ffn_loop, logit_bias=None):
    """Restates ``Qwen3MoeSparseMLP.forward`` (qwen3_moe.py:233-239).

    Returns ``(y (B,S,H), router_logits (T,E))``. ``logit_bias`` as in
    ``router_forward`` (the benchmark's skewed routing; None in the reference).
    """
    B, S, H = x.shape
    flat = x.reshape(B * S, H)
    logits, w, idx, _ = router_forward(flat, router_weight, top_k, norm_topk_prob, logit_bias)
    y = ffn(flat, idx, w, gate_up_proj, down_proj)
    return y.reshape(B, S, H), logits
