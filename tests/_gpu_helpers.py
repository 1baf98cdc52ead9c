"""Shared helpers of the GPU parity tests (CPU-side references and input builders)."""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from oracle import moe_oracle as O

DEV = "cuda"


def say(msg: str) -> None:
    print(msg, flush=True)


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def routing(T: int, K: int, E: int, seed: int = 0, mode: str = "uniform") -> torch.Tensor:
    """(T, K) int64 distinct expert ids per token.

    modes: "uniform" random; "zipf" heavy skew with empty experts;
    "one" every token picks expert 0 first; "low" only the K lowest ids.
    """
    g = gen(seed)
    scores = torch.rand(T, E, generator=g, dtype=torch.float64)
    if mode == "zipf":
        r = torch.randperm(E, generator=g).double()
        scores = scores.log() - 4.0 * torch.log(r + 1.0)
    elif mode == "one":
        scores[:, 0] += 10.0
    elif mode == "low":
        scores = -torch.arange(E, dtype=torch.float64).expand(T, E).clone()
    return scores.argsort(dim=1, descending=True)[:, :K].contiguous()


def seg_bounds(offs) -> list[tuple[int, int]]:
    offs = [int(v) for v in offs]
    out, lo = [], 0
    for hi in offs:
        out.append((lo, hi))
        lo = hi
    return out


def ref_grouped(A: torch.Tensor, W: torch.Tensor, offs, trans_w: bool) -> torch.Tensor:
    """fp64 per-expert A_e @ W[e]^T (trans_w) or A_e @ W[e]."""
    A = A.double().cpu()
    W = W.double().cpu()
    N = W.shape[1] if trans_w else W.shape[2]
    out = torch.zeros(A.shape[0], N, dtype=torch.float64)
    for e, (lo, hi) in enumerate(seg_bounds(offs)):
        if hi > lo:
            out[lo:hi] = A[lo:hi] @ (W[e].t() if trans_w else W[e])
    return out


def ref_wgrad(G: torch.Tensor, X: torch.Tensor, offs) -> torch.Tensor:
    """fp64 per-expert G_e^T @ X_e -> (E, G.cols, X.cols)."""
    G = G.double().cpu()
    X = X.double().cpu()
    b = seg_bounds(offs)
    out = torch.zeros(len(b), G.shape[1], X.shape[1], dtype=torch.float64)
    for e, (lo, hi) in enumerate(b):
        if hi > lo:
            out[e] = G[lo:hi].t() @ X[lo:hi]
    return out


def rel(a, b) -> float:
    return O.rel_l2(a, b)


def max_abs(a, b) -> float:
    return (a.detach().double().cpu() - b.detach().double().cpu()).abs().max().item()


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


def silu64(g: torch.Tensor) -> torch.Tensor:
    return F.silu(g.double())


def ref_moe_rows(x, idx, w, Wgu, Wdn, rows, gout=None):
    """fp64 forward (and expert-path backward) of the MoE FFN for selected token rows.

    Processes one expert at a time (weights converted once per hit expert).
    Returns ``out (R,H)``, and with ``gout``: ``dx_expert (R,H)`` and
    ``dw (R,K)`` = <gout[t], y_k[t]>.
    """
    rows = torch.as_tensor(rows, dtype=torch.long)
    R = rows.numel()
    K = idx.shape[1]
    I = Wgu.shape[1] // 2
    xr = x[rows].double()
    ir = idx[rows].cpu()
    wr = w[rows].double().cpu()
    H = xr.shape[1]
    out = torch.zeros(R, H, dtype=torch.float64)
    dx = torch.zeros(R, H, dtype=torch.float64)
    dw = torch.zeros(R, K, dtype=torch.float64)
    g = gout[rows].double() if gout is not None else None
    for e in torch.unique(ir).tolist():
        r_idx, k_idx = torch.nonzero(ir == e, as_tuple=True)
        Wg = Wgu[e].double()
        Wd = Wdn[e].double()
        xe = xr[r_idx]
        gu = xe @ Wg.t()
        gate, up = gu[:, :I], gu[:, I:]
        s = torch.sigmoid(gate)
        mid = gate * s * up
        y = mid @ Wd.t()
        out.index_add_(0, r_idx, wr[r_idx, k_idx].unsqueeze(1) * y)
        if g is not None:
            ge = g[r_idx]
            dw[r_idx, k_idx] = (ge * y).sum(1)
            dmid = (wr[r_idx, k_idx].unsqueeze(1) * ge) @ Wd
            dgate = dmid * up * s * (1 + gate * (1 - s))
            dup = dmid * gate * s
            dx.index_add_(0, r_idx, torch.cat([dgate, dup], 1) @ Wg)
    if gout is None:
        return out
    return out, dx, dw
