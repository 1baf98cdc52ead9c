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


def ref_grouped(A: torch.Tensor, W: torch.Tensor, offs, trans_w: bool, dev=DEV) -> torch.Tensor:
    """fp64 per-expert A_e @ W[e]^T (trans_w) or A_e @ W[e], evaluated with torch's fp64
    operations on ``dev`` (independent of the HIP kernels); returned on the CPU."""
    A = A.to(dev).double()
    N = W.shape[1] if trans_w else W.shape[2]
    out = torch.zeros(A.shape[0], N, dtype=torch.float64, device=dev)
    for e, (lo, hi) in enumerate(seg_bounds(offs)):
        if hi > lo:
            We = W[e].to(dev).double()
            out[lo:hi] = A[lo:hi] @ (We.t() if trans_w else We)
    return out.cpu()


def ref_wgrad(G: torch.Tensor, X: torch.Tensor, offs, dev=DEV) -> torch.Tensor:
    """fp64 per-expert G_e^T @ X_e -> (E, G.cols, X.cols), on ``dev``; returned on the CPU."""
    G = G.to(dev).double()
    X = X.to(dev).double()
    b = seg_bounds(offs)
    out = torch.zeros(len(b), G.shape[1], X.shape[1], dtype=torch.float64, device=dev)
    for e, (lo, hi) in enumerate(b):
        if hi > lo:
            out[e] = G[lo:hi].t() @ X[lo:hi]
    return out.cpu()


def _pair(a, b):
    """Both operands in fp64 on one device: the GPU when either lives there (full-size
    tensors stay off the host), else the CPU."""
    dev = a.device if a.is_cuda else (b.device if b.is_cuda else torch.device("cpu"))
    return a.detach().to(dev).double(), b.detach().to(dev).double()


def rel(a, b) -> float:
    """||a - b|| / ||b|| in fp64 (the oracle's rel_l2, on the operands' device)."""
    a, b = _pair(a, b)
    den = b.norm().item()
    num = (a - b).norm().item()
    if den == 0.0:
        return 0.0 if num == 0.0 else float("inf")
    return num / den


def max_abs(a, b) -> float:
    a, b = _pair(a, b)
    return (a - b).abs().max().item() if a.numel() else 0.0


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


def silu64(g: torch.Tensor) -> torch.Tensor:
    return F.silu(g.double())


# Max-abs bounds stated next to every rel-L2 check: no element may be off by more
# than this fraction of the reference's largest magnitude (bf16 outputs carry one
# bf16 rounding of themselves and of their bf16 intermediates; fp32 arithmetic
# only summation-order error).
MAX_ABS_FRAC = {torch.bfloat16: 2e-2, torch.float16: 3e-3, torch.float32: 1e-4}


def check_close(name: str, got, ref, rel_tol: float, max_abs_frac: float) -> tuple[float, float]:
    """Assert rel-L2 <= rel_tol and max |got - ref| <= max_abs_frac * max |ref|; print both."""
    r = rel(got, ref)
    m = max_abs(got, ref)
    scale = ref.detach().abs().max().item() if ref.numel() else 0.0
    say(f"  {name}: rel={r:.2e} maxabs={m:.2e} (bound {max_abs_frac * scale:.2e})")
    assert r < rel_tol, f"{name}: rel-L2 {r:.3e} >= {rel_tol:.1e}"
    assert m <= max_abs_frac * scale, f"{name}: max-abs {m:.3e} > {max_abs_frac:.0e} x {scale:.3e}"
    return r, m


def ref_layer_fp64(x, Wr, Wgu, Wdn, idx, logits, norm: bool, gout=None, dev=DEV):
    """fp64 truth of the whole MoE layer, given the routing ids and the router's fp32 logits.

    Evaluated with torch's fp64 operations on ``dev`` (independent of the HIP
    kernels; the GPU makes full-size configurations affordable), one expert at
    a time. Returns a dict: ``out`` (T,H); with ``gout`` also ``dx`` (expert
    path + router path), ``dw`` (T,K) = <gout[t], y_k[t]>, ``dWr`` (E,H),
    ``dWgu`` (E,2I,H), ``dWdn`` (E,H,I).
    """
    T, H = x.shape
    K = idx.shape[1]
    E, I2, _ = Wgu.shape
    I = I2 // 2
    xd = x.to(dev).double()
    lg = logits.to(dev).double()
    ix = idx.to(dev)
    w = torch.softmax(lg, -1).gather(1, ix)
    if norm:
        w = w / w.sum(-1, keepdim=True)
    res = {"out": torch.zeros(T, H, dtype=torch.float64, device=dev)}
    back = gout is not None
    if back:
        g = gout.to(dev).double()
        res.update(dx=torch.zeros(T, H, dtype=torch.float64, device=dev),
                   dw=torch.zeros(T, K, dtype=torch.float64, device=dev),
                   dWgu=torch.zeros(E, I2, H, dtype=torch.float64, device=dev),
                   dWdn=torch.zeros(E, H, I, dtype=torch.float64, device=dev))
    flat = ix.reshape(-1)
    order = torch.argsort(flat, stable=True)
    ends = torch.cumsum(torch.bincount(flat, minlength=E), 0).tolist()
    lo = 0
    for e, hi in enumerate(ends):
        if hi == lo:
            continue
        q = order[lo:hi]
        lo = hi
        t, k = q // K, q % K
        Wg = Wgu[e].to(dev).double()
        Wd = Wdn[e].to(dev).double()
        xe = xd[t]
        gu = xe @ Wg.t()
        gate, up = gu[:, :I], gu[:, I:]
        s = torch.sigmoid(gate)
        mid = gate * s * up
        y = mid @ Wd.t()
        we = w[t, k].unsqueeze(1)
        res["out"].index_add_(0, t, we * y)
        if back:
            ge = g[t]
            res["dw"][t, k] = (ge * y).sum(1)
            dy = we * ge
            res["dWdn"][e] = dy.t() @ mid
            dmid = dy @ Wd
            dgu = torch.cat([dmid * up * s * (1 + gate * (1 - s)), dmid * gate * s], 1)
            res["dWgu"][e] = dgu.t() @ xe
            res["dx"].index_add_(0, t, dgu @ Wg)
    if back:
        dl = O.router_backward_closed_form(lg, ix, res["dw"], norm)
        Wrd = Wr.to(dev).double()
        res["dx"] += dl @ Wrd
        res["dWr"] = dl.t() @ xd
    return res
