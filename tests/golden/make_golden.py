"""Writes the golden fixtures of the MoE block (tests/golden/*.npz) from the CPU oracle.

The reference holds no golden vectors for this path (its only MoE test,
tests/kernels.py:118-163, compares two of its own code paths), so the fixed
numbers here come from oracle/moe_oracle.py, whose functions are pinned by
brute force, closed forms and fp64 autograd in tests/test_oracle.py. Expected
values are computed in fp64. Run from the repository root:

    python tests/golden/make_golden.py

Fixtures (all arrays plain numbers, loadable with numpy's allow_pickle=False):

* ``block_fp32.npz`` -- the shape of the reference's own MoE test scaled down
  (T=64, H=32, I=16, E=8, K=2, fp32): inputs, fp32 logits, selected ids,
  renormalised weights, counts/offs/sorted_pair/inv_pos, the block output and
  the gradients of sum(out * grad_out) + sum(logits * grad_logits) with respect
  to x, the router weight and both expert weights.
* ``ties.npz`` -- integer-valued logits with many exact ties (and -inf), the
  ids the lower-expert-id rule selects, and the renormalised weights. Row 0 is
  all zeros (the reference's zero-initialised router); -1e30 stands in for
  -inf so that the GPU test can produce these logits exactly as x . I^T.
* ``permute_skew.npz`` -- skewed expert ids with empty experts and the stable
  counting-sort outputs.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import moe_oracle as O  # noqa: E402


def f32(t: torch.Tensor) -> np.ndarray:
    """fp64 truth stored as fp32 (7 significant digits; the checks are 1e-4 relative)."""
    return t.detach().float().numpy()


def block_fp32(seed: int = 7):
    T, H, I, E, K = 64, 32, 16, 8, 2
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g)
    wr = torch.randn(E, H, generator=g) * 0.3
    gu = torch.randn(E, 2 * I, H, generator=g) * 0.2
    dn = torch.randn(E, H, I, generator=g) * 0.2
    gout = torch.randn(T, H, generator=g)
    glog = torch.randn(T, E, generator=g) * 0.1
    logits32, _, idx, _ = O.router_forward(x, wr, K, norm_topk_prob=True)
    # fp64 truth given the selection
    xd, wrd, gud, dnd = (t.double().requires_grad_(True) for t in (x, wr, gu, dn))
    lg = xd @ wrd.t()
    w = torch.softmax(lg, -1).gather(1, idx)
    w = w / w.sum(-1, keepdim=True)
    out = O.expert_ffn_dense_fp64(xd, idx, w, gud, dnd)
    ((out * gout.double()).sum() + (lg * glog.double()).sum()).backward()
    counts, offs, sp, inv = O.permute(idx, E)
    return dict(T=T, H=H, I=I, E=E, K=K, x=x.numpy(), router_weight=wr.numpy(), gate_up_proj=gu.numpy(),
                down_proj=dn.numpy(), grad_out=gout.numpy(), grad_logits=glog.numpy(),
                logits=logits32.numpy(), top_indices=idx.numpy(), top_weights=f32(w),
                counts=counts, offs=offs, sorted_pair=sp, inv_pos=inv, out=f32(out),
                grad_x=f32(xd.grad), grad_router_weight=f32(wrd.grad), grad_gate_up_proj=f32(gud.grad),
                grad_down_proj=f32(dnd.grad))


def ties(seed: int = 8):
    T, E, K = 48, 40, 6
    rng = np.random.default_rng(seed)
    logits = rng.choice(np.array([-3.0, -1.0, 0.0, 0.0, 2.0, 2.0, 5.0], np.float32), size=(T, E))
    logits[0, :] = 0.0                      # the zero-initialised router: a full tie
    logits[1, ::3] = -1e30                  # effectively -inf, and exact through x . I^T
    idx = O.select_topk(logits, K)
    lg = torch.from_numpy(logits.astype(np.float64))
    w = torch.softmax(lg, -1).gather(1, torch.from_numpy(idx))
    w = (w / w.sum(-1, keepdim=True)).numpy()
    return dict(T=T, E=E, K=K, logits=logits, top_indices=idx, top_weights=w)


def permute_skew(seed: int = 9):
    T, E, K = 96, 16, 4
    rng = np.random.default_rng(seed)
    q = (np.arange(E) + 1.0) ** -1.5
    q[[3, 11]] = 0.0                         # two experts nobody picks
    q /= q.sum()
    idx = np.stack([rng.choice(E, size=K, replace=False, p=q) for _ in range(T)]).astype(np.int64)
    counts, offs, sp, inv = O.permute(idx, E)
    return dict(T=T, E=E, K=K, top_indices=idx, counts=counts, offs=offs, sorted_pair=sp, inv_pos=inv)


def main():
    for name, fn in (("block_fp32", block_fp32), ("ties", ties), ("permute_skew", permute_skew)):
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **fn())
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
