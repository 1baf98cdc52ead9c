"""The CPU oracle reproduces the committed golden fixtures (tests/golden/*.npz).

The fixtures were written by tests/golden/make_golden.py; this test pins the
oracle to those fixed numbers so a later change to it cannot drift silently.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

from oracle import moe_oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name: str) -> dict:
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_block_fixture():
    g = load("block_fp32")
    K, E = int(g["K"]), int(g["E"])
    x, wr = torch.from_numpy(g["x"]), torch.from_numpy(g["router_weight"])
    gu, dn = torch.from_numpy(g["gate_up_proj"]), torch.from_numpy(g["down_proj"])
    logits, _, idx, w32 = O.router_forward(x, wr, K, norm_topk_prob=True)
    assert np.array_equal(idx.numpy(), g["top_indices"])
    assert np.allclose(logits.numpy(), g["logits"], rtol=1e-6, atol=1e-6)
    assert np.allclose(w32.numpy(), g["top_weights"], rtol=1e-5, atol=1e-7)
    counts, offs, sp, inv = O.permute(idx, E)
    for k, v in (("counts", counts), ("offs", offs), ("sorted_pair", sp), ("inv_pos", inv)):
        assert np.array_equal(v, g[k]), k
    # the reference CPU path (loop) in fp64 reproduces the output and expert gradients
    xd, wrd, gud, dnd = (t.double().requires_grad_(True) for t in (x, wr, gu, dn))
    lg = xd @ wrd.t()
    w = torch.softmax(lg, -1).gather(1, idx)
    w = w / w.sum(-1, keepdim=True)
    out = O.expert_ffn_loop(xd, idx, w, gud, dnd)
    ((out * torch.from_numpy(g["grad_out"]).double()).sum()
     + (lg * torch.from_numpy(g["grad_logits"]).double()).sum()).backward()
    for name, got in (("out", out), ("grad_x", xd.grad), ("grad_router_weight", wrd.grad),
                      ("grad_gate_up_proj", gud.grad), ("grad_down_proj", dnd.grad)):
        assert O.rel_l2(got, torch.from_numpy(g[name])) < 1e-6, name


def test_ties_fixture():
    g = load("ties")
    assert np.array_equal(O.select_topk(g["logits"], int(g["K"])), g["top_indices"])
    assert (g["top_indices"][0] == np.arange(int(g["K"]))).all()


def test_permute_fixture():
    g = load("permute_skew")
    counts, offs, sp, inv = O.permute(g["top_indices"], int(g["E"]))
    assert (g["counts"] == 0).sum() >= 2
    for k, v in (("counts", counts), ("offs", offs), ("sorted_pair", sp), ("inv_pos", inv)):
        assert np.array_equal(v, g[k]), k
