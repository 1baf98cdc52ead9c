"""The HIP path against the committed golden fixtures (tests/golden/*.npz).

Routing ids, counts, offsets and the permutation bit-exact; fp32 values and
gradients within rel-L2 1e-4 of the fp64 truth stored in the fixtures.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests._gpu_helpers import DEV, max_abs, rel, say, to_np
from tests.test_golden import load

pytestmark = pytest.mark.gpu


def test_block_fixture_fp32():
    import pluggy_amd
    from pluggy_amd import ops

    g = load("block_fp32")
    T, H, I, E, K = (int(g[k]) for k in ("T", "H", "I", "E", "K"))
    say(f"golden block T={T} H={H} I={I} E={E} K={K} fp32")
    mlp = pluggy_amd.Qwen3MoeSparseMLP(H, I, E, K).to(DEV)
    with torch.no_grad():
        mlp.router.weight.copy_(torch.from_numpy(g["router_weight"]))
        mlp.experts.gate_up_proj.copy_(torch.from_numpy(g["gate_up_proj"]))
        mlp.experts.down_proj.copy_(torch.from_numpy(g["down_proj"]))
    x = torch.from_numpy(g["x"]).to(DEV).reshape(1, T, H).requires_grad_(True)
    out = mlp(x)
    logits = mlp.last_router_logits
    loss = (out.reshape(T, H) * torch.from_numpy(g["grad_out"]).to(DEV)).sum() + \
        (logits * torch.from_numpy(g["grad_logits"]).to(DEV)).sum()
    loss.backward()
    assert rel(logits, torch.from_numpy(g["logits"])) < 1e-5
    _, w, idx = mlp.router(x.detach().reshape(T, H))
    assert np.array_equal(to_np(idx), g["top_indices"])
    assert rel(w, torch.from_numpy(g["top_weights"])) < 1e-5
    assert np.array_equal(to_np(mlp.router.last_stats.expert_counts), g["counts"].astype(np.int32))
    counts, offs, sp, inv = ops.permute(idx, E)
    for k, v in (("counts", counts), ("offs", offs), ("sorted_pair", sp), ("inv_pos", inv)):
        assert np.array_equal(to_np(v), g[k].astype(np.int32)), k
    for name, got in (("out", out.reshape(T, H)), ("grad_x", x.grad.reshape(T, H)),
                      ("grad_router_weight", mlp.router.weight.grad),
                      ("grad_gate_up_proj", mlp.experts.gate_up_proj.grad),
                      ("grad_down_proj", mlp.experts.down_proj.grad)):
        ref = torch.from_numpy(g[name])
        r = rel(got, ref)
        say(f"  {name}: rel={r:.2e} maxabs={max_abs(got, ref):.2e}")
        assert r < 1e-4, name


def test_ties_fixture_through_the_router():
    """logits = x . I^T reproduces the tie fixture exactly; ids follow the lower-id rule."""
    from pluggy_amd import ops

    g = load("ties")
    T, E, K = (int(g[k]) for k in ("T", "E", "K"))
    x = torch.from_numpy(g["logits"]).to(DEV)
    eye = torch.eye(E, dtype=torch.float32, device=DEV)
    logits, _, ti, tw32, counts, _, _ = ops.router_forward(x, eye, K, True)
    assert torch.equal(logits.cpu(), torch.from_numpy(g["logits"]))
    assert np.array_equal(to_np(ti), g["top_indices"])
    assert rel(tw32, torch.from_numpy(g["top_weights"])) < 1e-6
    assert np.array_equal(to_np(counts), np.bincount(g["top_indices"].reshape(-1), minlength=E))


def test_permute_fixture():
    from pluggy_amd import ops

    g = load("permute_skew")
    counts, offs, sp, inv = ops.permute(torch.from_numpy(g["top_indices"]).to(DEV), int(g["E"]))
    for k, v in (("counts", counts), ("offs", offs), ("sorted_pair", sp), ("inv_pos", inv)):
        assert np.array_equal(to_np(v), g[k].astype(np.int32)), k
