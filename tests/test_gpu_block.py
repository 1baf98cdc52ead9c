"""GPU parity of the whole MoE block (router + experts, forward + backward).

* The reference's own test semantics (tests/kernels.py:118-163): same shapes,
  dtypes and loss, compared with the oracle's loop path (the reference CPU
  path) at the reference thresholds and at the north-star rel-L2 <= 1e-2.
* The benchmark configurations at full size: routing and permutation bit-exact
  (given the GPU's fp32 logits), router statistics against the oracle, every
  output row, the whole input gradient and every weight gradient against fp64
  truth with rel-L2 and max-abs bounds, bitwise run-to-run determinism.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from tests._gpu_helpers import (DEV, MAX_ABS_FRAC, check_close, gen, max_abs, ref_layer_fp64, rel, say,
                                to_np)

pytestmark = pytest.mark.gpu


def _mod():
    import pluggy_amd
    return pluggy_amd


def test_reference_kernels_semantics():
    """tests/kernels.py:118-163: T=128 H=64 I=32 E=8 K=2, bf16 hidden, fp32 weights x0.02."""
    pa = _mod()
    torch.manual_seed(0)
    T, H, I, E, K = 128, 64, 32, 8, 2
    hidden = torch.randn(T, H, dtype=torch.bfloat16)
    logits = torch.randn(T, E)
    probs = torch.softmax(logits, dim=-1)
    top_w, top_i = torch.topk(probs, K, dim=-1)
    top_w = (top_w / top_w.sum(-1, keepdim=True)).to(torch.bfloat16)
    gate_up = torch.randn(E, 2 * I, H) * 0.02
    down = torch.randn(E, H, I) * 0.02

    h1 = hidden.clone().requires_grad_(True)
    gu1 = gate_up.clone().requires_grad_(True)
    dn1 = down.clone().requires_grad_(True)
    out1 = O.expert_ffn_loop(h1, top_i, top_w, gu1, dn1)
    out1.float().pow(2).mean().backward()

    h2 = hidden.to(DEV).requires_grad_(True)
    gu2 = gate_up.to(DEV).requires_grad_(True)
    dn2 = down.to(DEV).requires_grad_(True)
    out2 = pa.moe_expert_ffn(h2, top_i.to(DEV), top_w.to(DEV), gu2, dn2)
    out2.float().pow(2).mean().backward()
    r = [rel(out2, out1), rel(h2.grad, h1.grad), rel(gu2.grad, gu1.grad), rel(dn2.grad, dn1.grad)]
    say(f"moe: rel_out={r[0]:.2e} dh={r[1]:.2e} dgu={r[2]:.2e} ddn={r[3]:.2e}")
    assert out2.dtype == torch.bfloat16 and gu2.grad.dtype == torch.float32
    assert r[0] < 3e-2 and r[1] < 5e-2 and r[2] < 5e-2 and r[3] < 5e-2
    assert max(r) < 1e-2


def _ref_block_fp64(x, Wr, Wgu, Wdn, idx, norm, gout, glogits):
    """fp64 autograd of the block given the routing ids (values and all grads)."""
    x = x.double().requires_grad_(True)
    Wr = Wr.double().requires_grad_(True)
    Wgu = Wgu.double().requires_grad_(True)
    Wdn = Wdn.double().requires_grad_(True)
    logits = x @ Wr.t()
    p = torch.softmax(logits, -1)
    w = p.gather(1, idx)
    if norm:
        w = w / w.sum(-1, keepdim=True)
    T, K = idx.shape
    I = Wgu.shape[1] // 2
    out = torch.zeros_like(x)
    for e in torch.unique(idx).tolist():
        r, k = torch.nonzero(idx == e, as_tuple=True)
        gu = x[r] @ Wgu[e].t()
        y = (torch.nn.functional.silu(gu[:, :I]) * gu[:, I:]) @ Wdn[e].t()
        out = out.index_add(0, r, w[r, k].unsqueeze(1) * y)
    loss = (out * gout.double()).sum() + (logits * glogits.double()).sum()
    loss.backward()
    return out.detach(), logits.detach(), x.grad, Wr.grad, Wgu.grad, Wdn.grad


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("norm", [True, False])
def test_sparse_mlp_module(dtype, norm):
    """Module forward/backward vs fp64 autograd, including the aux-loss path through the logits."""
    pa = _mod()
    B, S, H, E, K, I = 2, 256, 256, 16, 4, 128
    say(f"sparse MLP B={B} S={S} H={H} E={E} K={K} I={I} {dtype} norm={norm}")
    g = gen(21)
    x = torch.randn(B, S, H, generator=g).to(dtype)
    Wr = torch.randn(E, H, generator=g) * 0.05
    Wgu = (torch.randn(E, 2 * I, H, generator=g) * 0.05).to(dtype)
    Wdn = (torch.randn(E, H, I, generator=g) * 0.05).to(dtype)
    gout = torch.randn(B * S, H, generator=g).to(dtype)
    glog = torch.randn(B * S, E, generator=g) * 0.01

    mlp = pa.Qwen3MoeSparseMLP(H, I, E, K, norm).to(DEV)
    with torch.no_grad():
        mlp.router.weight.copy_(Wr)
        mlp.experts.gate_up_proj.data = Wgu.to(DEV)
        mlp.experts.down_proj.data = Wdn.to(DEV)
    xg = x.to(DEV).requires_grad_(True)
    out = mlp(xg)
    assert out.shape == (B, S, H) and out.dtype == dtype
    logits = mlp.last_router_logits
    assert logits.shape == (B * S, E) and logits.dtype == torch.float32
    loss = (out.reshape(B * S, H).float() * gout.to(DEV).float()).sum() + (logits * glog.to(DEV)).sum()
    loss.backward()

    idx = torch.from_numpy(O.select_topk(logits.detach().cpu(), K))
    ref = _ref_block_fp64(x.reshape(B * S, H), Wr, Wgu, Wdn, idx, norm, gout, glog)
    names = ["out", "logits", "dx", "dWr", "dWgu", "dWdn"]
    got = [out.reshape(B * S, H), logits, xg.grad.reshape(B * S, H), mlp.router.weight.grad,
           mlp.experts.gate_up_proj.grad, mlp.experts.down_proj.grad]
    tol = 1e-2 if dtype == torch.bfloat16 else 1e-4
    for n, a, b in zip(names, got, ref):
        check_close(n, a, b, tol, MAX_ABS_FRAC[dtype])
    # routing parity with the oracle on its own CPU logits (exempting genuine near-ties)
    _check_routing_vs_cpu(x.reshape(B * S, H), Wr, logits.detach().cpu(), K)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_sparse_mlp_module_any_size(dtype):
    """Hidden and intermediate sizes that are not multiples of 8 (the reference
    takes any): the host layer zero-pads them to the kernels' 16-byte rows and
    slices the result; values and every gradient vs fp64 autograd as above,
    and moe_expert_ffn on the same routing."""
    pa = _mod()
    B, S, H, E, K, I = 2, 96, 100, 8, 2, 52
    say(f"sparse MLP any size H={H} I={I} E={E} K={K} {dtype}")
    g = gen(23)
    x = torch.randn(B, S, H, generator=g).to(dtype)
    Wr = torch.randn(E, H, generator=g) * 0.05
    Wgu = (torch.randn(E, 2 * I, H, generator=g) * 0.05).to(dtype)
    Wdn = (torch.randn(E, H, I, generator=g) * 0.05).to(dtype)
    gout = torch.randn(B * S, H, generator=g).to(dtype)
    glog = torch.randn(B * S, E, generator=g) * 0.01
    mlp = pa.Qwen3MoeSparseMLP(H, I, E, K).to(DEV)
    with torch.no_grad():
        mlp.router.weight.copy_(Wr)
        mlp.experts.gate_up_proj.data = Wgu.to(DEV)
        mlp.experts.down_proj.data = Wdn.to(DEV)
    xg = x.to(DEV).requires_grad_(True)
    out = mlp(xg)
    assert out.shape == (B, S, H) and out.dtype == dtype
    logits = mlp.last_router_logits
    loss = (out.reshape(B * S, H).float() * gout.to(DEV).float()).sum() + (logits * glog.to(DEV)).sum()
    loss.backward()
    idx = torch.from_numpy(O.select_topk(logits.detach().cpu(), K))
    ref = _ref_block_fp64(x.reshape(B * S, H), Wr, Wgu, Wdn, idx, True, gout, glog)
    tol = 1e-2 if dtype == torch.bfloat16 else 1e-4
    names = ["out", "logits", "dx", "dWr", "dWgu", "dWdn"]
    got = [out.reshape(B * S, H), logits, xg.grad.reshape(B * S, H), mlp.router.weight.grad,
           mlp.experts.gate_up_proj.grad, mlp.experts.down_proj.grad]
    for n, a, b in zip(names, got, ref):
        check_close(n, a, b, tol, MAX_ABS_FRAC[dtype])
    # the operator alone, on the module's routing
    _, tw, ti = pa.router_topk(xg.detach().reshape(B * S, H), mlp.router.weight.detach(), K)
    h = xg.detach().reshape(B * S, H).clone().requires_grad_(True)
    gu = mlp.experts.gate_up_proj.detach().clone().requires_grad_(True)
    dn = mlp.experts.down_proj.detach().clone().requires_grad_(True)
    y = pa.moe_expert_ffn(h, ti, tw, gu, dn)
    (y.float() * gout.to(DEV).float()).sum().backward()
    hr = x.reshape(B * S, H).double().requires_grad_(True)
    gur, dnr = Wgu.double().requires_grad_(True), Wdn.double().requires_grad_(True)
    yr = O.expert_ffn_loop(hr, ti.cpu(), tw.cpu().double(), gur, dnr)
    (yr * gout.double()).sum().backward()
    for n, a, b in (("ffn out", y, yr), ("ffn dx", h.grad, hr.grad), ("ffn dWgu", gu.grad, gur.grad),
                    ("ffn dWdn", dn.grad, dnr.grad)):
        check_close(n, a, b, tol, MAX_ABS_FRAC[dtype])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_sparse_mlp_largest_expert_count_and_top_k(dtype):
    """E = 1024 and K = 64, the largest the kernels take (include/pmoe.h): the
    router's widest rows, 1024 groups in every grouped GEMM's scan, most of
    them empty or one-row; values and every gradient vs fp64 autograd."""
    pa = _mod()
    B, S, H, E, K, I = 1, 96, 128, 1024, 64, 64
    say(f"sparse MLP E={E} K={K} H={H} I={I} {dtype}")
    g = gen(29)
    x = torch.randn(B, S, H, generator=g).to(dtype)
    Wr = torch.randn(E, H, generator=g) * 0.05
    Wgu = (torch.randn(E, 2 * I, H, generator=g) * 0.05).to(dtype)
    Wdn = (torch.randn(E, H, I, generator=g) * 0.05).to(dtype)
    gout = torch.randn(B * S, H, generator=g).to(dtype)
    glog = torch.randn(B * S, E, generator=g) * 0.01
    mlp = pa.Qwen3MoeSparseMLP(H, I, E, K).to(DEV)
    with torch.no_grad():
        mlp.router.weight.copy_(Wr)
        mlp.experts.gate_up_proj.data = Wgu.to(DEV)
        mlp.experts.down_proj.data = Wdn.to(DEV)
    xg = x.to(DEV).requires_grad_(True)
    out = mlp(xg)
    logits = mlp.last_router_logits
    loss = (out.reshape(B * S, H).float() * gout.to(DEV).float()).sum() + (logits * glog.to(DEV)).sum()
    loss.backward()
    idx = torch.from_numpy(O.select_topk(logits.detach().cpu(), K))
    counts = np.bincount(idx.reshape(-1).numpy(), minlength=E)
    say(f"  experts hit {(counts > 0).sum()} of {E}, max rows {counts.max()}")
    ref = _ref_block_fp64(x.reshape(B * S, H), Wr, Wgu, Wdn, idx, True, gout, glog)
    tol = 1e-2 if dtype == torch.bfloat16 else 1e-4
    names = ["out", "logits", "dx", "dWr", "dWgu", "dWdn"]
    got = [out.reshape(B * S, H), logits, xg.grad.reshape(B * S, H), mlp.router.weight.grad,
           mlp.experts.gate_up_proj.grad, mlp.experts.down_proj.grad]
    for n, a, b in zip(names, got, ref):
        check_close(n, a, b, tol, MAX_ABS_FRAC[dtype])
    for e in np.nonzero(counts == 0)[0][:8]:
        assert torch.count_nonzero(mlp.experts.gate_up_proj.grad[e]) == 0


@pytest.mark.parametrize("E,K", [(4, 4), (1, 1)])
def test_sparse_mlp_every_expert_and_single_expert(E, K):
    """K = E (every token uses every expert) and E = K = 1 (a dense SwiGLU MLP) vs fp64 autograd."""
    pa = _mod()
    B, S, H, I = 1, 200, 256, 64
    say(f"sparse MLP edge E={E} K={K}")
    g = gen(31 + E)
    x = torch.randn(B, S, H, generator=g).to(torch.bfloat16)
    Wr = torch.randn(E, H, generator=g) * 0.05
    Wgu = (torch.randn(E, 2 * I, H, generator=g) * 0.05).to(torch.bfloat16)
    Wdn = (torch.randn(E, H, I, generator=g) * 0.05).to(torch.bfloat16)
    gout = torch.randn(B * S, H, generator=g).to(torch.bfloat16)
    glog = torch.randn(B * S, E, generator=g) * 0.01
    mlp = pa.Qwen3MoeSparseMLP(H, I, E, K, True).to(DEV)
    with torch.no_grad():
        mlp.router.weight.copy_(Wr)
        mlp.experts.gate_up_proj.data = Wgu.to(DEV)
        mlp.experts.down_proj.data = Wdn.to(DEV)
    xg = x.to(DEV).requires_grad_(True)
    out = mlp(xg)
    logits = mlp.last_router_logits
    loss = (out.reshape(B * S, H).float() * gout.to(DEV).float()).sum() + (logits * glog.to(DEV)).sum()
    loss.backward()
    idx = torch.from_numpy(O.select_topk(logits.detach().cpu(), K))
    # every expert is selected, in id order of the logits; all counts equal T
    assert sorted(set(idx.reshape(-1).tolist())) == list(range(E))
    ref = _ref_block_fp64(x.reshape(B * S, H), Wr, Wgu, Wdn, idx, True, gout, glog)
    names = ["out", "logits", "dx", "dWr", "dWgu", "dWdn"]
    got = [out.reshape(B * S, H), logits, xg.grad.reshape(B * S, H), mlp.router.weight.grad,
           mlp.experts.gate_up_proj.grad, mlp.experts.down_proj.grad]
    # (E = 1: the routing weight is the constant 1, so the router's gradient comes from the logits
    # term alone)
    for n, a, b in zip(names, got, ref):
        check_close(n, a, b, 1e-2, MAX_ABS_FRAC[torch.bfloat16])
    counts = mlp.router.last_stats.expert_counts
    assert to_np(counts).tolist() == [B * S] * E


def test_sparse_mlp_empty_batch():
    """No tokens: empty output, zero parameter gradients, zero counts (torch's semantics on empty tensors)."""
    pa = _mod()
    H, E, K, I = 256, 8, 2, 64
    mlp = pa.Qwen3MoeSparseMLP(H, I, E, K, True).to(DEV)
    with torch.no_grad():
        mlp.experts.gate_up_proj.data = (torch.randn(E, 2 * I, H, generator=gen(3)) * 0.05).to(DEV)
        mlp.experts.down_proj.data = (torch.randn(E, H, I, generator=gen(4)) * 0.05).to(DEV)
    x = torch.zeros(1, 0, H, device=DEV, requires_grad=True)
    out = mlp(x)
    assert out.shape == (1, 0, H)
    assert mlp.last_router_logits.shape == (0, E)
    out.sum().backward()
    assert x.grad is not None and x.grad.shape == (1, 0, H)
    for name, prm in mlp.named_parameters():
        assert prm.grad is None or torch.count_nonzero(prm.grad).item() == 0, name
    assert to_np(mlp.router.last_stats.expert_counts).tolist() == [0] * E


@pytest.mark.parametrize("entry", ["module", "expert_ffn"])
def test_fp32_master_weights_under_autocast(entry):
    """The trainer's regime (fp32 parameters, bf16 autocast): the expert weight
    gradients arrive in fp32 straight from the GEMMs, and rounded to bf16 they
    equal, bit for bit, the gradients of bf16 copies of the same weights."""
    pa = _mod()
    T, H, E, K, I = 384, 256, 16, 4, 128
    say(f"fp32 masters under autocast ({entry}) T={T} H={H} E={E} K={K} I={I}")
    g = gen(61)
    x = torch.randn(T, H, generator=g).to(DEV)
    Wr = (torch.randn(E, H, generator=g) * 0.05).to(DEV)
    Wgu = (torch.randn(E, 2 * I, H, generator=g) * 0.05).to(DEV)
    Wdn = (torch.randn(E, H, I, generator=g) * 0.05).to(DEV)
    gout = torch.randn(T, H, generator=g).to(DEV)
    ti, tw = None, None
    if entry == "expert_ffn":
        _, tw, ti = pa.router_topk(x.to(torch.bfloat16), Wr, K)

    def run(gu, dn):
        with torch.autocast("cuda", dtype=torch.bfloat16):
            if entry == "module":
                out = pa.sparse_moe_block(x, Wr, gu, dn, K)[0]
            else:
                out = pa.moe_expert_ffn(x, ti, tw, gu, dn)
        out.backward(gout)
        return out.detach()

    masters = [Wgu.clone().requires_grad_(True), Wdn.clone().requires_grad_(True)]
    out_m = run(*masters)
    copies = [Wgu.to(torch.bfloat16).requires_grad_(True), Wdn.to(torch.bfloat16).requires_grad_(True)]
    out_c = run(*copies)
    assert torch.equal(out_m, out_c)
    for name, m, c in zip(("gate_up", "down"), masters, copies):
        assert m.grad.dtype == torch.float32 and c.grad.dtype == torch.bfloat16, name
        assert torch.equal(m.grad.to(torch.bfloat16), c.grad), name
        assert torch.count_nonzero(m.grad).item() > 0, name


def test_fp32_master_weights_empty_batch():
    """No tokens under autocast with fp32 masters: zero fp32 weight gradients."""
    pa = _mod()
    H, E, K, I = 256, 8, 2, 64
    say(f"fp32 masters, empty batch H={H} E={E} K={K} I={I}")
    mlp = pa.Qwen3MoeSparseMLP(H, I, E, K, True).to(DEV)
    x = torch.zeros(1, 0, H, device=DEV, requires_grad=True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out = mlp(x)
    out.sum().backward()
    for prm in (mlp.experts.gate_up_proj, mlp.experts.down_proj):
        assert prm.grad is None or (prm.grad.dtype == torch.float32 and torch.count_nonzero(prm.grad).item() == 0)


def _check_routing_vs_cpu(x, Wr, gpu_logits, K, bias=None):
    """GPU ids == oracle ids on the GPU logits (bit-exact); vs CPU logits except near-ties."""
    cpu_logits = torch.nn.functional.linear(x.float(), Wr.float())
    if bias is not None:
        cpu_logits = cpu_logits + bias.float()
    r = rel(gpu_logits, cpu_logits)
    assert r < 1e-5, f"logits rel {r}"
    a = O.select_topk(gpu_logits, K)
    b = O.select_topk(cpu_logits, K)
    bad = np.nonzero((np.sort(a, 1) != np.sort(b, 1)).any(1))[0]
    srt = np.sort(cpu_logits.numpy(), 1)[:, ::-1]
    for t in bad:
        gap = srt[t, K - 1] - srt[t, K]
        assert gap <= 1e-5 * max(1.0, abs(srt[t, K - 1])), f"row {t}: routing differs away from a tie"
    return len(bad)


def _run_config(cfg_id, tokens: int | None = None, router_dtype=None):
    """One configuration at full size: routing, counts and permutation bit-exact;
    the router statistics against the oracle; every output row, the whole input
    gradient, every expert's weight gradients and the full router weight gradient
    against fp64 truth (``ref_layer_fp64``) with rel-L2 and max-abs bounds;
    bitwise run-to-run determinism. ``router_dtype``: the router weight in that
    dtype (its rounding is the truth's weight too), else fp32."""
    from pluggy_amd.workloads import CONFIGS, MoEConfig, make_inputs

    pa = _mod()
    cfg = cfg_id if isinstance(cfg_id, MoEConfig) else CONFIGS[cfg_id]
    inp = make_inputs(cfg, tokens=tokens)
    T = inp["x"].shape[0]
    H, E, K, I = cfg.hidden, cfg.experts, cfg.top_k, cfg.inter
    say(f"config {cfg_id if isinstance(cfg_id, int) else '-'} ({cfg.name}) T={T} H={H} E={E} K={K} I={I} {cfg.dtype} backward={cfg.backward}")
    mlp = pa.Qwen3MoeSparseMLP(H, I, E, K, cfg.norm_topk_prob).to(DEV)
    if router_dtype is not None:
        inp["router_weight"] = inp["router_weight"].to(router_dtype)
        mlp.router.to(router_dtype)
    with torch.no_grad():
        mlp.router.weight.copy_(inp["router_weight"])
        mlp.experts.gate_up_proj.data = inp["gate_up_proj"].to(DEV)
        mlp.experts.down_proj.data = inp["down_proj"].to(DEV)
    bias = inp.get("logit_bias")
    if bias is not None:
        mlp.router.logit_bias = bias.to(DEV)

    def step():
        for prm in mlp.parameters():
            prm.grad = None
        xg = inp["x"].to(DEV).reshape(1, T, H).requires_grad_(cfg.backward)
        out = mlp(xg)
        if cfg.backward:
            out.reshape(T, H).backward(inp["grad_out"].to(DEV))
        torch.cuda.synchronize()
        grads = [None if prm.grad is None else prm.grad.clone() for prm in
                 (mlp.router.weight, mlp.experts.gate_up_proj, mlp.experts.down_proj)]
        return out.reshape(T, H), mlp.last_router_logits, xg.grad, mlp.router.last_stats, grads

    out, logits, dx, stats, grads = step()
    lg = logits.detach().cpu()
    idx = O.select_topk(lg, K)
    # 1. routing: bit-exact on the GPU logits; near-tie-only differences on CPU logits
    n_tie = _check_routing_vs_cpu(inp["x"], inp["router_weight"].float(), lg, K, bias)
    say(f"  routing ok (near-tie rows vs CPU logits: {n_tie})")
    counts = to_np(stats.expert_counts)
    assert np.array_equal(counts, np.bincount(idx.reshape(-1), minlength=E))
    say(f"  expert counts min={counts.min()} max={counts.max()} empty={(counts == 0).sum()}")
    # router statistics vs the oracle on the same logits
    _, rps, rl2 = O.router_stats(lg, torch.from_numpy(idx), E)
    assert rel(stats.prob_sum, rps) < 1e-5
    assert abs(stats.lse_sq_sum.item() - rl2.item()) <= 1e-5 * abs(rl2.item()) + 1e-6
    # 2. permutation bit-exact
    from pluggy_amd import ops
    c2, offs, sp, inv = ops.permute(torch.from_numpy(idx).to(DEV), E)
    rc, ro, rsp, rinv = O.permute(idx, E)
    assert np.array_equal(to_np(offs), ro) and np.array_equal(to_np(sp), rsp) and np.array_equal(to_np(inv), rinv)
    # 3. every value against fp64 truth given the GPU's routing
    ref = ref_layer_fp64(inp["x"], inp["router_weight"].float(), inp["gate_up_proj"], inp["down_proj"],
                         torch.from_numpy(idx), lg, cfg.norm_topk_prob,
                         gout=inp["grad_out"] if cfg.backward else None)
    tol = {torch.bfloat16: 1e-2, torch.float16: 2e-3, torch.float32: 1e-4}[cfg.dtype]
    frac = MAX_ABS_FRAC[cfg.dtype]
    check_close("out", out, ref["out"], tol, frac)
    if cfg.backward:
        check_close("dx", dx.reshape(T, H), ref["dx"], tol, frac)
        # (the router weight gradient inherits the bf16 rounding of the expert outputs
        # through d top_weights; the router backward alone is checked at 1e-5 in the stage tests)
        check_close("d router.weight", grads[0], ref["dWr"], tol, frac)
        check_close("d gate_up_proj", grads[1], ref["dWgu"], tol, frac)
        check_close("d down_proj", grads[2], ref["dWdn"], tol, frac)
        for name, gW in (("gate_up", grads[1]), ("down", grads[2])):
            for e in np.nonzero(counts == 0)[0]:
                assert torch.count_nonzero(gW[e]) == 0, f"empty expert {e}: nonzero d {name}"
        # the heaviest and the lightest populated expert on their own (a large
        # tensor-wide rel-L2 could hide one expert's error)
        pop = np.nonzero(counts)[0]
        for e in (pop[np.argmax(counts[pop])], pop[np.argmin(counts[pop])]):
            check_close(f"expert {e} ({counts[e]} rows) d gate_up", grads[1][e], ref["dWgu"][e], tol, frac)
            check_close(f"expert {e} ({counts[e]} rows) d down", grads[2][e], ref["dWdn"][e], tol, frac)
    if cfg.dtype == torch.float32:
        # the reference CPU path itself (loop path) on the whole layer
        p = torch.softmax(lg.double(), -1)
        w = p.gather(1, torch.from_numpy(idx))
        if cfg.norm_topk_prob:
            w = w / w.sum(-1, keepdim=True)
        ref_loop = O.expert_ffn_loop(inp["x"], torch.from_numpy(idx), w.float(), inp["gate_up_proj"],
                                     inp["down_proj"])
        r = rel(out, ref_loop)
        say(f"  out vs oracle loop path rel={r:.2e}")
        assert r < 1e-4
    # 4. bitwise determinism
    out2, logits2, dx2, _, grads2 = step()
    assert torch.equal(out2, out) and torch.equal(logits2, logits)
    if cfg.backward:
        assert torch.equal(dx2, dx) and all(torch.equal(a, b) for a, b in zip(grads, grads2))
    say("  deterministic ok")


def test_config1_small_fp32():
    _run_config(1)


def test_config2_qwen3_30b_a3b():
    _run_config(2)


def test_config4_skewed():
    _run_config(4)


@pytest.mark.parametrize("router_dtype", [torch.float16, torch.float32])
def test_config2_fp16(router_dtype):
    """Config 2's layer with fp16 tensors (activations and expert weights), the
    expert path on the fp16 MFMAs. With an fp16 router weight (a module in
    fp16, the only pairing the reference's F.linear takes for fp16 input) the
    router runs on the fp16 MFMAs too; with an fp32 one, on fp32 copies of x.
    Every value and gradient against fp64 at fp16's bar (rel-L2 2e-3)."""
    import dataclasses

    from pluggy_amd.workloads import CONFIGS

    _run_config(dataclasses.replace(CONFIGS[2], name="qwen3-30b-a3b-fp16", dtype=torch.float16),
                router_dtype=router_dtype)


def test_config_climbmix():
    """pluggy's own MoE training shape (H=1024, E=32, top-4, I=512, T=8192)."""
    from pluggy_amd.workloads import CLIMBMIX

    _run_config(CLIMBMIX)


def test_config5_decode():
    _run_config(5)


def test_config3_qwen3_235b_a22b():
    _run_config(3)


def test_fp32_masters_any_size_under_autocast():
    """Unaligned H and I (zero-padded on the host) with fp32 master weights
    under bf16 autocast: the pad happens in fp32, so the expert weight
    gradients still arrive in fp32 from the GEMMs (autograd slices them back),
    and they match fp64 autograd on the bf16 copies at the bf16 bar."""
    pa = _mod()
    B, S, H, E, K, I = 2, 96, 100, 8, 2, 52
    say(f"fp32 masters, any size, autocast: H={H} I={I} E={E} K={K}")
    g = gen(29)
    x = torch.randn(B, S, H, generator=g)
    Wr = torch.randn(E, H, generator=g) * 0.05
    Wgu = (torch.randn(E, 2 * I, H, generator=g) * 0.05).to(torch.bfloat16).float()
    Wdn = (torch.randn(E, H, I, generator=g) * 0.05).to(torch.bfloat16).float()
    gout = torch.randn(B * S, H, generator=g)
    mlp = pa.Qwen3MoeSparseMLP(H, I, E, K).to(DEV)
    with torch.no_grad():
        mlp.router.weight.copy_(Wr)
        mlp.experts.gate_up_proj.copy_(Wgu)
        mlp.experts.down_proj.copy_(Wdn)
    xg = x.to(DEV).requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out = mlp(xg)
    out.reshape(B * S, H).backward(gout.to(DEV))
    for prm in (mlp.experts.gate_up_proj, mlp.experts.down_proj):
        assert prm.grad.dtype == torch.float32 and prm.grad.shape == prm.shape
    # fp64 truth on the operands the kernels saw: bf16 x and router weight, the masters' (bf16-valued) copies
    idx = torch.from_numpy(O.select_topk(mlp.last_router_logits.detach().cpu(), K))
    ref = _ref_block_fp64(x.reshape(B * S, H).to(torch.bfloat16).float(), Wr.to(torch.bfloat16).float(), Wgu, Wdn,
                          idx, True, gout, torch.zeros(B * S, E))
    frac = MAX_ABS_FRAC[torch.bfloat16]
    check_close("out", out.reshape(B * S, H), ref[0], 1e-2, frac)
    check_close("d gate_up_proj (fp32)", mlp.experts.gate_up_proj.grad, ref[4], 1e-2, frac)
    check_close("d down_proj (fp32)", mlp.experts.down_proj.grad, ref[5], 1e-2, frac)


def test_router_weight_is_split_once_per_step_and_cached():
    """bf16 activations beside an fp32 router weight: the forward splits the
    weight into its bf16 pieces once and its backward reuses them (one split
    per step); inside pluggy_amd.weight_cast_cache the pieces are kept across
    steps until the weight changes in place. Outputs and gradients equal, bit
    for bit, the path where the kernels split the weight inside every call."""
    import pluggy_amd.moe as M

    pa = _mod()
    T, H, E, K, I = 512, 256, 16, 4, 128
    say(f"router pieces T={T} H={H} E={E} K={K} I={I}")
    g = gen(71)
    x = torch.randn(T, H, generator=g).bfloat16().to(DEV)
    gout = torch.randn(T, H, generator=g).bfloat16().to(DEV)
    mlp = pa.Qwen3MoeSparseMLP(H, I, E, K).to(DEV)
    with torch.no_grad():
        for prm in mlp.parameters():
            prm.copy_(torch.randn(prm.shape, generator=g) * 0.05)
    mlp.experts.gate_up_proj.data = mlp.experts.gate_up_proj.data.bfloat16()
    mlp.experts.down_proj.data = mlp.experts.down_proj.data.bfloat16()
    assert mlp.router.weight.dtype == torch.float32

    def step():
        mlp.zero_grad(set_to_none=True)
        xg = x.clone().reshape(1, T, H).requires_grad_(True)
        out = mlp(xg)
        out.reshape(T, H).backward(gout)
        return [out.detach().clone(), xg.grad.clone()] + [p.grad.clone() for p in mlp.parameters()]

    def unsplit_step():
        orig = M._router_pieces
        M._router_pieces = lambda *a, **k: None
        try:
            return step()
        finally:
            M._router_pieces = orig

    real, n = M.ops.split_router_weight, [0]

    def counting(w):
        n[0] += 1
        return real(w)

    plain = unsplit_step()
    M.ops.split_router_weight = counting
    try:
        first = step()
        assert n[0] == 1, "one split per step, reused by the backward"
        with pa.weight_cast_cache():
            a, b = step(), step()
            assert n[0] == 2, "the cached pieces were made again"
            with torch.no_grad():
                mlp.router.weight.mul_(0.5)
            c = step()
            assert n[0] == 3, "the pieces of the changed weight were not remade"
    finally:
        M.ops.split_router_weight = real
    for u, v, w_, z in zip(plain, first, a, b):
        assert torch.equal(u, v) and torch.equal(u, w_) and torch.equal(u, z)
    for u, v in zip(c, unsplit_step()):
        assert torch.equal(u, v)


def test_weight_cast_cache_reuses_copies_until_the_master_changes():
    """Inside pluggy_amd.weight_cast_cache the bf16 copies of fp32 masters are
    made once and reused (outputs and fp32 weight gradients bitwise equal to
    the uncached path); an in-place update of a master (an optimizer step)
    makes a new copy, again bitwise equal to the uncached path on the updated
    weights; leaving the context drops the copies."""
    import pluggy_amd.moe as M

    pa = _mod()
    T, H, E, K, I = 512, 256, 16, 4, 128
    say(f"weight cast cache T={T} H={H} E={E} K={K} I={I}")
    g = gen(67)
    x = torch.randn(T, H, generator=g).to(DEV)
    gout = torch.randn(T, H, generator=g).to(DEV)
    mlp = pa.Qwen3MoeSparseMLP(H, I, E, K).to(DEV)
    with torch.no_grad():
        for prm in mlp.parameters():
            prm.copy_(torch.randn(prm.shape, generator=g) * 0.05)

    def step():
        mlp.zero_grad(set_to_none=True)
        xg = x.clone().reshape(1, T, H).requires_grad_(True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            out = mlp(xg)
        out.reshape(T, H).backward(gout)
        return [out.detach().clone(), xg.grad.clone()] + [p.grad.clone() for p in mlp.parameters()]

    plain = step()
    with pa.weight_cast_cache():
        first = step()
        copies = {k: v[2] for k, v in M._cast_cache.items()}
        assert len(copies) == 2  # the two expert masters
        second = step()
        assert all(M._cast_cache[k][2] is c for k, c in copies.items()), "the copies were made again"
        for a, b, c in zip(plain, first, second):
            assert torch.equal(a, b) and torch.equal(a, c)
        with torch.no_grad():  # an optimizer-style in-place update bumps the version
            mlp.experts.gate_up_proj.mul_(0.5)
        third = step()
        key = (id(mlp.experts.gate_up_proj), torch.bfloat16)  # copies are kept per master and dtype
        assert M._cast_cache[key][2] is not copies[key]
    assert not M._cast_cache
    fresh = step()
    for a, b in zip(third, fresh):
        assert torch.equal(a, b)
