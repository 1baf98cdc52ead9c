"""The block's neighbours fused into the MoE row kernels (RMSNorm, residual add).

Each kernel against fp64 on the CPU, then the whole MoE half of a block,
``x + SparseMLP(RMSNorm(x))`` (qwen3_moe.py:281), through ``moe_sublayer``:
values and every gradient against fp64 autograd (rel-L2 <= 1e-2 for bf16
compute), against the unfused composition, and compiled == eager.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F
from torch import nn

from oracle import moe_oracle as O
from tests._gpu_helpers import DEV, MAX_ABS_FRAC, check_close, gen, max_abs, rel, say
from tests.test_gpu_block import _check_routing_vs_cpu

pytestmark = pytest.mark.gpu
f32, bf16 = torch.float32, torch.bfloat16


def _ops():
    from pluggy_amd import ops
    return ops


def _bf16_ulp(v: torch.Tensor) -> torch.Tensor:
    a = v.abs().clamp_min(2.0 ** -126)
    return torch.exp2(torch.floor(torch.log2(a)) - 7)


@pytest.mark.parametrize("x_dtype,out_dtype,H", [(f32, bf16, 2048), (f32, f32, 2048), (bf16, bf16, 776),
                                                 (f32, bf16, 3000)])
def test_rmsnorm_forward(x_dtype, out_dtype, H):
    T = 300
    say(f"rmsnorm fwd T={T} H={H} x={x_dtype} out={out_dtype}")
    g = gen(51)
    x = (torch.randn(T, H, generator=g) * 3).to(x_dtype)
    w = 1 + 0.1 * torch.randn(H, generator=g)
    eps = torch.finfo(x_dtype).eps
    n, r = _ops().rmsnorm_forward(x.to(DEV), w.to(DEV), eps, out_dtype)
    x64 = x.double()
    r64 = 1.0 / torch.sqrt(x64.pow(2).mean(-1) + eps)
    n64 = x64 * r64[:, None] * w.double()
    assert rel(r, r64) < 1e-6
    if out_dtype == f32:
        assert rel(n, n64) < 1e-6
        if x_dtype == f32:  # torch's own RMSNorm on the same GPU
            assert rel(n, F.rms_norm(x.to(DEV), (H,), w.to(DEV), eps)) < 1e-6
    else:  # one rounding of the fp32 value: within half a bf16 ulp of the exact one (+ fp32 noise)
        err = (n.double().cpu() - n64).abs() / _bf16_ulp(n64)
        say(f"  max error {err.max().item():.3f} bf16 ulp")
        assert err.max().item() <= 0.5 + 1e-3


@pytest.mark.parametrize("K,res_dtype", [(8, f32), (3, f32), (8, bf16)])
def test_combine_residual_and_backward(K, res_dtype):
    T, H = 300, 256
    P = T * K
    say(f"combine_residual T={T} K={K} H={H} res={res_dtype}")
    g = gen(52)
    y = torch.randn(P, H, generator=g).to(bf16)
    w = torch.rand(T, K, generator=g)
    inv_pos = torch.randperm(P, generator=g).to(torch.int32).reshape(T, K)
    res = torch.randn(T, H, generator=g).to(res_dtype)
    gout = torch.randn(T, H, generator=g).to(res_dtype)
    ops = _ops()
    out = ops.combine_residual(y.to(DEV), w.to(DEV), inv_pos.reshape(-1).to(DEV), res.to(DEV))
    assert out.dtype == res_dtype
    yg = y.double()[inv_pos.long()]                                   # (T, K, H)
    ref = res.double() + (w.double()[:, :, None] * yg).sum(1)
    r = rel(out, ref)
    say(f"  out rel={r:.2e} maxabs={max_abs(out, ref):.2e}")
    assert r < (1e-6 if res_dtype == f32 else 4e-3)
    gy, gw = ops.combine_residual_backward(gout.to(DEV), y.to(DEV), w.to(DEV), inv_pos.reshape(-1).to(DEV))
    gy_ref = torch.zeros(P, H, dtype=torch.float64)
    gy_ref[inv_pos.long().reshape(-1)] = (w.double()[:, :, None] * gout.double()[:, None, :]).reshape(P, H)
    gw_ref = (gout.double()[:, None, :] * yg).sum(-1)
    assert rel(gy, gy_ref) < 4e-3 and rel(gw, gw_ref) < 1e-5


def _ref_norm_bwd(gxp, inv_pos, add, x, w, res, eps):
    """fp64 autograd of n = RMSNorm(x) with upstream g = add + K-sum of gxp."""
    x64 = x.double().requires_grad_(True)
    w64 = w.double().requires_grad_(True)
    r = 1.0 / torch.sqrt(x64.pow(2).mean(-1, keepdim=True) + eps)
    n = x64 * r * w64
    gup = torch.zeros_like(n)
    if add is not None:
        gup = gup + add.double()
    if gxp is not None:
        gup = gup + gxp.double()[inv_pos.long()].sum(1)
    (n * gup).sum().backward()
    gx = x64.grad + (res.double() if res is not None else 0.0)
    return gx, w64.grad


@pytest.mark.parametrize("K,H,x_dtype,terms", [(8, 2048, f32, "all"), (3, 776, f32, "all"), (8, 3000, f32, "all"),
                                               (8, 2048, bf16, "all"), (8, 2048, f32, "no_perm"),
                                               (8, 2048, f32, "no_add_res"),
                                               # rows wider than the register kernel's 4096: walked twice
                                               (8, 7168, f32, "all"), (3, 5000, bf16, "all"),
                                               (8, 16384, f32, "no_add_res"), (4, 6144, f32, "no_perm")])
def test_dispatch_rmsnorm_backward(K, H, x_dtype, terms):
    T = 300
    P = T * K
    say(f"dispatch_rmsnorm_bwd T={T} K={K} H={H} x={x_dtype} terms={terms}")
    g = gen(53)
    x = (torch.randn(T, H, generator=g) * 2).to(x_dtype)
    w = 1 + 0.1 * torch.randn(H, generator=g)
    gxp = torch.randn(P, H, generator=g).to(bf16)
    inv_pos = torch.randperm(P, generator=g).to(torch.int32).reshape(T, K)
    add = torch.randn(T, H, generator=g).to(bf16)
    res = torch.randn(T, H, generator=g).to(x_dtype)
    if terms == "no_perm":
        gxp = None
    if terms == "no_add_res":
        add = res = None
    eps = torch.finfo(x_dtype).eps
    ops = _ops()
    xd, wd = x.to(DEV), w.to(DEV)
    _, rstd = ops.rmsnorm_forward(xd, wd, eps, bf16)
    dev = lambda t: None if t is None else t.to(DEV)  # noqa: E731
    gx, gw = ops.dispatch_rmsnorm_backward(dev(gxp), inv_pos.reshape(-1).to(DEV), dev(add), xd, wd, rstd, dev(res), K)
    gx_ref, gw_ref = _ref_norm_bwd(gxp, inv_pos, add, x, w, res, eps)
    tol = 1e-5 if x_dtype == f32 else 4e-3
    say(f"  gx rel={rel(gx, gx_ref):.2e} gw rel={rel(gw, gw_ref):.2e}")
    assert gx.dtype == x_dtype and rel(gx, gx_ref) < tol and rel(gw, gw_ref) < 1e-5
    gx2, gw2 = ops.dispatch_rmsnorm_backward(dev(gxp), inv_pos.reshape(-1).to(DEV), dev(add), xd, wd, rstd, dev(res),
                                             K, need_weight=False)
    assert gw2 is None and torch.equal(gx2, gx)


def _ref_sublayer_fp64(x, nw, eps, Wr, Wgu, Wdn, idx, gout, glog, n_kernel):
    """fp64 autograd of x + SparseMLP(RMSNorm(x)) given the routing ids; the MLP
    sees the kernel's bf16 normed rows ``n_kernel`` (values), and gradients pass
    that rounding unchanged."""
    x = x.double().requires_grad_(True)
    nw = nw.double().requires_grad_(True)
    Wr, Wgu, Wdn = (t.double().requires_grad_(True) for t in (Wr, Wgu, Wdn))
    n = x * (1.0 / torch.sqrt(x.pow(2).mean(-1, keepdim=True) + eps)) * nw
    n = n + (n_kernel.double() - n).detach()
    logits = n @ Wr.t()
    p = torch.softmax(logits, -1)
    w = p.gather(1, idx)
    w = w / w.sum(-1, keepdim=True)
    I = Wgu.shape[1] // 2
    out = x.clone()
    for e in torch.unique(idx).tolist():
        r, k = torch.nonzero(idx == e, as_tuple=True)
        gu = n[r] @ Wgu[e].t()
        y = (F.silu(gu[:, :I]) * gu[:, I:]) @ Wdn[e].t()
        out = out.index_add(0, r, w[r, k].unsqueeze(1) * y)
    ((out * gout.double()).sum() + (logits * glog.double()).sum()).backward()
    return [out.detach(), logits.detach(), x.grad, nw.grad, Wr.grad, Wgu.grad, Wdn.grad], n.detach()


@pytest.mark.parametrize("x_dtype,autocast", [(f32, True), (bf16, False)])
def test_moe_sublayer_vs_fp64_and_unfused(x_dtype, autocast):
    import pluggy_amd as pa
    B, S, H, E, K, I = 2, 128, 256, 16, 4, 128
    say(f"moe_sublayer B={B} S={S} H={H} E={E} K={K} I={I} x={x_dtype} autocast={autocast}")
    g = gen(54)
    x = (torch.randn(B, S, H, generator=g) * 2).to(x_dtype)
    nw = 1 + 0.1 * torch.randn(H, generator=g)
    Wr = torch.randn(E, H, generator=g) * 0.05
    Wgu = (torch.randn(E, 2 * I, H, generator=g) * 0.05).to(bf16)
    Wdn = (torch.randn(E, H, I, generator=g) * 0.05).to(bf16)
    gout = torch.randn(B * S, H, generator=g).to(x_dtype)
    glog = torch.randn(B * S, E, generator=g) * 0.01

    norm = nn.RMSNorm(H).to(DEV)
    mlp = pa.Qwen3MoeSparseMLP(H, I, E, K).to(DEV)
    with torch.no_grad():
        norm.weight.copy_(nw)
        mlp.router.weight.copy_(Wr)
        mlp.experts.gate_up_proj.copy_(Wgu.float())
        mlp.experts.down_proj.copy_(Wdn.float())
    if not autocast:  # a bf16 model: bf16 expert weights, fp32 router and norm weights
        mlp.experts.gate_up_proj.data = Wgu.to(DEV)
        mlp.experts.down_proj.data = Wdn.to(DEV)

    def run(fused):
        for p in list(norm.parameters()) + list(mlp.parameters()):
            p.grad = None
        xg = x.to(DEV).requires_grad_(True)
        with torch.autocast("cuda", dtype=bf16, enabled=autocast):
            out = pa.moe_sublayer(xg, norm, mlp) if fused else xg + mlp(norm(xg))
            logits = mlp.last_router_logits
            loss = (out.reshape(B * S, H).float() * gout.to(DEV).float()).sum() + (logits * glog.to(DEV)).sum()
        loss.backward()
        assert out.dtype == x_dtype
        return [out.reshape(B * S, H), logits, xg.grad.reshape(B * S, H), norm.weight.grad, mlp.router.weight.grad,
                mlp.experts.gate_up_proj.grad, mlp.experts.down_proj.grad]

    got = [t.detach().clone() for t in run(True)]
    eps = torch.finfo(x_dtype).eps
    idx = torch.from_numpy(O.select_topk(got[1].cpu(), K))
    # the normed rows the kernels saw (same kernel, same bits)
    n_kernel, _ = _ops().rmsnorm_forward(x.reshape(B * S, H).to(DEV), nw.to(DEV), eps, bf16)
    n_kernel = n_kernel.cpu()
    ref, _ = _ref_sublayer_fp64(x.reshape(B * S, H), nw, eps, Wr, Wgu.float(), Wdn.float(), idx, gout, glog, n_kernel)
    _check_routing_vs_cpu(n_kernel, Wr.to(bf16) if autocast else Wr, got[1].cpu(), K)
    names = ["out", "logits", "dx", "dnorm_w", "dWr", "dWgu", "dWdn"]
    for n, a, b in zip(names, got, ref):
        check_close(n, a, b, 1e-2, MAX_ABS_FRAC[torch.bfloat16])
    unfused = run(False)
    for n, a, b in zip(names, got, unfused):
        r = rel(a, b)
        say(f"  vs unfused {n}: rel={r:.2e}")
        assert r < 1e-2, n


def test_moe_sublayer_wide_hidden():
    """The fused half-block beyond H = 4096 (the RMSNorm backward walks each
    row twice): H = 5120 under bf16 autocast with an fp32 stream, values and
    every gradient against fp64 autograd and against the unfused composition."""
    import pluggy_amd as pa
    B, S, H, E, K, I = 1, 96, 5120, 8, 2, 64
    say(f"moe_sublayer wide hidden B={B} S={S} H={H} E={E} K={K} I={I}")
    g = gen(58)
    x = torch.randn(B, S, H, generator=g) * 2
    nw = 1 + 0.1 * torch.randn(H, generator=g)
    Wr = torch.randn(E, H, generator=g) * 0.02
    Wgu = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(bf16)
    Wdn = (torch.randn(E, H, I, generator=g) * 0.05).to(bf16)
    gout = torch.randn(B * S, H, generator=g)
    glog = torch.randn(B * S, E, generator=g) * 0.01
    norm = nn.RMSNorm(H).to(DEV)
    mlp = pa.Qwen3MoeSparseMLP(H, I, E, K).to(DEV)
    with torch.no_grad():
        norm.weight.copy_(nw)
        mlp.router.weight.copy_(Wr)
        mlp.experts.gate_up_proj.copy_(Wgu.float())
        mlp.experts.down_proj.copy_(Wdn.float())

    def run(fused):
        for p in list(norm.parameters()) + list(mlp.parameters()):
            p.grad = None
        xg = x.to(DEV).requires_grad_(True)
        with torch.autocast("cuda", dtype=bf16):
            out = pa.moe_sublayer(xg, norm, mlp) if fused else xg + mlp(norm(xg))
            logits = mlp.last_router_logits
            loss = (out.reshape(B * S, H).float() * gout.to(DEV)).sum() + (logits * glog.to(DEV)).sum()
        loss.backward()
        return [out.reshape(B * S, H), logits, xg.grad.reshape(B * S, H), norm.weight.grad, mlp.router.weight.grad,
                mlp.experts.gate_up_proj.grad, mlp.experts.down_proj.grad]

    got = [t.detach().clone() for t in run(True)]
    eps = torch.finfo(f32).eps
    idx = torch.from_numpy(O.select_topk(got[1].cpu(), K))
    n_kernel, _ = _ops().rmsnorm_forward(x.reshape(B * S, H).to(DEV), nw.to(DEV), eps, bf16)
    ref, _ = _ref_sublayer_fp64(x.reshape(B * S, H), nw, eps, Wr.to(bf16).float(), Wgu.float(), Wdn.float(), idx,
                                gout, glog, n_kernel.cpu())
    names = ["out", "logits", "dx", "dnorm_w", "dWr", "dWgu", "dWdn"]
    for n, a, b in zip(names, got, ref):
        check_close(n, a, b, 1e-2, MAX_ABS_FRAC[bf16])
    for n, a, b in zip(names, got, run(False)):
        r = rel(a, b)
        say(f"  vs unfused {n}: rel={r:.2e}")
        assert r < 1e-2, n


class _FusedHalfBlock(nn.Module):
    def __init__(self, H, I, E, K):
        super().__init__()
        import pluggy_amd as pa
        self.norm2 = nn.RMSNorm(H)
        self.ffn = pa.Qwen3MoeSparseMLP(H, I, E, K)

    def forward(self, x):
        import pluggy_amd as pa
        return pa.moe_sublayer(x, self.norm2, self.ffn)


@pytest.mark.timeout(600)  # inductor compiles its kernels on first use
@pytest.mark.parametrize("backend", ["aot_eager", "inductor"])
def test_moe_sublayer_compiled_matches_eager(backend):
    """aot_eager runs the eager kernels: bitwise equal. Inductor (the trainer's
    ``block.compile(mode="default")``, trainer.py:291-293) generates the loss
    terms around the fused custom op: the dtype's bar, and bitwise reproducible."""
    B, S, H, E, K, I = 2, 64, 256, 16, 4, 128
    say(f"moe_sublayer compiled[{backend}] B={B} S={S} H={H} E={E} K={K} I={I} (autocast bf16, fp32 stream)")
    torch.manual_seed(0)
    blk = _FusedHalfBlock(H, I, E, K).to(DEV)
    g = gen(55)
    with torch.no_grad():
        for p in blk.parameters():
            p.copy_(torch.randn(p.shape, generator=g) * 0.05 + (1.0 if p.dim() == 1 else 0.0))
    x0 = torch.randn(B, S, H, generator=g).to(DEV)

    def run(mod):
        for p in blk.parameters():
            p.grad = None
        x = x0.clone().requires_grad_(True)
        with torch.autocast("cuda", dtype=bf16):
            y = mod(x)
            z = torch.logsumexp(blk.ffn.last_router_logits, -1).pow(2).mean()
        (y.pow(2).mean() + 1e-3 * z).backward()
        return [y.detach(), z.detach(), x.grad] + [p.grad.clone() for p in blk.parameters()]

    eager = run(blk)
    torch._dynamo.reset()
    if backend == "inductor":
        compiled = torch.compile(blk, mode="default", fullgraph=True)
    else:
        compiled = torch.compile(blk, backend="aot_eager", fullgraph=True)
    got = run(compiled)
    got2 = run(compiled)
    for i, (a, b, c) in enumerate(zip(eager, got, got2)):
        if backend == "aot_eager":
            assert torch.equal(a, b), i
        else:
            check_close(f"record {i} (inductor vs eager)", b, a, 1e-2, MAX_ABS_FRAC[bf16])
        assert torch.equal(b, c), i


@pytest.mark.timeout(600)
def test_moe_sublayer_trainer_regime_config2():
    """The trainer's form of the MoE half-block at the Qwen3-30B-A3B shape
    (config 2: T = 8192, H = 2048, E = 128, K = 8, I = 768): ``moe_sublayer``
    under bf16 autocast with an fp32 residual stream, an fp32 norm weight and
    fp32 master weights (trainer.py:466-472, qwen3_moe.py:281). Every value and
    gradient against fp64 truth given the kernels' routing and normed rows
    (``ref_layer_fp64`` on the GPU, plus the RMSNorm and the logits' own
    gradient in fp64): out, the input gradient, the norm-weight gradient, the
    router weight gradient and both fp32 expert weight gradients, with the
    rel-L2 <= 1e-2 and max-abs bounds of the full-size configuration tests."""
    import pluggy_amd as pa
    from pluggy_amd.workloads import CONFIGS, make_inputs
    from tests._gpu_helpers import ref_layer_fp64

    cfg = CONFIGS[2]
    inp = make_inputs(cfg)
    T, H, E, K, I = inp["x"].shape[0], cfg.hidden, cfg.experts, cfg.top_k, cfg.inter
    say(f"moe_sublayer trainer regime at config 2: T={T} H={H} E={E} K={K} I={I}, fp32 stream + masters, autocast bf16")
    g = gen(57)
    x = inp["x"].float()                      # the fp32 residual stream
    nw = 1 + 0.1 * torch.randn(H, generator=g)
    gout = inp["grad_out"].float()
    glog = torch.randn(T, E, generator=g) * 0.01
    eps = torch.finfo(f32).eps
    norm = nn.RMSNorm(H, eps=eps).to(DEV)
    mlp = pa.Qwen3MoeSparseMLP(H, I, E, K).to(DEV)
    with torch.no_grad():
        norm.weight.copy_(nw)
        mlp.router.weight.copy_(inp["router_weight"])
        mlp.experts.gate_up_proj.copy_(inp["gate_up_proj"].float())  # fp32 masters holding bf16 values
        mlp.experts.down_proj.copy_(inp["down_proj"].float())
    xg = x.to(DEV).reshape(1, T, H).requires_grad_(True)
    with torch.autocast("cuda", dtype=bf16):
        out = pa.moe_sublayer(xg, norm, mlp)
        logits = mlp.last_router_logits
        loss = (out.reshape(T, H).float() * gout.to(DEV)).sum() + (logits * glog.to(DEV)).sum()
    loss.backward()
    torch.cuda.synchronize()
    assert out.dtype == f32 and xg.grad.dtype == f32
    assert mlp.experts.gate_up_proj.grad.dtype == f32 and mlp.experts.down_proj.grad.dtype == f32
    lg = logits.detach().float().cpu()
    idx = torch.from_numpy(O.select_topk(lg, K))
    # the normed rows the kernels saw (the same kernel gives the same bits)
    n_kernel, _ = _ops().rmsnorm_forward(x.to(DEV), nw.to(DEV), eps, bf16)
    nr = _check_routing_vs_cpu(n_kernel.cpu(), inp["router_weight"].to(bf16), lg, K)
    say(f"  routing ok (near-tie rows vs CPU logits: {nr})")
    # under autocast the router runs on the bf16 copy of its fp32 weight (the
    # master's gradient is the copy's)
    wr_b = inp["router_weight"].to(bf16).float()
    ref = ref_layer_fp64(n_kernel, wr_b, inp["gate_up_proj"], inp["down_proj"], idx, lg, True, gout=gout)
    # the logits' own gradient (the aux-loss path): d n += glog W_r, d W_r += glog^T n
    Wr = wr_b.to(DEV).double()
    n64 = n_kernel.double()
    gl = glog.to(DEV).double()
    dn = ref["dx"] + gl @ Wr
    dWr = ref["dWr"] + gl.t() @ n64
    # RMSNorm backward and the residual term in fp64 autograd (forward values
    # replaced by the kernel's rounded rows, gradients through the exact norm)
    x64 = x.to(DEV).double().requires_grad_(True)
    w64 = nw.to(DEV).double().requires_grad_(True)
    n_exact = x64 * torch.rsqrt(x64.pow(2).mean(-1, keepdim=True) + eps) * w64
    gx, gw = torch.autograd.grad(n_exact, (x64, w64), grad_outputs=dn)
    gx = gx + gout.to(DEV).double()
    out_ref = x.to(DEV).double() + ref["out"]
    frac = MAX_ABS_FRAC[bf16]
    check_close("out", out.reshape(T, H), out_ref, 1e-2, frac)
    check_close("dx", xg.grad.reshape(T, H), gx, 1e-2, frac)
    check_close("d norm.weight", norm.weight.grad, gw, 1e-2, frac)
    check_close("d router.weight", mlp.router.weight.grad, dWr, 1e-2, frac)
    check_close("d gate_up_proj (fp32 master)", mlp.experts.gate_up_proj.grad, ref["dWgu"], 1e-2, frac)
    check_close("d down_proj (fp32 master)", mlp.experts.down_proj.grad, ref["dWdn"], 1e-2, frac)
