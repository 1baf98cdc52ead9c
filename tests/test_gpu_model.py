"""The drop-in inside a model trained the way the reference trainer trains it.

The trainer keeps fp32 parameters, runs the forward under
``torch.autocast(cuda, bf16)`` (pluggy/training/trainer.py:469), compiles every
transformer block (:292-293) and adds the MoE aux losses to the LM loss
(pluggy/objectives/autoregressive.py:49-57, qwen3_moe.py:428-444).

* Under autocast the sparse MLP takes bf16 operands and returns the residual
  stream's dtype: its values and every gradient match fp64 autograd of the
  block on the bf16-rounded operands (rel-L2 <= 1e-2), routing bit-exact but
  for genuine near-ties.
* A two-block model (RMSNorm -> dense mixer -> residual, RMSNorm -> drop-in
  sparse MLP -> residual, LM head, cross entropy + load-balance + z aux loss)
  with every block compiled ``fullgraph=True`` under autocast gives the eager
  loss, gradients and AdamW update over two steps (rel-L2 <= 1e-5).

The dense mixer stands in for attention, which is not part of this build.
"""

from __future__ import annotations

import copy

import pytest
import torch
import torch.nn.functional as F
from torch import nn

from oracle import moe_oracle as O
from tests._gpu_helpers import DEV, MAX_ABS_FRAC, check_close, gen, max_abs, rel, say
from tests.test_gpu_block import _check_routing_vs_cpu, _ref_block_fp64

pytestmark = pytest.mark.gpu


def _pa():
    import pluggy_amd
    return pluggy_amd


@pytest.mark.parametrize("x_dtype", [torch.float32, torch.bfloat16])
def test_autocast_sparse_mlp(x_dtype):
    pa = _pa()
    B, S, H, E, K, I = 2, 128, 256, 16, 4, 128
    say(f"autocast sparse MLP B={B} S={S} H={H} E={E} K={K} I={I} x={x_dtype}")
    g = gen(31)
    x = torch.randn(B, S, H, generator=g).to(x_dtype)
    Wr = torch.randn(E, H, generator=g) * 0.05
    Wgu = torch.randn(E, 2 * I, H, generator=g) * 0.05
    Wdn = torch.randn(E, H, I, generator=g) * 0.05
    gout = torch.randn(B * S, H, generator=g)
    glog = torch.randn(B * S, E, generator=g) * 0.01

    mlp = pa.Qwen3MoeSparseMLP(H, I, E, K).to(DEV)  # fp32 master parameters
    with torch.no_grad():
        mlp.router.weight.copy_(Wr)
        mlp.experts.gate_up_proj.copy_(Wgu)
        mlp.experts.down_proj.copy_(Wdn)
    xg = x.to(DEV).requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out = mlp(xg)
        logits = mlp.last_router_logits
        loss = (out.reshape(B * S, H).float() * gout.to(DEV)).sum() + (logits * glog.to(DEV)).sum()
    assert out.dtype == x_dtype and logits.dtype == torch.float32
    loss.backward()
    assert xg.grad.dtype == x_dtype
    assert all(p.grad.dtype == torch.float32 for p in mlp.parameters())

    # the kernels saw bf16 operands: fp64 truth on exactly those values
    bf = lambda t: t.to(torch.bfloat16).double()  # noqa: E731
    xr = bf(x.reshape(B * S, H))
    _check_routing_vs_cpu(xr, bf(Wr), logits.detach().cpu(), K)
    idx = torch.from_numpy(O.select_topk(logits.detach().cpu(), K))
    ref = _ref_block_fp64(xr, bf(Wr), bf(Wgu), bf(Wdn), idx, True, gout, glog)
    names = ["out", "logits", "dx", "dWr", "dWgu", "dWdn"]
    got = [out.reshape(B * S, H), logits, xg.grad.reshape(B * S, H), mlp.router.weight.grad,
           mlp.experts.gate_up_proj.grad, mlp.experts.down_proj.grad]
    for n, a, b in zip(names, got, ref):
        check_close(n, a, b, 1e-2, MAX_ABS_FRAC[torch.bfloat16])

    # the operator entry points follow the same rule
    with torch.autocast("cuda", dtype=torch.bfloat16):
        lg, tw, ti = pa.router_topk(xg.detach().reshape(B * S, H), mlp.router.weight, K)
        y = pa.moe_expert_ffn(xg.detach().reshape(B * S, H), ti, tw, mlp.experts.gate_up_proj,
                              mlp.experts.down_proj)
    assert tw.dtype == x_dtype and y.dtype == x_dtype
    assert torch.equal(lg, logits.detach())
    check_close("moe_expert_ffn out", y, ref[0], 1e-2, MAX_ABS_FRAC[torch.bfloat16])


def test_fp16_autocast_takes_fp16_operands():
    """Under fp16 autocast the expert path takes fp16 operands (fp16 MFMAs,
    fp32 masters' copies) and so does the router (the fp16-rounded input and
    weight): the module over fp32 parameters gives, bit for bit, what the same
    module in fp16 gives on the fp16-rounded input (values cast to fp32, and
    the fp32 masters' gradients rounded to fp16 equal the fp16 module's)."""
    pa = _pa()
    mlp = pa.Qwen3MoeSparseMLP(64, 32, 8, 2).to(DEV)
    g = gen(51)
    with torch.no_grad():
        for prm in mlp.parameters():
            prm.copy_(torch.randn(prm.shape, generator=g) * 0.05)
    x0 = torch.randn(1, 40, 64, generator=g).to(DEV)
    half = copy.deepcopy(mlp).half()

    def run(m, x_in, autocast):
        x = x_in.clone().requires_grad_(True)
        for prm in m.parameters():
            prm.grad = None
        with torch.autocast("cuda", dtype=torch.float16, enabled=autocast):
            y = m(x)
            lg = m.last_router_logits
        (y.float().pow(2).sum() + lg.sum()).backward()
        return [y.detach(), lg.detach(), x.grad] + [prm.grad.clone() for prm in m.parameters()]

    amp, ref = run(mlp, x0, True), run(half, x0.half(), False)
    assert amp[0].dtype == torch.float32 and ref[0].dtype == torch.float16
    assert all(p_.dtype == torch.float32 for p_ in amp[3:]), "fp32 masters keep fp32 gradients"
    names = ["y", "logits", "dx"] + [n for n, _ in mlp.named_parameters()]
    for n, a, b in zip(names, amp, ref):
        assert torch.equal(a.to(b.dtype), b), n


def test_fp16_tensors_run_fp16_gemms():
    """fp16 activations, weights and routing weights, as the reference runs
    them (F.grouped_mm in fp16, moe.py:110-119): the result is fp16 from the
    fp16 MFMA path. The forward equals an fp64 evaluation that rounds to fp16
    where the kernels store (gate/up pre-activations, the weighted SwiGLU rows,
    the down rows, the combined output) within rel-L2 5e-5, which skipping
    those roundings (fp32 arithmetic: about 2e-4) or rounding to bf16 (about
    1e-3) would not meet; values and gradients are within fp16's rounding of
    fp64 on the fp16 inputs (rel-L2 2e-3)."""
    pa = _pa()
    T, H, E, K, I = 96, 64, 8, 2, 32
    g = gen(53)
    x = torch.randn(T, H, generator=g).half()
    Wgu = (torch.randn(E, 2 * I, H, generator=g) * 0.05).half()
    Wdn = (torch.randn(E, H, I, generator=g) * 0.05).half()
    lg = torch.randn(T, E, generator=g)
    tw, ti = torch.softmax(lg, -1).topk(K, dim=-1)
    tw = (tw / tw.sum(-1, keepdim=True)).half()
    gout = torch.randn(T, H, generator=g)
    h = x.to(DEV).requires_grad_(True)
    gu, dn = Wgu.to(DEV).requires_grad_(True), Wdn.to(DEV).requires_grad_(True)
    y = pa.moe_expert_ffn(h, ti.to(DEV), tw.to(DEV), gu, dn)
    assert y.dtype == torch.float16
    (y.float() * gout.to(DEV)).sum().backward()
    # fp64 with the kernels' fp16 stores, in their order (the routing weight scales the SwiGLU row)
    r16 = lambda t: t.half().double()  # noqa: E731
    x64, w64 = x.double(), tw.double()
    pre = r16(torch.einsum("tkjh,th->tkj", Wgu.double()[ti], x64))           # (T, K, 2I)
    gate, up = pre[..., :I], pre[..., I:]
    mid = r16(w64.unsqueeze(-1) * gate * torch.sigmoid(gate) * up)
    rows = r16(torch.einsum("tkhi,tki->tkh", Wdn.double()[ti], mid))
    emu = r16(rows.sum(1))
    check_close("out vs fp16-rounding emulation", y, emu, 5e-5, 2e-3)
    hr = x.double().requires_grad_(True)
    gur, dnr = Wgu.double().requires_grad_(True), Wdn.double().requires_grad_(True)
    yr = O.expert_ffn_loop(hr, ti, tw.double(), gur, dnr)
    (yr * gout.double()).sum().backward()
    for n, a, b in (("out", y, yr), ("dx", h.grad, hr.grad), ("dWgu", gu.grad, gur.grad), ("dWdn", dn.grad, dnr.grad)):
        assert a.dtype == torch.float16, n
        check_close(n, a, b, 2e-3, 3e-3)


class _Block(nn.Module):
    """Qwen3MoeTransformerBlock.forward (qwen3_moe.py:275-282) with a dense mixer for attention."""

    def __init__(self, H, I, E, K):
        super().__init__()
        self.norm1 = nn.RMSNorm(H)
        self.mix = nn.Linear(H, H, bias=False)
        self.norm2 = nn.RMSNorm(H)
        self.ffn = _pa().Qwen3MoeSparseMLP(H, I, E, K)

    def forward(self, x):
        x = x + self.mix(self.norm1(x))
        return x + self.ffn(self.norm2(x))


class _TinyMoeLM(nn.Module):
    def __init__(self, V=256, H=256, I=128, E=16, K=4, L=2):
        super().__init__()
        self.E, self.K = E, K
        self.embed = nn.Embedding(V, H)
        self.blocks = nn.ModuleList(_Block(H, I, E, K) for _ in range(L))
        self.norm = nn.RMSNorm(H)
        self.lm_head = nn.Linear(H, V, bias=False)
        g = gen(41)
        with torch.no_grad():
            for name, p in self.named_parameters():
                if "norm" not in name:
                    p.copy_(torch.randn(p.shape, generator=g) * (1.0 if "embed" in name else 0.05))

    def forward(self, tokens):
        x = self.embed(tokens)
        for b in self.blocks:
            x = b(x)
        return self.lm_head(self.norm(x))

    def aux_loss(self):
        """Qwen3Moe.aux_loss (qwen3_moe.py:428-444) with coefficients 1e-2 and 1e-3."""
        logits = [b.ffn.last_router_logits for b in self.blocks]
        stable_topk = lambda lg, k: torch.sort(lg, dim=-1, descending=True, stable=True)[1][:, :k]  # noqa: E731
        return 1e-2 * O.load_balancing_loss(logits, self.E, self.K, select=stable_topk) + 1e-3 * O.router_z_loss(logits)


def _compile(mod, backend):
    if backend == "inductor":  # the trainer's block.compile(mode="default") (trainer.py:291-293)
        return torch.compile(mod, mode="default", fullgraph=True)
    return torch.compile(mod, backend="aot_eager", fullgraph=True)


def _train_steps(model, backend, steps=2):
    torch.manual_seed(7)
    opt = torch.optim.AdamW(model.parameters(), lr=1e-3)
    blocks = model.blocks
    if backend:
        model.blocks = nn.ModuleList(_compile(b, backend) for b in blocks)
    g = gen(43)
    record = []
    for _ in range(steps):
        tokens = torch.randint(0, 256, (2, 65), generator=g).to(DEV)
        opt.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            logits = model(tokens[:, :-1])
            loss = F.cross_entropy(logits.float().reshape(-1, logits.shape[-1]), tokens[:, 1:].reshape(-1))
            loss = loss + model.aux_loss()
        loss.backward()
        record.append(loss.detach().clone())
        record.extend(p.grad.clone() for p in model.parameters())
        opt.step()
    record.extend(p.detach().clone() for p in model.parameters())
    model.blocks = blocks
    return record


@pytest.mark.timeout(600)  # inductor compiles its kernels on first use
@pytest.mark.parametrize("backend", ["aot_eager", "inductor"])
def test_compiled_model_train_steps_match_eager(backend):
    say(f"tiny MoE LM: 2 blocks, autocast bf16, per-block compile [{backend}], AdamW, 2 steps")
    base = _TinyMoeLM().to(DEV)
    eager = _train_steps(copy.deepcopy(base), None)
    torch._dynamo.reset()
    compiled = _train_steps(copy.deepcopy(base), backend)
    say(f"  loss eager {eager[0].item():.6f} compiled {compiled[0].item():.6f}")
    assert torch.isfinite(eager[0])
    # The MoE kernels are deterministic; the dense GEMMs around them are the
    # library's, whose reduction order is not promised, so the aot_eager bar is
    # 1e-5 (a block traced without autocast would be off by ~1e-3). Inductor
    # fuses the RMSNorms, residual adds and casts into generated kernels with
    # their own fp32 reduction order, which moves a bf16 rounding now and then:
    # 2e-3 (the routing itself must not change).
    tol = 1e-5 if backend == "aot_eager" else 2e-3
    same, worst = 0, 0.0
    for i, (a, b) in enumerate(zip(eager, compiled)):
        same += int(torch.equal(a, b))
        worst = max(worst, rel(b, a))
        assert rel(b, a) <= tol, f"record {i}: rel {rel(b, a):.3e}"
    say(f"  {same}/{len(eager)} records bitwise equal, worst rel {worst:.2e}")
    # every parameter moved, the routers included (the aux loss reaches them through the logits)
    moved = [not torch.equal(p, q) for p, q in zip(base.parameters(), compiled[-len(list(base.parameters())):])]
    assert all(moved)


class _ClimbmixStandIn(nn.Module):
    """Qwen3Moe (qwen3_moe.py:319-489) at the shape of configs/qwen3_moe_climbmix.json:4-19:
    emb_dim 1024, 32 experts, top-4, moe_ffn_dim 512, norm_topk_prob, aux and z coefficients
    1e-3, zero-initialised routers (:165-166). Two of its twelve layers; a dense mixer
    stands in for attention and a 512-token vocabulary for Qwen3's, neither of which is
    part of this build. The forward harvests the router logits and updates the expert
    counts after the stack as the reference's does (:446-489)."""

    def __init__(self, V=512, H=1024, I=512, E=32, K=4, L=2):
        super().__init__()
        self.num_experts, self.top_k = E, K
        self.router_aux_loss_coef, self.router_z_loss_coef = 1e-3, 1e-3
        self.token_emb = nn.Embedding(V, H)
        self.blocks = nn.ModuleList(_Block(H, I, E, K) for _ in range(L))
        self.norm = nn.RMSNorm(H)
        self.lm_head = nn.Linear(H, V, bias=False)
        g = gen(61)
        with torch.no_grad():
            for name, p in self.named_parameters():
                if "norm" in name:
                    continue
                if "router" in name:
                    p.zero_()
                else:
                    p.copy_(torch.randn(p.shape, generator=g) * 0.02)
        self._router_logits = []

    def forward(self, tokens):
        for b in self.blocks:
            b.ffn.last_router_logits = None
        x = self.token_emb(tokens)
        for b in self.blocks:
            x = b(x)
        self._router_logits = [b.ffn.last_router_logits for b in self.blocks]
        self._update_expert_counts(self._router_logits)
        return self.lm_head(self.norm(x))

    def _update_expert_counts(self, router_logits):  # replaced by install_stats_aux
        raise AssertionError("install_stats_aux was not applied")


def _climbmix_steps(model, backend, steps=2):
    """The trainer's step (trainer.py:440-500) at the climbmix optimizer settings
    (configs/qwen3_moe_climbmix.json:24-33): fp32 parameters, bf16 autocast, CE +
    aux loss, clip to norm 1.0, fused AdamW(3e-4, betas (0.9, 0.95), wd 0.1)."""
    pa = _pa()
    pa.install_stats_aux(model)
    if backend:
        model.blocks = nn.ModuleList(_compile(b, backend) for b in model.blocks)
        model.norm = _compile(model.norm, backend)
    opt = torch.optim.AdamW(model.parameters(), lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1, fused=True)
    g = gen(67)
    out = []
    for step in range(steps):
        tokens = torch.randint(0, 512, (2, 4097), generator=g).to(DEV)  # micro batch 2 x seq 4096
        opt.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            logits = model(tokens[:, :-1])
            ce = F.cross_entropy(logits.float().reshape(-1, logits.shape[-1]), tokens[:, 1:].reshape(-1))
            aux = model.aux_loss()
        (ce + aux).backward()
        rec = {"ce": ce.detach().clone(), "aux": aux.detach().clone(),
               "counts": model.last_tokens_per_expert.clone(),
               "grads": [p.grad.clone() for p in model.parameters()]}
        torch.nn.utils.clip_grad_norm_(model.parameters(), 1.0)
        opt.step()
        out.append(rec)
        say(f"  [{backend or 'eager'}] step {step}: ce {rec['ce'].item():.5f} aux {rec['aux'].item():.6f}")
    return out


@pytest.mark.timeout(600)  # inductor compiles its kernels on first use
def test_climbmix_shape_compiled_training():
    """Two layers of the climbmix model, trained two steps eager and with every
    block (and the final norm) compiled by inductor, the trainer's default.

    Step 0 is the reference's all-tie start (zero routers): every token goes to
    experts 0..3, so the counts are 2T for those four and 0 for the rest, the load-balance
    loss is exactly K and the z-loss (ln E)^2; eager and compiled give the same
    losses and gradients to 2e-3. Step 1 (routers moved by one AdamW step) gives
    the same loss to 1e-3."""
    say("climbmix shape: H=1024 E=32 K=4 I=512, 2 layers, T=8192, autocast bf16, fused AdamW")
    torch.manual_seed(0)
    base = _ClimbmixStandIn().to(DEV)
    eager = _climbmix_steps(copy.deepcopy(base), None)
    torch._dynamo.reset()
    comp = _climbmix_steps(copy.deepcopy(base), "inductor")
    T, E, K, L = 8192, 32, 4, 2
    import math
    want_counts = torch.tensor([float(L * T)] * K + [0.0] * (E - K))
    want_aux = 1e-3 * K + 1e-3 * math.log(E) ** 2
    for run in (eager, comp):
        assert torch.equal(run[0]["counts"].cpu(), want_counts)
        assert abs(run[0]["aux"].item() - want_aux) <= 1e-6 * want_aux
        assert all(torch.isfinite(r["ce"]) for r in run)
    assert rel(comp[0]["ce"], eager[0]["ce"]) <= 1e-4
    worst = 0.0
    for i, (a, b) in enumerate(zip(eager[0]["grads"], comp[0]["grads"])):
        worst = max(worst, rel(b, a))
        assert rel(b, a) <= 2e-3, f"step-0 grad {i}: rel {rel(b, a):.3e}"
    say(f"  step 0 grads: worst rel {worst:.2e}")
    # every router received a gradient at the all-tie start (the aux loss reaches it)
    for blk_grads in (eager[0]["grads"], comp[0]["grads"]):
        names = [n for n, _ in base.named_parameters()]
        for n, gr in zip(names, blk_grads):
            if "router" in n:
                assert gr.abs().max().item() > 0, n
    assert rel(comp[1]["ce"], eager[1]["ce"]) <= 1e-3
    assert rel(comp[1]["aux"], eager[1]["aux"]) <= 1e-3
