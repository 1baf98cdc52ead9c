"""The pmoe custom ops under torch.library's checks and torch.compile.

The reference compiles every transformer block (pluggy/training/trainer.py:
292-293), so the drop-in must trace without graph breaks: the MoE half of a
block (RMSNorm -> sparse MLP -> residual add, qwen3_moe.py:281) is compiled
with ``fullgraph=True``, including the gradient of an aux loss through the
router logits. With ``backend="aot_eager"`` the same kernels run, so the
results must equal eager bit for bit. With the trainer's own backend (inductor,
``block.compile(mode="default")``) the RMSNorm, the residual add and the
z-loss become generated kernels whose fp32 reductions may be ordered
differently, so the bar is the dtype's (rel-L2 and max-abs as everywhere
else), the routing must equal eager's, and a second call must reproduce the
first bit for bit.
"""

import pytest
import torch
from torch import nn

from _gpu_helpers import DEV, MAX_ABS_FRAC, check_close, gen, say

pytestmark = pytest.mark.gpu


def _pa():
    import pluggy_amd
    return pluggy_amd


def _weights(E, H, I, seed=0):
    g = gen(seed)
    rw = (torch.randn(E, H, generator=g) * 0.02).to(DEV)
    gu = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    dn = (torch.randn(E, H, I, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    return rw, gu, dn


def test_opcheck_custom_ops():
    _pa()
    T, H, E, K, I = 96, 128, 8, 2, 64
    rw, gu, dn = _weights(E, H, I)
    x = torch.randn(T, H, generator=gen(1)).to(torch.bfloat16).to(DEV)
    say(f"opcheck T={T} H={H} E={E} K={K} I={I}")
    tests = ("test_schema", "test_autograd_registration", "test_faketensor")
    torch.library.opcheck(torch.ops.pmoe.router_fwd, (x, rw, K, True, None), test_utils=tests)
    torch.library.opcheck(torch.ops.pmoe.sparse_moe_fwd, (x.requires_grad_(True), rw.requires_grad_(True),
                                                          gu.requires_grad_(True), dn.requires_grad_(True), K, True,
                                                          None), test_utils=tests)
    logits, tw, ti = _pa().router_topk(x.detach(), rw.detach(), K)
    torch.library.opcheck(torch.ops.pmoe.expert_ffn_fwd, (x.detach(), ti, tw, gu.detach(), dn.detach()),
                          test_utils=tests)


class _MoEHalfBlock(nn.Module):
    """x + SparseMLP(RMSNorm(x)): the MoE half of Qwen3MoeTransformerBlock (qwen3_moe.py:281)."""

    def __init__(self, H, I, E, K):
        super().__init__()
        self.norm = nn.RMSNorm(H, eps=1e-6)
        self.ffn = _pa().Qwen3MoeSparseMLP(H, I, E, K)

    def forward(self, x):
        y = x + self.ffn(self.norm(x))
        z = torch.logsumexp(self.ffn.last_router_logits, dim=-1).pow(2).mean()  # router z-loss (qwen3_moe.py:311-316)
        return y, z


@pytest.mark.timeout(600)  # inductor compiles its kernels on first use
@pytest.mark.parametrize("backend", ["aot_eager", "inductor"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_compiled_block_matches_eager(dtype, backend):
    B, S, H, E, K, I = 2, 128, 256, 16, 4, 128
    say(f"compile[{backend}] B={B} S={S} H={H} E={E} K={K} I={I} {dtype}")
    torch.manual_seed(0)
    block = _MoEHalfBlock(H, I, E, K).to(DEV)
    rw, gu, dn = _weights(E, H, I, seed=3)
    with torch.no_grad():
        block.ffn.router.weight.copy_(rw)
        block.ffn.experts.gate_up_proj.copy_(gu.float())
        block.ffn.experts.down_proj.copy_(dn.float())
    block = block.to(dtype)
    block.ffn.router.weight.data = block.ffn.router.weight.data.float()  # fp32 router, as BASELINE config 2
    x0 = torch.randn(B, S, H, generator=gen(5)).to(dtype).to(DEV)

    def run(mod):
        for prm in block.parameters():
            prm.grad = None
        x = x0.clone().requires_grad_(True)
        y, z = mod(x)
        (y.float().pow(2).mean() + 1e-3 * z).backward()
        ids = block.ffn.router.last_stats.expert_counts.clone()
        return [y.detach(), z.detach(), x.grad] + [prm.grad.clone() for prm in block.parameters()], ids

    eager, eager_counts = run(block)
    torch._dynamo.reset()
    if backend == "inductor":
        compiled = torch.compile(block, mode="default", fullgraph=True)  # trainer.py:291-293
    else:
        compiled = torch.compile(block, backend="aot_eager", fullgraph=True)
    got, got_counts = run(compiled)
    got2, _ = run(compiled)  # a second call reuses the compiled graph
    assert torch.equal(got_counts, eager_counts)
    names = ["y", "z", "dx"] + [n for n, _ in block.named_parameters()]
    for n, a, b, c in zip(names, eager, got, got2):
        say(f"  {n}: max|compiled - eager| = {(a.float() - b.float()).abs().max().item():.3e}")
        if backend == "aot_eager":
            assert torch.equal(a, b), n
        else:
            check_close(f"{n} (inductor vs eager)", b, a, 1e-2 if dtype == torch.bfloat16 else 1e-5,
                        MAX_ABS_FRAC[dtype])
        assert torch.equal(b, c), n


@pytest.mark.timeout(600)  # inductor compiles its kernels on first use
def test_compiled_block_dynamic_sequence_lengths():
    """The trainer's compiled blocks see different sequence lengths; after the
    first recompile torch.compile traces them with a symbolic length, through
    the custom ops' fake implementations. Three lengths under inductor, each
    against eager (bf16 bar) with the same routing."""
    from _gpu_helpers import MAX_ABS_FRAC, check_close
    H, E, K, I = 256, 16, 4, 128
    torch.manual_seed(0)
    block = _MoEHalfBlock(H, I, E, K).to(DEV)
    rw, gu, dn = _weights(E, H, I, seed=7)
    with torch.no_grad():
        block.ffn.router.weight.copy_(rw)
        block.ffn.experts.gate_up_proj.copy_(gu.float())
        block.ffn.experts.down_proj.copy_(dn.float())
    block = block.to(torch.bfloat16)
    block.ffn.router.weight.data = block.ffn.router.weight.data.float()
    torch._dynamo.reset()
    compiled = torch.compile(block, mode="default", fullgraph=True)

    def run(mod, x0):
        for prm in block.parameters():
            prm.grad = None
        x = x0.clone().requires_grad_(True)
        y, z = mod(x)
        (y.float().pow(2).mean() + 1e-3 * z).backward()
        counts = block.ffn.router.last_stats.expert_counts.clone()
        return [y.detach(), x.grad] + [prm.grad.clone() for prm in block.parameters()], counts

    for S in (128, 96, 160):
        say(f"dynamic compile S={S}")
        x0 = torch.randn(2, S, H, generator=gen(100 + S)).to(torch.bfloat16).to(DEV)
        ref, ref_counts = run(block, x0)
        got, got_counts = run(compiled, x0)
        assert torch.equal(ref_counts, got_counts)
        for i, (a, b) in enumerate(zip(ref, got)):
            check_close(f"S={S} record {i}", b, a, 1e-2, MAX_ABS_FRAC[torch.bfloat16])
