"""GPU: the block's forward under HIP graph capture (torch.cuda.CUDAGraph).

A serving loop replays a captured forward instead of launching its kernels
one by one. Every entry point the forward calls takes the caller's stream,
allocates nothing itself and never synchronises the host, and no kernel of the
path clears memory with hipMemsetAsync, so the forward captures as it stands.
Checked at the decode size (the few-token tile shapes) and at 1024 tokens (the
regular tiles): three replays, each on a new input written into the captured
input tensor, with eager forwards in between, every replay bitwise equal to the
eager forward on the same input (the kernels are deterministic).
"""

from __future__ import annotations

import pytest
import torch

from tests._gpu_helpers import DEV, gen, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def layer():
    import pluggy_amd
    from pluggy_amd.workloads import CONFIGS, make_inputs

    cfg = CONFIGS[5]  # the config-2 layer (H 2048, E 128, K 8, I 768)
    inp = make_inputs(cfg, device=DEV)
    mlp = pluggy_amd.Qwen3MoeSparseMLP(cfg.hidden, cfg.inter, cfg.experts, cfg.top_k).to(DEV)
    with torch.no_grad():
        mlp.router.weight.copy_(inp["router_weight"])
    mlp.experts.gate_up_proj.data = inp["gate_up_proj"]
    mlp.experts.down_proj.data = inp["down_proj"]
    return mlp, cfg


@pytest.mark.parametrize("T", [64, 1024])
def test_forward_graph_replays_match_eager(layer, T):
    mlp, cfg = layer
    H = cfg.hidden
    say(f"graph capture of the forward, T={T}")
    g = gen(31 + T)
    xs = [torch.randn(1, T, H, generator=g).to(torch.bfloat16).to(DEV) for _ in range(4)]
    x = xs[0].clone()
    with torch.no_grad():
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):  # warm-up on a side stream, as torch's capture recipe asks
            for _ in range(2):
                mlp(x)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            y = mlp(x)
        for r in range(1, 4):
            x.copy_(xs[r])
            graph.replay()
            torch.cuda.synchronize()
            got = y.clone()
            want = mlp(xs[r])  # eager, between replays
            torch.cuda.synchronize()
            assert torch.equal(got, want), f"replay {r} differs from the eager forward"
            assert not torch.equal(got, mlp(xs[r - 1])), "the replay read the new input"



def test_backward_under_capture_raises(layer):
    """The backward ops refuse a capturing stream with a clear error before any
    C-ABI call: a capture of forward + backward raises the guard's
    RuntimeError (the forward kernels in it are capture-safe; no backward
    kernel is launched)."""
    mlp, cfg = layer
    say("graph capture of forward + backward must raise the capture guard")
    g = gen(5)
    x = torch.randn(1, 256, cfg.hidden, generator=g).to(torch.bfloat16).to(DEV).requires_grad_(True)
    dy = torch.randn(1, 256, cfg.hidden, generator=g).to(torch.bfloat16).to(DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up: forward and backward once, eagerly
        mlp(x).backward(dy)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="not supported under HIP graph capture"):
        with torch.cuda.graph(graph):
            y = mlp(x)
            y.backward(dy)
    torch.cuda.synchronize()
    x.grad = None
    mlp(x).backward(dy)  # eager work still runs after the refused capture
    torch.cuda.synchronize()
    assert x.grad is not None and torch.isfinite(x.grad.float()).all()


@pytest.mark.skip(reason="the MoE backward is not supported under HIP graph capture: the one trial capture of it "
                         "(torch.cuda.make_graphed_callables on the block) ended in a host segmentation fault whose "
                         "cause is not known, and the backward ops now refuse a capturing stream")
def test_backward_graph_replays_match_eager(layer):
    """Forward and backward captured with torch.cuda.make_graphed_callables and
    replayed three times, each replay's output and gradients bitwise equal to
    eager on the same input (kept, skipped, until the capture is supported)."""
    mlp, cfg = layer
    g = gen(11)
    xs = [torch.randn(1, 256, cfg.hidden, generator=g).to(torch.bfloat16).to(DEV) for _ in range(4)]
    dy = torch.randn(1, 256, cfg.hidden, generator=g).to(torch.bfloat16).to(DEV)
    x0 = xs[0].clone().requires_grad_(True)
    graphed = torch.cuda.make_graphed_callables(mlp, (x0,))
    for r in range(1, 4):
        xg = xs[r].clone().requires_grad_(True)
        out = graphed(xg)
        out.backward(dy)
        torch.cuda.synchronize()
        got_out, got_gx = out.detach().clone(), xg.grad.clone()
        xe = xs[r].clone().requires_grad_(True)
        want = mlp(xe)
        want.backward(dy)
        torch.cuda.synchronize()
        assert torch.equal(got_out, want.detach()) and torch.equal(got_gx, xe.grad)
