"""GPU: pmoe_expert_ffn_forward_noalloc (static device scratch) against pmoe_expert_ffn_forward.

The allocation-free variant runs the same kernels with the permutation's
chunk histograms in a static device array instead of a caller workspace, so
every output must equal the workspace entry point's bit for bit. Two calls in
a row, the second smaller, and the largest size the static scratch admits;
sizes beyond it are rejected before any launch.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from tests._gpu_helpers import DEV, gen, routing, say

pytestmark = pytest.mark.gpu


def _inputs(T, K, E, H, I, seed):
    g = gen(seed)
    return {
        "hidden": torch.randn(T, H, generator=g).to(torch.bfloat16).to(DEV),
        "idx": routing(T, K, E, seed=seed, mode="zipf").to(DEV),
        "w": torch.rand(T, K, generator=g).to(DEV),
        "gu": (torch.randn(E, 2 * I, H, generator=g) * 0.05).to(torch.bfloat16).to(DEV),
        "dn": (torch.randn(E, H, I, generator=g) * 0.05).to(torch.bfloat16).to(DEV),
    }


def _outputs(T, K, E, H, I):
    """out, counts, offs, sorted_pair, inv_pos, sorted_token, sorted_w, gate_up_out, mid, y."""
    P = T * K
    bf, i32 = torch.bfloat16, torch.int32
    return [torch.empty(T, H, dtype=bf, device=DEV), torch.empty(E, dtype=i32, device=DEV),
            torch.empty(E, dtype=i32, device=DEV), torch.empty(P, dtype=i32, device=DEV),
            torch.empty(P, dtype=i32, device=DEV), torch.empty(P, dtype=i32, device=DEV),
            torch.empty(P, dtype=torch.float32, device=DEV), torch.empty(P, 2 * I, dtype=bf, device=DEV),
            torch.empty(P, I, dtype=bf, device=DEV), torch.empty(P, H, dtype=bf, device=DEV)]


def _call(name, inp, outs, T, K, E, H, I, ws=None):
    from pluggy_amd import _lib

    p = _lib.ptr
    args = [p(inp["hidden"]), p(inp["idx"]), p(inp["w"]), _lib.PMOE_F32, p(inp["gu"]), p(inp["dn"]), _lib.PMOE_BF16,
            T, K, E, H, I] + [p(o) for o in outs]
    if ws is not None:
        args += [p(ws), ws.numel()]
    _lib.call(name, *args, _lib.stream_of(inp["hidden"]))


@pytest.mark.parametrize("first,second", [
    ((131072, 8, 128, 64, 32), (4096, 8, 128, 256, 128)),    # the largest admitted size, then a smaller one
    ((6000, 6, 100, 128, 64), (1500, 2, 16, 64, 32)),
])
def test_noalloc_forward_matches_workspace_entry_point(first, second):
    from pluggy_amd import _lib

    for n, (T, K, E, H, I) in enumerate((first, second)):
        say(f"noalloc call {n}: T={T} K={K} E={E} H={H} I={I} pairs={T * K}")
        inp = _inputs(T, K, E, H, I, seed=7 + n)
        got = _outputs(T, K, E, H, I)
        _call("pmoe_expert_ffn_forward_noalloc", inp, got, T, K, E, H, I)
        want = _outputs(T, K, E, H, I)
        ws = _lib.workspace(_lib.size("pmoe_expert_ffn_forward_workspace_size", T, K, E), inp["hidden"].device)
        _call("pmoe_expert_ffn_forward", inp, want, T, K, E, H, I, ws)
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(got, want)):
            assert torch.equal(a, b), f"output {i} differs"


def test_noalloc_rejects_sizes_beyond_the_static_scratch():
    from pluggy_amd import _lib

    T, K, E, H, I = 131073, 8, 128, 64, 32  # one chunk more than 256 KiB of histograms hold
    dev = ctypes.c_void_p(256)  # routing weights must be given; the size check returns before any launch
    outs = [None] * 10
    outs[6] = dev  # sorted_w
    with pytest.raises(RuntimeError, match="static maximum"):
        _lib.call("pmoe_expert_ffn_forward_noalloc", None, None, dev, _lib.PMOE_F32, None, None, _lib.PMOE_BF16,
                  T, K, E, H, I, *outs, None)
