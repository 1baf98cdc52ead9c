"""Shape-only (fake) implementations of the pmoe custom ops, on the CPU.

These are what ``torch.compile`` and FakeTensor tracing see in place of the
HIP kernels; the GPU tests compare them with the real outputs
(``tests/test_gpu_compile.py``).
"""

import pytest
import torch

pytestmark = []

T, H, E, K, I = 64, 32, 8, 2, 16
P = T * K


def _meta(*shape, dtype=torch.bfloat16):
    return torch.empty(*shape, dtype=dtype, device="meta")


def _sig(ts):
    return [(tuple(t.shape), t.dtype) for t in ts]


@pytest.fixture(scope="module")
def pmoe_ops():
    import pluggy_amd  # noqa: F401  (registers the ops)
    return torch.ops.pmoe


def test_router_fwd_fake(pmoe_ops):
    out = pmoe_ops.router_fwd(_meta(T, H), _meta(E, H, dtype=torch.float32), K, True, None)
    f32, bf = torch.float32, torch.bfloat16
    assert _sig(out) == [((T, E), f32), ((T, K), bf), ((T, K), torch.int64), ((T, K), f32), ((E,), torch.int32),
                         ((E,), f32), ((1,), f32)]


def test_router_bwd_fake(pmoe_ops):
    x, w = _meta(T, H), _meta(E, H, dtype=torch.float32)
    gx, gw = pmoe_ops.router_bwd(x, w, _meta(T, E, dtype=torch.float32), _meta(T, K, dtype=torch.int64),
                                 _meta(T, K, dtype=torch.float32), _meta(T, K), None, True)
    assert _sig([gx, gw]) == [((T, H), torch.bfloat16), ((E, H), torch.float32)]


def test_expert_ffn_fwd_fake(pmoe_ops):
    out = pmoe_ops.expert_ffn_fwd(_meta(T, H), _meta(T, K, dtype=torch.int64), _meta(T, K), _meta(E, 2 * I, H),
                                  _meta(E, H, I))
    bf, i32, f32 = torch.bfloat16, torch.int32, torch.float32
    # out, then what the backward reads: offs, inv_pos, sorted_token, sorted_w, gate_up_out, mid
    assert _sig(out) == [((T, H), bf), ((E,), i32), ((P,), i32), ((P,), i32), ((P,), f32), ((P, 2 * I), bf),
                         ((P, I), bf)]


def test_sparse_moe_fwd_fake(pmoe_ops):
    out = pmoe_ops.sparse_moe_fwd(_meta(T, H), _meta(E, H, dtype=torch.float32), _meta(E, 2 * I, H), _meta(E, H, I),
                                  K, False, None)
    bf, f32, i32 = torch.bfloat16, torch.float32, torch.int32
    assert _sig(out) == [((T, H), bf), ((T, E), f32), ((E,), i32), ((E,), f32), ((1,), f32), ((T, K), torch.int64),
                         ((T, K), f32), ((T, K), bf), ((E,), i32), ((P,), i32), ((P,), i32), ((P,), f32),
                         ((P, 2 * I), bf), ((P, I), bf)]


def test_backward_fakes_drop_unneeded_grads(pmoe_ops):
    gu, dn = _meta(E, 2 * I, H), _meta(E, H, I)
    i32, f32 = torch.int32, torch.float32
    # the down dgrad: grad_gate_up_out and, when asked, the routing weights' gradient (fp32)
    g_gu, g_w = pmoe_ops.expert_bwd_dgrad(_meta(T, H), dn, _meta(E, dtype=i32), _meta(P, dtype=i32),
                                          _meta(P, dtype=i32), _meta(P, dtype=f32), _meta(P, 2 * I), K, True)
    assert _sig([g_gu, g_w]) == [((P, 2 * I), torch.bfloat16), ((T, K), f32)]
    _, g_w = pmoe_ops.expert_bwd_dgrad(_meta(T, H), dn, _meta(E, dtype=i32), _meta(P, dtype=i32),
                                       _meta(P, dtype=i32), _meta(P, dtype=f32), _meta(P, 2 * I), K, False)
    assert g_w.numel() == 0
    args = (_meta(P, 2 * I), _meta(T, H), _meta(T, H), gu, dn, _meta(E, dtype=i32), _meta(P, dtype=i32),
            _meta(P, dtype=i32), _meta(P, I), None, K)
    gh, ggu, gdn = pmoe_ops.expert_bwd(*args, [True, False, True], [False, False])
    assert _sig([gh, gdn]) == [((T, H), torch.bfloat16), ((E, H, I), torch.bfloat16)]
    assert ggu.numel() == 0  # absent gradient: empty stand-in
    # gradients of fp32 master weights come out in fp32 from bf16 operands
    gh, ggu, gdn = pmoe_ops.expert_bwd(*args, [False, True, True], [True, True])
    assert _sig([ggu, gdn]) == [((E, 2 * I, H), torch.float32), ((E, H, I), torch.float32)]
    assert gh.numel() == 0


def test_forward_ops_take_optional_masters(pmoe_ops):
    # the fp32 masters ride along for autograd only: outputs are those of the bf16 copies
    f32 = torch.float32
    out = pmoe_ops.sparse_moe_fwd(_meta(T, H), _meta(E, H, dtype=f32), _meta(E, 2 * I, H), _meta(E, H, I), K, True,
                                  None, _meta(E, 2 * I, H, dtype=f32), _meta(E, H, I, dtype=f32))
    assert _sig(out[:1]) == [((T, H), torch.bfloat16)] and len(out) == 14
    out = pmoe_ops.expert_ffn_fwd(_meta(T, H), _meta(T, K, dtype=torch.int64), _meta(T, K), _meta(E, 2 * I, H),
                                  _meta(E, H, I), None, _meta(E, H, I, dtype=f32))
    assert _sig(out[:1]) == [((T, H), torch.bfloat16)] and len(out) == 7


def test_moe_sublayer_fwd_fake(pmoe_ops):
    # fp32 residual stream, bf16 compute (the experts' dtype)
    out = pmoe_ops.moe_sublayer_fwd(_meta(T, H, dtype=torch.float32), _meta(H, dtype=torch.float32), 1e-6,
                                    _meta(E, H, dtype=torch.bfloat16), _meta(E, 2 * I, H), _meta(E, H, I), K, True,
                                    None)
    bf, f32, i32 = torch.bfloat16, torch.float32, torch.int32
    assert _sig(out) == [((T, H), f32), ((T, E), f32), ((E,), i32), ((E,), f32), ((1,), f32), ((T, H), bf),
                         ((T,), f32), ((T, K), torch.int64), ((T, K), f32), ((T, K), bf), ((E,), i32), ((P,), i32),
                         ((P,), i32), ((P,), f32), ((P, 2 * I), bf), ((P, I), bf)]


def test_sublayer_backward_fakes(pmoe_ops):
    x, nw = _meta(T, H, dtype=torch.float32), _meta(H, dtype=torch.float32)
    i32 = torch.int32
    outs = pmoe_ops.sublayer_bwd(_meta(P, 2 * I), _meta(T, H), _meta(T, H), _meta(E, 2 * I, H), _meta(E, H, I),
                                 _meta(E, dtype=i32), _meta(P, dtype=i32), _meta(P, dtype=i32), _meta(P, I),
                                 _meta(T, H), x, nw, _meta(T, dtype=torch.float32), x, K, [True, False, True, True],
                                 [False, True])
    assert _sig(outs) == [((T, H), torch.float32), ((0,), torch.float32), ((E, 2 * I, H), torch.bfloat16),
                          ((E, H, I), torch.float32)]


@pytest.mark.parametrize("op", ["router_bwd", "expert_bwd_dgrad", "expert_bwd", "sublayer_bwd"])
def test_backward_ops_refuse_a_capturing_stream(monkeypatch, op):
    """Under HIP graph capture each backward op raises before any C-ABI call
    (the capture state is faked here, so nothing reaches the library: CPU
    tensors would make a C-ABI call fail differently)."""
    import torch

    import pluggy_amd  # noqa: F401  (registers torch.ops.pmoe)

    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    t = torch.zeros(4, 8)
    i32 = torch.zeros(4, dtype=torch.int32)
    args = {
        "router_bwd": (t, torch.zeros(2, 8), torch.zeros(4, 2), torch.zeros(4, 1, dtype=torch.int64),
                       torch.zeros(4, 1), None, None, True),
        "expert_bwd_dgrad": (t, torch.zeros(2, 8, 4), i32[:2], i32, i32, torch.zeros(4), torch.zeros(4, 8), 1, False),
        "expert_bwd": (torch.zeros(4, 8), t, t, torch.zeros(2, 8, 8), torch.zeros(2, 8, 4), i32[:2], i32, i32,
                       torch.zeros(4, 4), None, 1, [True, False, False], [False, False]),
        "sublayer_bwd": (torch.zeros(4, 8), t, t, torch.zeros(2, 8, 8), torch.zeros(2, 8, 4), i32[:2], i32, i32,
                         torch.zeros(4, 4), None, t, torch.ones(8), torch.ones(4), None, 1,
                         [True, False, False, False], [False, False]),
    }[op]
    with pytest.raises(RuntimeError, match="not supported under HIP graph capture"):
        getattr(torch.ops.pmoe, op)(*args)


def test_weight_cast_cache_keys_on_the_master_version():
    """The cached bf16 copy of an fp32 master is reused while its version,
    storage and layout are unchanged, remade after an in-place update, and
    (the documented limit) not remade after a write through ``.data``."""
    import pluggy_amd
    import pluggy_amd.moe as M

    w = torch.nn.Parameter(torch.randn(4, 8))
    with pluggy_amd.weight_cast_cache():
        c1, master = M._compute_weight(w, torch.bfloat16)
        assert master is w and c1.dtype == torch.bfloat16 and torch.equal(c1, w.detach().to(torch.bfloat16))
        c2, _ = M._compute_weight(w, torch.bfloat16)
        assert c2 is c1
        with torch.no_grad():
            w.add_(1.0)
        c3, _ = M._compute_weight(w, torch.bfloat16)
        assert c3 is not c1 and torch.equal(c3, w.detach().to(torch.bfloat16))
        w.data.mul_(2.0)  # not tracked by the version counter
        c4, _ = M._compute_weight(w, torch.bfloat16)
        assert c4 is c3
        # non-leaf tensors (e.g. the padded master) are cast every time
        p = w * 1.0
        a, _ = M._compute_weight(p, torch.bfloat16)
        b, _ = M._compute_weight(p, torch.bfloat16)
        assert a is not b
    assert not M._cast_cache
    c5, _ = M._compute_weight(w, torch.bfloat16)
    assert torch.equal(c5, w.detach().to(torch.bfloat16))
