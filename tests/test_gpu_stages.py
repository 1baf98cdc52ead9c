"""GPU parity of each kernel stage against CPU references (fp64 or the oracle).

Integer work (permutation, selection, row gather) must be bit-exact. GEMM
stages are compared with fp64 per-expert products: rel-L2 <= 1e-2 for bf16
<= 5e-4 for fp16 (its outputs are rounded to 11
significant bits: RMS error about 1.4e-4, where a bf16 rounding by mistake
would give about 1.1e-3) and <= 1e-5 for fp32 arithmetic; the max-abs error is
printed next to each figure.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from tests._gpu_helpers import (DEV, MAX_ABS_FRAC, check_close, gen, max_abs, ref_grouped, ref_wgrad, rel,
                                routing, say, seg_bounds, silu64, to_np)

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: 1e-2, torch.float16: 5e-4, torch.float32: 1e-5}
# row movers (one rounding of an fp32 sum) and the whole-operator comparisons
ROW_TOL = {torch.bfloat16: 4e-3, torch.float16: 5e-4, torch.float32: 1e-6}
DTYPES = [torch.bfloat16, torch.float16, torch.float32]


def _ops():
    from pluggy_amd import ops
    return ops


# ------------------------------------------------------------- permutation


@pytest.mark.parametrize("T,K,E,mode", [
    (1, 1, 1, "uniform"), (7, 2, 8, "uniform"), (2048, 2, 8, "uniform"), (3000, 4, 33, "one"),
    (100, 8, 8, "uniform"), (8192, 8, 128, "uniform"), (8192, 8, 128, "zipf"), (4099, 6, 1000, "low"),
    # one chunk of pairs or less: the single-block path (P = 2048 is its largest case)
    (256, 8, 128, "zipf"), (64, 8, 1000, "low"), (40, 3, 256, "one"), (257, 8, 128, "uniform"),
    # 64 chunks, the most the scatter scans itself; then the separate-scan path
    (16384, 8, 128, "zipf"), (20000, 8, 128, "uniform"), (9000, 8, 1000, "low"),
])
def test_permute_bitexact(T, K, E, mode):
    say(f"permute T={T} K={K} E={E} mode={mode}")
    idx = routing(T, K, E, seed=T + E, mode=mode)
    counts, offs, sp, inv = _ops().permute(idx.to(DEV), E)
    torch.cuda.synchronize()
    rc, ro, rsp, rinv = O.permute(idx, E)
    assert np.array_equal(to_np(counts), rc.astype(np.int32))
    assert np.array_equal(to_np(offs), ro)
    assert np.array_equal(to_np(sp), rsp)
    assert np.array_equal(to_np(inv), rinv)
    # the one-pass form with the GEMMs' row tables (bf16, fp16 and fp32 weights, and none)
    for wdt in (torch.bfloat16, torch.float16, torch.float32, None):
        w = None if wdt is None else torch.rand(T, K, generator=gen(T)).to(wdt)
        c2, o2, sp2, inv2, tok, sw = _ops().permute_rows(idx.to(DEV), None if w is None else w.to(DEV), E)
        assert np.array_equal(to_np(c2), rc.astype(np.int32)) and np.array_equal(to_np(o2), ro)
        assert np.array_equal(to_np(sp2), rsp) and np.array_equal(to_np(inv2), rinv)
        assert np.array_equal(to_np(tok), rsp // K)
        if w is None:
            assert sw is None
        else:
            assert torch.equal(sw.cpu(), w.float().reshape(-1)[torch.from_numpy(rsp).long()])


def test_permute_deterministic():
    idx = routing(8192, 8, 128, seed=3, mode="zipf").to(DEV)
    a = _ops().permute(idx, 128)
    b = _ops().permute(idx, 128)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


# ----------------------------------------------------------- row movement


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("T,K,E,H", [(300, 4, 16, 264), (64, 8, 128, 2048), (200, 3, 12, 520), (128, 8, 16, 4096)])
def test_dispatch_combine(dtype, T, K, E, H):
    say(f"dispatch/combine T={T} K={K} E={E} H={H} {dtype}")
    ops = _ops()
    g = gen(1)
    x = torch.randn(T, H, generator=g).to(dtype)
    idx = routing(T, K, E, seed=2)
    w = torch.rand(T, K, generator=g).to(dtype)
    counts, offs, sp, inv = ops.permute(idx.to(DEV), E)
    xp = ops.dispatch(x.to(DEV), inv, K)
    ref_xp = x[torch.from_numpy(O.permute(idx, E)[2].astype(np.int64)) // K]
    assert torch.equal(xp.cpu(), ref_xp), "dispatch must be a bit-exact gather"
    # combine: out[t] = sum_k w[t,k] * y[inv[t,k]]
    y = torch.randn(T * K, H, generator=g).to(dtype)
    out = ops.combine(y.to(DEV), w.to(DEV), inv)
    inv_c = inv.cpu().long().view(T, K)
    ref = (w.double().unsqueeze(-1) * y.double()[inv_c]).sum(1)
    say(f"  combine rel={rel(out, ref):.2e} maxabs={max_abs(out, ref):.2e}")
    assert rel(out, ref) < ROW_TOL[dtype]
    # combine backward
    go = torch.randn(T, H, generator=g).to(dtype)
    gy, gw = ops.combine_backward(go.to(DEV), y.to(DEV), w.to(DEV), inv)
    ref_gy = torch.zeros(T * K, H, dtype=torch.float64)
    ref_gy[inv_c.reshape(-1)] = (w.double().unsqueeze(-1) * go.double().unsqueeze(1)).reshape(T * K, H)
    ref_gw = (go.double().unsqueeze(1) * y.double()[inv_c]).sum(-1)
    assert rel(gy, ref_gy) < ROW_TOL[dtype]
    assert rel(gw, ref_gw) < max(ROW_TOL[dtype], 1e-5)
    # dispatch backward: grad_x[t] = sum_k gxp[inv[t,k]]
    gxp = torch.randn(T * K, H, generator=g).to(dtype)
    gx = ops.dispatch_backward(gxp.to(DEV), inv, T, K)
    ref_gx = gxp.double()[inv_c].sum(1)
    assert rel(gx, ref_gx) < ROW_TOL[dtype]
    # with an addend row (the router's share of the input gradient), summed first
    add = torch.randn(T, H, generator=g).to(dtype)
    gx2 = ops.dispatch_backward(gxp.to(DEV), inv, T, K, add=add.to(DEV))
    assert rel(gx2, ref_gx + add.double()) < ROW_TOL[dtype]


# -------------------------------------------------------------- GEMMs


GEMM_CASES = [
    # T, K, E, H, I, routing mode
    (512, 4, 16, 256, 192, "uniform"),
    (300, 2, 8, 264, 40, "uniform"),      # ragged H and I (masking along k and n)
    (1024, 8, 64, 512, 128, "zipf"),       # skewed: empty experts, heavy experts
    (37, 3, 5, 128, 64, "one"),            # tiny: every group below one tile
    (600, 4, 12, 320, 320, "zipf"),        # partial column tiles on the 64-deep-stage engine
    # at most 32 rows per expert on average: the forward GEMMs take the few-token
    # tiles (32 rows x 128 columns, 128-deep stages)
    (64, 8, 128, 2048, 768, "uniform"),    # the decode layer shape
    (100, 4, 32, 264, 72, "zipf"),         # ragged k tail, partial column tiles, experts over 32 rows
    # the Qwen3-235B-A22B layer widths (H = 4096, I = 1536: 128-stage gate_up reductions, 3072-wide
    # gate_up rows) with about 1024 rows per expert, skewed
    (1024, 8, 8, 4096, 1536, "zipf"),
    # one GPU's share at EP = 8 of config 2 (16 experts of about 520 rows, K = 1): down dgrad on the
    # 128-row tiles, the other row-grouped GEMMs on 256-row ones (cases above with 128 to 256 rows
    # per expert and few column tiles take 128-row tiles throughout)
    (8320, 1, 16, 2048, 768, "uniform"),
]


def test_gemm_cases_cover_both_row_tile_shapes():
    """The EP=8-share case above runs down dgrad on the 128-row tiles on this
    device (the engine's choice depends on the CU count), the larger cases on
    256-row tiles, so the stage tests below cover both shapes."""
    from pluggy_amd import _lib

    for code in (_lib.PMOE_BF16, _lib.PMOE_F16):  # fp16 takes the same tiles
        q = lambda kind, T, K, E, H, I: _lib.load().pmoe_expert_gemm_tile_rows(  # noqa: E731
            kind, T * K, E, H, I, code, 0)
        assert q(2, 8320, 1, 16, 2048, 768) == 128  # down dgrad at the EP=8 share
        assert q(0, 8320, 1, 16, 2048, 768) == 256  # gate_up fwd there
        assert q(0, 1024, 8, 8, 4096, 1536) == 256
        assert q(0, 64, 8, 128, 2048, 768) == 32    # the decode shape's forward


def _gemm_inputs(T, K, E, H, I, mode, dtype, seed=0):
    ops = _ops()
    g = gen(seed)
    idx = routing(T, K, E, seed=seed + 11, mode=mode)
    x = torch.randn(T, H, generator=g).to(dtype)
    wgu = (torch.randn(E, 2 * I, H, generator=g) * 0.05).to(dtype)
    wdn = (torch.randn(E, H, I, generator=g) * 0.05).to(dtype)
    counts, offs, sp, inv = ops.permute(idx.to(DEV), E)
    xp = ops.dispatch(x.to(DEV), inv, K)
    return idx, x, wgu, wdn, offs, sp, inv, xp


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("case", GEMM_CASES)
def test_gate_up_swiglu(dtype, case):
    T, K, E, H, I, mode = case
    say(f"gate_up_swiglu {case} {dtype}")
    ops = _ops()
    idx, x, wgu, wdn, offs, sp, inv, xp = _gemm_inputs(T, K, E, H, I, mode, dtype)
    gu, mid = ops.gate_up_swiglu(xp, wgu.to(DEV), offs)
    o = offs.cpu()
    ref = ref_grouped(xp, wgu, o, trans_w=True)
    check_close("gate_up", gu, ref, TOL[dtype], MAX_ABS_FRAC[dtype])
    gq = gu.cpu().double()
    ref_mid = silu64(gq[:, :I]) * gq[:, I:]
    check_close("mid", mid, ref_mid, TOL[dtype], MAX_ABS_FRAC[dtype])


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("case", GEMM_CASES)
def test_down_proj(dtype, case):
    T, K, E, H, I, mode = case
    say(f"down_proj {case} {dtype}")
    ops = _ops()
    idx, x, wgu, wdn, offs, sp, inv, xp = _gemm_inputs(T, K, E, H, I, mode, dtype)
    mid = torch.randn(T * K, I, generator=gen(5)).to(dtype)
    y = ops.down_proj(mid.to(DEV), wdn.to(DEV), offs)
    ref = ref_grouped(mid, wdn, offs.cpu(), trans_w=True)
    check_close("y", y, ref, TOL[dtype], MAX_ABS_FRAC[dtype])


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("case", GEMM_CASES)
def test_down_proj_backward(dtype, case):
    T, K, E, H, I, mode = case
    say(f"down_proj_backward {case} {dtype}")
    ops = _ops()
    idx, x, wgu, wdn, offs, sp, inv, xp = _gemm_inputs(T, K, E, H, I, mode, dtype)
    g = gen(7)
    P = T * K
    gy = torch.randn(P, H, generator=g).to(dtype)
    gu = torch.randn(P, 2 * I, generator=g).to(dtype)
    mid = torch.randn(P, I, generator=g).to(dtype)
    ggu, gdn, _ = ops.down_proj_backward(gy.to(DEV), mid.to(DEV), gu.to(DEV), wdn.to(DEV), offs)
    o = offs.cpu()
    dmid = ref_grouped(gy, wdn, o, trans_w=False)          # (P, I) = gy_e @ W_dn[e]
    gate, up = gu.double()[:, :I], gu.double()[:, I:]
    s = torch.sigmoid(gate)
    ref_ggu = torch.cat([dmid * up * s * (1 + gate * (1 - s)), dmid * gate * s], dim=1)
    check_close("dgate_up", ggu, ref_ggu, TOL[dtype], MAX_ABS_FRAC[dtype])
    ref_gdn = ref_wgrad(gy, mid, o)                        # (E, H, I)
    check_close("d down_proj", gdn, ref_gdn, TOL[dtype], MAX_ABS_FRAC[dtype])
    empty = [e for e, (lo, hi) in enumerate(seg_bounds(o)) if hi == lo]
    for e in empty:
        assert torch.count_nonzero(gdn[e]).item() == 0, "an empty expert has a zero weight gradient"


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("case", GEMM_CASES)
def test_gate_up_backward(dtype, case):
    T, K, E, H, I, mode = case
    say(f"gate_up_backward {case} {dtype}")
    ops = _ops()
    idx, x, wgu, wdn, offs, sp, inv, xp = _gemm_inputs(T, K, E, H, I, mode, dtype)
    P = T * K
    ggu = torch.randn(P, 2 * I, generator=gen(9)).to(dtype)
    gxp, gwgu = ops.gate_up_backward(ggu.to(DEV), xp, wgu.to(DEV), offs)
    o = offs.cpu()
    ref_gxp = ref_grouped(ggu, wgu, o, trans_w=False)      # (P, H) = ggu_e @ W_gu[e]
    check_close("d x_perm", gxp, ref_gxp, TOL[dtype], MAX_ABS_FRAC[dtype])
    ref_gw = ref_wgrad(ggu, xp, o)                         # (E, 2I, H)
    check_close("d gate_up_proj", gwgu, ref_gw, TOL[dtype], MAX_ABS_FRAC[dtype])


@pytest.mark.parametrize("half", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", GEMM_CASES)
def test_weight_gradients_in_fp32(case, half):
    """16-bit operands, fp32 weight gradients (for fp32 master weights): the
    unrounded accumulators of the same tiles, so rounding them gives the 16-bit
    entry point's output bit for bit, and they sit within fp32 summation error
    of the fp64 product."""
    T, K, E, H, I, mode = case
    say(f"wgrad fp32 out {case} {half}")
    ops = _ops()
    bf, f32 = half, torch.float32
    idx, x, wgu, wdn, offs, sp, inv, xp = _gemm_inputs(T, K, E, H, I, mode, bf)
    g = gen(8)
    P = T * K
    gy = torch.randn(P, H, generator=g).to(bf).to(DEV)
    mid = torch.randn(P, I, generator=g).to(bf).to(DEV)
    ggu = torch.randn(P, 2 * I, generator=g).to(bf).to(DEV)
    o = offs.cpu()
    for name, f32_out, bf_out, ref in (
            ("down", ops.down_proj_wgrad(gy, mid, offs, E, f32), ops.down_proj_wgrad(gy, mid, offs, E),
             ref_wgrad(gy.cpu(), mid.cpu(), o)),
            ("gate_up", ops.gate_up_wgrad(ggu, xp, offs, E, f32), ops.gate_up_wgrad(ggu, xp, offs, E),
             ref_wgrad(ggu.cpu(), xp.cpu(), o))):
        assert f32_out.dtype == f32 and bf_out.dtype == bf
        check_close(name, f32_out, ref, 2e-5, 1e-5)
        assert torch.equal(f32_out.to(bf), bf_out), name
        for e, (lo, hi) in enumerate(seg_bounds(o)):
            if hi == lo:
                assert torch.count_nonzero(f32_out[e]).item() == 0, "an empty expert has a zero weight gradient"


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("case", GEMM_CASES)
def test_gathered_rows_and_routing_weights(dtype, case):
    """The forward and backward GEMMs over rows gathered from token-major tensors
    (hidden, the output gradient) with the routing weight in the activation:
    against fp64 of the materialised form (x[sorted_token], w * mid, ...)."""
    T, K, E, H, I, mode = case
    say(f"gathered rows {case} {dtype}")
    ops = _ops()
    idx, x, wgu, wdn, offs, sp, inv, xp = _gemm_inputs(T, K, E, H, I, mode, dtype)
    g = gen(13)
    P = T * K
    tw = torch.rand(T, K, generator=g).to(dtype)
    gout = torch.randn(T, H, generator=g).to(dtype)
    stok, sw = ops.sort_rows(sp, tw.to(DEV), K)
    o = offs.cpu()
    # sort_rows: token and weight of every sorted row, bit for bit
    sp64 = sp.cpu().long()
    assert torch.equal(stok.cpu(), (sp64 // K).int())
    assert torch.equal(sw.cpu(), tw.reshape(-1)[sp64].float())
    tok = stok.cpu().long()
    w64 = sw.cpu().double().unsqueeze(1)
    # forward: gate_up over gathered rows, weighted mid
    gu, mid = ops.gate_up_swiglu(x.to(DEV), wgu.to(DEV), offs, stok, sw)
    ref_gu = ref_grouped(x[tok], wgu, o, trans_w=True)
    check_close("gate_up (gathered)", gu, ref_gu, TOL[dtype], MAX_ABS_FRAC[dtype])
    gq = gu.cpu().double()
    check_close("w * mid", mid, w64 * silu64(gq[:, :I]) * gq[:, I:], TOL[dtype], MAX_ABS_FRAC[dtype])
    # down backward from the gathered output gradient
    ggu, gdn, part = ops.down_proj_backward(gout.to(DEV), mid, gu, wdn.to(DEV), offs, stok, sw, need_part=True)
    G = gout[tok]
    acc = ref_grouped(G, wdn, o, trans_w=False)                     # d(w * mid)
    gate, up = gq[:, :I], gq[:, I:]
    s_ = torch.sigmoid(gate)
    dm = w64 * acc
    ref_ggu = torch.cat([dm * up * s_ * (1 + gate * (1 - s_)), dm * gate * s_], dim=1)
    check_close("dgate_up (gathered, weighted)", ggu, ref_ggu, TOL[dtype], MAX_ABS_FRAC[dtype])
    check_close("d down_proj (gathered)", gdn, ref_wgrad(G, mid.cpu(), o), TOL[dtype], MAX_ABS_FRAC[dtype])
    # the routing weights' gradient: <acc, silu(g) u> per row, by 64-column block, then summed per pair
    prod = acc * (gate * s_ * up)
    nb = (I + 63) // 64
    ref_part = torch.stack([prod[:, 64 * c:64 * (c + 1)].sum(1) for c in range(nb)], 1)
    check_close("weight partials", part, ref_part, 1e-5, 1e-4)
    gtw = ops.pair_weight_grad(part, inv, K)
    ref_gtw = ref_part.sum(1)[inv.cpu().long()].reshape(T, K)
    check_close("d top_weights", gtw, ref_gtw, 1e-5, 1e-4)
    # gate_up backward: dgrad on the sorted rows, wgrad over gathered rows
    g2 = torch.randn(P, 2 * I, generator=gen(17)).to(dtype)
    gxp, gwgu = ops.gate_up_backward(g2.to(DEV), x.to(DEV), wgu.to(DEV), offs, row_index=stok)
    check_close("d x_perm", gxp, ref_grouped(g2, wgu, o, trans_w=False), TOL[dtype], MAX_ABS_FRAC[dtype])
    check_close("d gate_up_proj (gathered)", gwgu, ref_wgrad(g2, x[tok], o), TOL[dtype], MAX_ABS_FRAC[dtype])
    if dtype != torch.float32:
        # fp32 weight gradients over gathered rows: the same tiles unrounded
        f32 = torch.float32
        gw32 = ops.gate_up_wgrad(g2.to(DEV), x.to(DEV), offs, E, f32, row_index=stok)
        gd32 = ops.down_proj_wgrad(gout.to(DEV), mid, offs, E, f32, row_index=stok)
        assert torch.equal(gw32.to(dtype), gwgu) and torch.equal(gd32.to(dtype), gdn)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_epilogue_stores_stay_inside_the_rows(dtype):
    """The epilogues write through buffer descriptors sized to a tile's valid
    rows, with a slab's first row in the instruction's scalar offset: rows past
    the last one must be dropped. One expert of 100 rows (one partial 256-row
    tile) writes into buffers that hold 256 sentinel rows after the 100 the
    call sees: the forward (gate_up pre-activations, the weighted SwiGLU, the
    down rows) and the down dgrad with its routing-weight partials leave every
    sentinel row as it was, and the 100 rows match fp64."""
    from pluggy_amd._lib import call, dtype_code, ptr, stream_of

    P, E, H, I, X = 100, 1, 256, 256, 256
    say(f"epilogue bounds P={P} H={H} I={I} {dtype}")
    g = gen(23)
    dt = dtype_code(dtype)
    nan = float("nan")
    x = torch.randn(P + X, H, generator=g).to(dtype).to(DEV)
    wgu = (torch.randn(E, 2 * I, H, generator=g) * 0.05).to(dtype).to(DEV)
    wdn = (torch.randn(E, H, I, generator=g) * 0.05).to(dtype).to(DEV)
    sw = torch.rand(P + X, generator=g).to(DEV)
    offs = torch.tensor([P], dtype=torch.int32, device=DEV)
    gu = torch.full((P + X, 2 * I), nan, dtype=dtype, device=DEV)
    mid = torch.full((P + X, I), nan, dtype=dtype, device=DEV)
    y = torch.full((P + X, H), nan, dtype=dtype, device=DEV)
    call("pmoe_gate_up_swiglu", ptr(x), None, ptr(sw), P, ptr(wgu), ptr(offs), dt, P, E, H, I, ptr(gu), ptr(mid),
         stream_of(x))
    call("pmoe_down_proj", ptr(mid), ptr(wdn), ptr(offs), dt, P, E, H, I, ptr(y), stream_of(x))
    gout = torch.randn(P + X, H, generator=g).to(dtype).to(DEV)
    gu_in = gu.clone()
    gu_in[P:] = torch.randn(X, 2 * I, generator=g).to(dtype).to(DEV)  # finite past the rows
    ggu = torch.full((P + X, 2 * I), nan, dtype=dtype, device=DEV)
    part = torch.full((P + X, 4), nan, device=DEV)
    call("pmoe_down_proj_backward", ptr(gout), None, ptr(sw), P, None, ptr(gu_in), ptr(wdn), ptr(offs), dt, P, E, H,
         I, ptr(ggu), None, dt, ptr(part), 4, stream_of(x))
    torch.cuda.synchronize()
    for name, t in (("gate_up_out", gu), ("mid", mid), ("y", y), ("d gate_up_out", ggu), ("partials", part)):
        assert torch.isnan(t[P:]).all(), f"{name}: rows past the tile's last were written"
        assert not torch.isnan(t[:P]).any(), f"{name}: a row was not written"
    # the visible rows against fp64
    x64, w64 = x[:P].double().cpu(), sw[:P].double().cpu().unsqueeze(1)
    ref_gu = x64 @ wgu[0].double().cpu().T
    check_close("gate_up_out", gu[:P], ref_gu, TOL[dtype], MAX_ABS_FRAC[dtype])
    gq = gu[:P].double().cpu()
    check_close("mid", mid[:P], w64 * silu64(gq[:, :I]) * gq[:, I:], TOL[dtype], MAX_ABS_FRAC[dtype])
    check_close("y", y[:P], mid[:P].double().cpu() @ wdn[0].double().cpu().T, TOL[dtype], MAX_ABS_FRAC[dtype])
    acc = gout[:P].double().cpu() @ wdn[0].double().cpu()
    gate, up = gu_in[:P].double().cpu()[:, :I], gu_in[:P].double().cpu()[:, I:]
    s_ = torch.sigmoid(gate)
    ref_ggu = torch.cat([w64 * acc * up * s_ * (1 + gate * (1 - s_)), w64 * acc * gate * s_], dim=1)
    check_close("d gate_up_out", ggu[:P], ref_ggu, TOL[dtype], MAX_ABS_FRAC[dtype])


# Rows per expert with every kind of short last m-tile (1, 127, 128, 129 and
# 255 rows of a 256-row tile), experts of under 128 rows (nothing but a short
# tile), full experts (no last tile) and an empty expert.
SHORT_ROWS = [1, 127, 128, 129, 255, 256, 257, 383, 384, 385, 511, 640, 0, 64, 700, 900]


@pytest.mark.parametrize("H, I", [(320, 640), (2048, 768), (768, 200)])
def test_forward_gemms_short_last_tiles(H, I):
    """gate_up (gathered and materialised rows) and down forward at row counts
    whose experts end in short last m-tiles, against fp64. H = 320 and 768: the
    down GEMM's last 256-column tile ends past N; I = 640 and 200: an odd count
    of 128-column activation tiles, the last one partial at I = 200."""
    say(f"short last tiles H={H} I={I}")
    ops = _ops()
    E, dt = len(SHORT_ROWS), torch.bfloat16
    idx = torch.repeat_interleave(torch.arange(E), torch.tensor(SHORT_ROWS)).reshape(-1, 1)
    idx = idx[torch.randperm(idx.shape[0], generator=gen(3))]
    T = idx.shape[0]
    g = gen(21)
    x = torch.randn(T, H, generator=g).to(dt)
    wgu = (torch.randn(E, 2 * I, H, generator=g) * 0.05).to(dt)
    wdn = (torch.randn(E, H, I, generator=g) * 0.05).to(dt)
    tw = torch.rand(T, 1, generator=g).to(dt)
    counts, offs, sp, inv = ops.permute(idx.to(DEV), E)
    assert counts.cpu().tolist() == SHORT_ROWS
    xp = ops.dispatch(x.to(DEV), inv, 1)
    o = offs.cpu()
    gu, mid = ops.gate_up_swiglu(xp, wgu.to(DEV), offs)
    ref = ref_grouped(xp, wgu, o, trans_w=True)
    check_close("gate_up", gu, ref, TOL[dt], MAX_ABS_FRAC[dt])
    gq = gu.cpu().double()
    check_close("mid", mid, silu64(gq[:, :I]) * gq[:, I:], TOL[dt], MAX_ABS_FRAC[dt])
    stok, sw = ops.sort_rows(sp, tw.to(DEV), 1)
    gu2, mid2 = ops.gate_up_swiglu(x.to(DEV), wgu.to(DEV), offs, stok, sw)
    assert torch.equal(gu2, gu), "gathered rows give the materialised rows' pre-activations bit for bit"
    w64 = sw.cpu().double().unsqueeze(1)
    check_close("w * mid (gathered)", mid2, w64 * silu64(gq[:, :I]) * gq[:, I:], TOL[dt], MAX_ABS_FRAC[dt])
    y = ops.down_proj(mid, wdn.to(DEV), offs)
    check_close("y", y, ref_grouped(mid.cpu(), wdn, o, trans_w=True), TOL[dt], MAX_ABS_FRAC[dt])


def test_row_heavy_experts_super_blocks():
    """Experts of 20 and 18 m-tiles against 2 n-tiles (H = 512, I = 256) take the
    super-block tile order (16 m-tiles x 2 n-tiles, then the rest) in the
    forward GEMMs and gate_up's input gradient; their last m-tiles hold 136
    rows (regular) and 48 rows (wide in the forward GEMMs), and a 300-row
    expert has a wide 44-row last tile. Against fp64."""
    ops = _ops()
    H, I, dt = 512, 256, torch.bfloat16
    rows = [5000, 300, 4400]
    say(f"super-blocks rows={rows} H={H} I={I}")
    E = len(rows)
    idx = torch.repeat_interleave(torch.arange(E), torch.tensor(rows)).reshape(-1, 1)
    idx = idx[torch.randperm(idx.shape[0], generator=gen(5))]
    T = idx.shape[0]
    g = gen(23)
    x = torch.randn(T, H, generator=g).to(dt)
    wgu = (torch.randn(E, 2 * I, H, generator=g) * 0.05).to(dt)
    wdn = (torch.randn(E, H, I, generator=g) * 0.05).to(dt)
    counts, offs, sp, inv = ops.permute(idx.to(DEV), E)
    assert counts.cpu().tolist() == rows
    xp = ops.dispatch(x.to(DEV), inv, 1)
    o = offs.cpu()
    gu, mid = ops.gate_up_swiglu(xp, wgu.to(DEV), offs)
    check_close("gate_up", gu, ref_grouped(xp, wgu, o, trans_w=True), TOL[dt], MAX_ABS_FRAC[dt])
    y = ops.down_proj(mid, wdn.to(DEV), offs)
    check_close("y", y, ref_grouped(mid.cpu(), wdn, o, trans_w=True), TOL[dt], MAX_ABS_FRAC[dt])
    gy = torch.randn(T, H, generator=gen(29)).to(dt)
    ggu, gdn, _ = ops.down_proj_backward(gy.to(DEV), mid, gu, wdn.to(DEV), offs)
    dmid = ref_grouped(gy, wdn, o, trans_w=False)
    gq = gu.cpu().double()
    gate, up = gq[:, :I], gq[:, I:]
    s_ = torch.sigmoid(gate)
    ref_ggu = torch.cat([dmid * up * s_ * (1 + gate * (1 - s_)), dmid * gate * s_], dim=1)
    check_close("dgate_up", ggu, ref_ggu, TOL[dt], MAX_ABS_FRAC[dt])
    gx = ops.gate_up_dgrad(ggu, wgu.to(DEV), offs)
    check_close("dx_perm", gx, ref_grouped(ggu.cpu(), wgu, o, trans_w=False), TOL[dt], MAX_ABS_FRAC[dt])


# ----------------------------------------------------------------- router


def _router_weight(W, x_dtype):
    """The router weight beside x of x_dtype: fp32, except fp16 beside fp16 x
    (the fp16 router takes both operands in fp16)."""
    return W.half() if x_dtype == torch.float16 else W


@pytest.mark.parametrize("x_dtype", DTYPES)
@pytest.mark.parametrize("T,H,E,K,norm", [(2048, 512, 8, 2, True), (1000, 2048, 128, 8, True),
                                          (300, 256, 60, 4, False), (64, 2048, 128, 8, True),
                                          # the largest expert count and top-k the kernels take
                                          (256, 256, 1024, 64, True), (130, 264, 200, 13, False),
                                          # the four-rows-per-wave kernel (E <= 256): scalar loads
                                          # (E not a multiple of 4), two experts per lane, K > 16
                                          (2500, 256, 125, 7, True), (70, 512, 30, 3, False),
                                          (2100, 256, 256, 40, True)])
def test_router_forward(x_dtype, T, H, E, K, norm):
    say(f"router T={T} H={H} E={E} K={K} norm={norm} {x_dtype}")
    ops = _ops()
    g = gen(T + E)
    x = torch.randn(T, H, generator=g).to(x_dtype)
    W = _router_weight(torch.randn(E, H, generator=g) * 0.02, x_dtype)
    logits, tw, ti, tw32, counts, psum, lse2 = ops.router_forward(x.to(DEV), W.to(DEV), K, norm)
    ref_logits = (x.double() @ W.double().t())
    r = rel(logits, ref_logits)
    say(f"  logits rel={r:.2e} maxabs={max_abs(logits, ref_logits):.2e}")
    assert r < 1e-5
    # routing is bit-exact given identical fp32 logits
    lg = logits.cpu()
    sel = O.select_topk(lg, K)
    assert np.array_equal(to_np(ti), sel)
    # weights: closed form on the GPU's own logits (fp64)
    ls = lg.double().gather(1, torch.from_numpy(sel))
    p = torch.softmax(lg.double(), -1).gather(1, torch.from_numpy(sel))
    ref_w = torch.softmax(ls, -1) if norm else p
    assert rel(tw32, ref_w) < 1e-5
    assert tw.dtype == x_dtype and rel(tw, ref_w) < {torch.bfloat16: 4e-3, torch.float16: 5e-4}.get(x_dtype, 1e-5)
    # statistics
    rc, rps, rl2 = O.router_stats(lg, torch.from_numpy(sel), E)
    assert np.array_equal(to_np(counts), rc.astype(np.int32))
    assert rel(psum, rps) < 1e-5
    assert abs(lse2.item() - rl2.item()) <= 1e-5 * abs(rl2.item()) + 1e-6


def test_router_ties_and_bias():
    """Zero router weight: every logit ties, so the top-k is experts 0..K-1 with weight 1/K."""
    ops = _ops()
    T, H, E, K = 333, 256, 128, 8
    x = torch.randn(T, H, generator=gen(0)).bfloat16().to(DEV)
    W = torch.zeros(E, H, device=DEV)
    logits, tw, ti, tw32, counts, psum, lse2 = ops.router_forward(x, W, K, True)
    assert torch.equal(ti.cpu(), torch.arange(K).expand(T, K))
    assert torch.allclose(tw32.cpu(), torch.full((T, K), 1.0 / K))
    assert torch.allclose(lse2.cpu(), torch.tensor([T * np.log(E) ** 2], dtype=torch.float32), rtol=1e-5)
    # an additive bias that ranks experts in reverse order
    bias = torch.arange(E, dtype=torch.float32, device=DEV)
    logits, tw, ti, *_ = ops.router_forward(x, W, K, True, bias)
    assert torch.equal(ti.cpu(), torch.arange(E - 1, E - 1 - K, -1).expand(T, K))
    assert torch.equal(logits.cpu(), bias.cpu().expand(T, E))


@pytest.mark.parametrize("norm", [True, False])
@pytest.mark.parametrize("x_dtype", DTYPES)
@pytest.mark.parametrize("T,H,E,K", [(700, 512, 64, 6),
                                     # several 1024-token split-K chunks of the weight gradient and a
                                     # ragged last one; then the config-2 shape (8 chunks)
                                     (3000, 512, 64, 6), (8192, 2048, 128, 8),
                                     # the largest expert count and top-k
                                     (256, 256, 1024, 64)])
def test_router_backward(norm, x_dtype, T, H, E, K):
    say(f"router backward T={T} H={H} E={E} K={K} norm={norm} {x_dtype}")
    ops = _ops()
    g = gen(4)
    x = torch.randn(T, H, generator=g).to(x_dtype)
    W = _router_weight(torch.randn(E, H, generator=g) * 0.05, x_dtype)
    logits, tw, ti, tw32, *_ = ops.router_forward(x.to(DEV), W.to(DEV), K, norm)
    gw = torch.randn(T, K, generator=g).to(x_dtype)
    gl = torch.randn(T, E, generator=g) * 0.1
    gx, gW = ops.router_backward(x.to(DEV), W.to(DEV), logits, ti, tw32, gw.to(DEV), gl.to(DEV), norm)
    assert gx.dtype == x_dtype and gW.dtype == W.dtype
    dl = O.router_backward_closed_form(logits.cpu(), ti.cpu(), gw.double(), norm, grad_logits=gl)
    ref_gx = (dl.to(DEV) @ W.double().to(DEV)).cpu()
    ref_gW = (dl.to(DEV).t() @ x.double().to(DEV)).cpu()
    check_close("dx", gx, ref_gx, {torch.bfloat16: 1e-2, torch.float16: 1e-3}.get(x_dtype, 1e-5),
                MAX_ABS_FRAC[x_dtype])
    if x_dtype == torch.float16:
        check_close("dW", gW, ref_gW, 1e-3, MAX_ABS_FRAC[x_dtype])
        # Both gradients are formed far more exactly than fp16 holds them, so
        # they are the fp16 roundings of the exact values except where an exact
        # value lies within the residual error of a rounding boundary. dx's bf16
        # pieces leave dl exact to 2^-17, dW's fp16 pieces to 2^-22; dropping
        # either low piece (2^-9 or 2^-12) moves most elements by an ulp.
        for name, got, ref, bound in (("dx", gx, ref_gx, 0.08), ("dW", gW, ref_gW, 0.01)):
            miss = (got.cpu() != ref.half()).double().mean().item()
            say(f"  {name}: {miss:.4f} of the fp16 elements differ from the exact value's rounding")
            assert miss < bound, (name, miss)
    else:
        check_close("dW", gW, ref_gW, 1e-5, 5e-5)


def test_router_weight_pieces():
    """pmoe_router_split_weight writes [lo; hi; mid; hi] with hi = bf16(W),
    mid = bf16(W - hi), lo = bf16(W - hi - mid) (both residuals exact in fp32)
    and hi + mid + lo = W to 2^-24; the router forward and backward given
    these pieces (PMOE_BF16X3) equal, bit for bit, the calls that split the
    fp32 weight themselves, and the backward refuses pieces for E not a
    multiple of 8."""
    ops = _ops()
    T, H, E, K = 3000, 512, 64, 6
    say(f"router weight pieces T={T} H={H} E={E} K={K}")
    g = gen(8)
    W = torch.randn(E, H, generator=g) * 0.05
    # zeros, a tiny value and values that need all three pieces
    W[0, :5] = torch.tensor([0.0, -0.0, 1e-30, 1.0 + 2.0 ** -8 + 2.0 ** -16 + 2.0 ** -23, -(1.0 + 2.0 ** -23)])
    Wd = W.to(DEV)
    pieces = ops.split_router_weight(Wd)
    assert pieces.shape == (4 * E, H) and pieces.dtype == torch.bfloat16
    lo, hi, mid, hi2 = pieces.view(4, E, H).cpu()
    assert torch.equal(hi, hi2) and torch.equal(hi, W.bfloat16())
    r1 = W - hi.float()
    assert torch.equal(mid, r1.bfloat16()) and torch.equal(lo, (r1 - mid.float()).bfloat16())
    err = (hi.double() + mid.double() + lo.double() - W.double()).abs()
    assert bool((err <= W.double().abs() * 2.0 ** -24).all())
    assert float(mid[0, 3]) != 0.0 and float(lo[0, 3]) != 0.0  # the special value uses every piece
    x = torch.randn(T, H, generator=g).bfloat16().to(DEV)
    a = ops.router_forward(x, Wd, K, True)
    b = ops.router_forward(x, Wd, K, True, pieces=pieces)
    assert all(torch.equal(u, v) for u, v in zip(a, b))
    logits, tw, ti, tw32 = a[:4]
    gw = torch.randn(T, K, generator=g).bfloat16().to(DEV)
    gl = (torch.randn(T, E, generator=g) * 0.1).to(DEV)
    gx0, gW0 = ops.router_backward(x, Wd, logits, ti, tw32, gw, gl, True)
    gx1, gW1 = ops.router_backward(x, Wd, logits, ti, tw32, gw, gl, True, pieces=pieces)
    assert gW1.dtype == torch.float32 and torch.equal(gx0, gx1) and torch.equal(gW0, gW1)
    W60 = Wd[:60].contiguous()
    p60 = ops.split_router_weight(W60)
    lg, _, ti60, tw60 = ops.router_forward(x, W60, K, True, pieces=p60)[:4]
    with pytest.raises(RuntimeError, match="multiple of 8"):
        ops.router_backward(x, W60, lg, ti60, tw60, gw, None, True, pieces=p60)


# ------------------------------------------------- fused C entry points


@pytest.mark.parametrize("dtype", DTYPES)
def test_fused_expert_ffn_entry_points(dtype):
    """pmoe_expert_ffn_forward/backward (the whole-operator C ABI) == the per-stage path, bitwise."""
    from pluggy_amd._lib import call, dtype_code, ptr, size, workspace

    import pluggy_amd
    T, K, E, H, I = 300, 4, 16, 256, 64
    say(f"fused entry points T={T} K={K} E={E} H={H} I={I} {dtype}")
    g = gen(31)
    x = torch.randn(T, H, generator=g).to(dtype).to(DEV)
    idx = routing(T, K, E, seed=5, mode="zipf").to(DEV)
    w = torch.rand(T, K, generator=g).to(dtype).to(DEV)
    wgu = (torch.randn(E, 2 * I, H, generator=g) * 0.05).to(dtype).to(DEV)
    wdn = (torch.randn(E, H, I, generator=g) * 0.05).to(dtype).to(DEV)
    gout = torch.randn(T, H, generator=g).to(dtype).to(DEV)
    # stage path through autograd
    xs = x.clone().requires_grad_(True)
    ws_ = w.clone().requires_grad_(True)
    a = wgu.clone().requires_grad_(True)
    b = wdn.clone().requires_grad_(True)
    out_s = pluggy_amd.moe_expert_ffn(xs, idx, ws_, a, b)
    out_s.backward(gout)
    # fused entry points
    P = T * K
    dt = dtype_code(dtype)
    out = torch.empty(T, H, dtype=dtype, device=DEV)
    counts = torch.empty(E, dtype=torch.int32, device=DEV)
    offs = torch.empty(E, dtype=torch.int32, device=DEV)
    sp = torch.empty(P, dtype=torch.int32, device=DEV)
    inv = torch.empty(P, dtype=torch.int32, device=DEV)
    stok = torch.empty(P, dtype=torch.int32, device=DEV)
    sw = torch.empty(P, dtype=torch.float32, device=DEV)
    gu = torch.empty(P, 2 * I, dtype=dtype, device=DEV)
    mid = torch.empty(P, I, dtype=dtype, device=DEV)
    y = torch.empty(P, H, dtype=dtype, device=DEV)
    wsp = workspace(size("pmoe_expert_ffn_forward_workspace_size", T, K, E), DEV)
    stream = torch.cuda.current_stream().cuda_stream
    call("pmoe_expert_ffn_forward", ptr(x), ptr(idx), ptr(w), dt, ptr(wgu), ptr(wdn), dt, T, K, E, H, I, ptr(out),
         ptr(counts), ptr(offs), ptr(sp), ptr(inv), ptr(stok), ptr(sw), ptr(gu), ptr(mid), ptr(y), ptr(wsp),
         wsp.numel(), stream)
    gx = torch.empty_like(x)
    gw = torch.empty_like(w)
    ggu = torch.empty_like(wgu)
    gdn = torch.empty_like(wdn)
    wsb = workspace(size("pmoe_expert_ffn_backward_workspace_size", T, K, H, I, dt), DEV)
    call("pmoe_expert_ffn_backward", ptr(gout), ptr(x), dt, ptr(wgu), ptr(wdn), dt, T, K, E, H, I, ptr(offs),
         ptr(inv), ptr(stok), ptr(sw), ptr(gu), ptr(mid), ptr(gx), ptr(gw), ptr(ggu), ptr(gdn), dt, ptr(wsb),
         wsb.numel(), stream)
    torch.cuda.synchronize()
    assert torch.equal(out, out_s)
    assert torch.equal(gx, xs.grad) and torch.equal(gw, ws_.grad)
    assert torch.equal(ggu, a.grad) and torch.equal(gdn, b.grad)
    if dtype != torch.float32:
        # weight gradients of fp32 masters: the unrounded accumulators of the same tiles
        ggu32 = torch.empty(wgu.shape, dtype=torch.float32, device=DEV)
        gdn32 = torch.empty(wdn.shape, dtype=torch.float32, device=DEV)
        call("pmoe_expert_ffn_backward", ptr(gout), ptr(x), dt, ptr(wgu), ptr(wdn), dt, T, K, E, H, I, ptr(offs),
             ptr(inv), ptr(stok), ptr(sw), ptr(gu), ptr(mid), None, None, ptr(ggu32), ptr(gdn32),
             dtype_code(torch.float32), ptr(wsb), wsb.numel(), stream)
        torch.cuda.synchronize()
        assert torch.equal(ggu32.to(dtype), ggu) and torch.equal(gdn32.to(dtype), gdn)


def test_argument_errors_raise():
    """Rejected arguments come back as RuntimeError with the library's message (no kernel launched)."""
    ops = _ops()
    idx = torch.zeros(4, 3, dtype=torch.int64, device=DEV)
    with pytest.raises(RuntimeError, match="exceeds num_experts"):
        ops.permute(idx, 2)
    x = torch.zeros(4, 12, dtype=torch.bfloat16, device=DEV)  # H not a multiple of 8
    with pytest.raises(RuntimeError, match="multiple of 8"):
        ops.router_forward(x, torch.zeros(4, 12, device=DEV), 2)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        import pluggy_amd
        pluggy_amd.moe_expert_ffn(torch.zeros(4, 8), torch.zeros(4, 1, dtype=torch.int64), torch.ones(4, 1),
                                  torch.zeros(2, 16, 8), torch.zeros(2, 8, 8))


@pytest.mark.parametrize("n,E", [(0, 4), (1, 1), (4096, 128), (100000, 33)])
def test_count_invalid_ids(n, E):
    """The id check counts exactly the ids outside [0, E) (negative and >= E)."""
    g = gen(n + E)
    ids = torch.randint(-3, E + 3, (n,), generator=g, dtype=torch.int64)
    got = int(_ops().count_invalid_ids(ids.reshape(-1, 1).to(DEV), E).item())
    assert got == int(((ids < 0) | (ids >= E)).sum())


@pytest.mark.parametrize("bad", [-1, 8, 1 << 40])
def test_moe_expert_ffn_rejects_out_of_range_ids(bad):
    """moe_expert_ffn raises on an id outside [0, E), as the reference's F.one_hot /
    bincount do (moe.py:50, :107), instead of routing the pair to a clamped expert."""
    import pluggy_amd
    T, H, I, E, K = 16, 64, 32, 8, 2
    idx = torch.stack([torch.arange(T) % E, (torch.arange(T) + 1) % E], 1)
    idx[5, 1] = bad
    w = torch.full((T, K), 0.5)
    args = (torch.randn(T, H).to(DEV), idx.to(DEV), w.to(DEV), torch.randn(E, 2 * I, H).to(DEV) * 0.02,
            torch.randn(E, H, I).to(DEV) * 0.02)
    with pytest.raises(RuntimeError, match="outside"):
        pluggy_amd.moe_expert_ffn(*args)
    idx[5, 1] = 3
    out = pluggy_amd.moe_expert_ffn(args[0], idx.to(DEV), *args[2:])
    assert torch.isfinite(out).all()
