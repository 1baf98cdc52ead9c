"""Operator level of the MoE block: router and dropless expert FFN on HIP.

Mirrors the reference operator surface:

* ``moe_expert_ffn`` replaces ``pluggy.kernels.moe.moe_expert_ffn``
  (pluggy/kernels/moe.py:127-168): same arguments, same shapes, same errors
  (AssertionError on rank/shape), a freshly allocated output, inputs never
  mutated. It always runs the HIP grouped path; ``use_grouped_mm`` is accepted
  for signature compatibility.
* ``router_topk`` is the arithmetic of ``Qwen3MoeTopKRouter.forward``
  (pluggy/models/qwen3_moe/qwen3_moe.py:168-178) with fp32 logits and the
  "ties -> lower expert id" selection rule.

Each entry point is a ``torch.library`` custom op (namespace ``pmoe``) with a
shape-only fake implementation and a registered autograd formula, so a block
that calls them traces under ``torch.compile`` without graph breaks, as the
reference's per-block ``torch.compile`` expects (pluggy/training/trainer.py:
292-293). Each stage (router, permutation, row gather, each grouped GEMM,
combine, and their backward) is one C-ABI call on the current stream;
``stage_timer()`` brackets the stages with HIP events.
"""

from __future__ import annotations

import contextlib
import weakref
from collections import defaultdict
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import ops
from ._lib import require_gpu


@dataclass
class RouterStats:
    """Additive per-layer routing statistics emitted by the fused router."""

    expert_counts: torch.Tensor   # (E,) int32: picks per expert over all slots
    prob_sum: torch.Tensor        # (E,) fp32: sum over tokens of softmax(logits)
    lse_sq_sum: torch.Tensor      # (1,) fp32: sum over tokens of logsumexp(logits)^2
    tokens: int


# ------------------------------------------------------------ stage timing


class StageTimer:
    """HIP-event timing of each named stage on the stream it runs on."""

    def __init__(self):
        self.records: dict[str, list] = defaultdict(list)

    @contextlib.contextmanager
    def mark(self, name: str):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        try:
            yield
        finally:
            end.record()
            self.records[name].append((start, end))

    def summary(self) -> dict[str, dict[str, float]]:
        """name -> {"calls", "total_ms", "mean_ms"} (synchronises)."""
        torch.cuda.synchronize()
        out = {}
        for name, evs in self.records.items():
            ms = [s.elapsed_time(e) for s, e in evs]
            out[name] = {"calls": len(ms), "total_ms": sum(ms), "mean_ms": sum(ms) / len(ms)}
        return out


_timer: StageTimer | None = None


@contextlib.contextmanager
def stage_timer():
    """Collect per-stage HIP-event timings of every MoE call made inside the block."""
    global _timer
    prev, _timer = _timer, StageTimer()
    try:
        yield _timer
    finally:
        _timer = prev


def _stage(name: str):
    return _timer.mark(name) if _timer is not None else contextlib.nullcontext()


def _refuse_capture(op: str) -> None:
    """The backward ops refuse to run while the current stream is capturing a
    HIP graph, before any C-ABI call. The forward captures and replays bitwise
    equal to eager (its entry points allocate nothing, never synchronise and
    clear no memory with hipMemsetAsync); the backward is not claimed under
    capture: the one trial capture of it (torch.cuda.make_graphed_callables on
    the block) ended in a host segmentation fault whose cause is not known."""
    if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
        raise RuntimeError(f"pmoe::{op}: the MoE backward is not supported under HIP graph capture "
                           "(capture the forward only)")


# ---------------------------------------------------------------- autocast


def _amp_dtype(t: torch.Tensor) -> torch.dtype | None:
    """The operand dtype for the kernels under CUDA autocast, or None when it is off.

    The reference trainer runs the model under ``torch.autocast(cuda, bf16)``
    with fp32 parameters (pluggy/training/trainer.py:469). There the router's
    linear runs in bf16 (qwen3_moe.py:172), and the expert weights are cast to
    the activation dtype with the stated intent "bf16 under autocast"
    (moe.py:110-112). The drop-in therefore hands the kernels bf16 operands
    whenever bf16 autocast is on, whatever the residual stream's dtype, and
    returns its outputs in the input's dtype as the reference does. (torch's
    ``F.grouped_mm`` is not on autocast's bf16 list, so with an fp32 residual
    stream the reference's expert GEMMs actually run in fp32; this build keeps
    the stated bf16 intent.) Under fp16 autocast the expert path and the
    router take fp16 operands likewise (fp16 MFMAs, fp32 accumulation; see
    ``_router_x``, ``_router_operand``). Any other autocast dtype gives fp32
    operands.
    """
    if t.is_cuda and torch.is_autocast_enabled("cuda"):
        dt = torch.get_autocast_dtype("cuda")
        return dt if dt in (torch.bfloat16, torch.float16) else torch.float32
    return None


def _compute_dtype(t: torch.Tensor) -> torch.dtype:
    """The dtype the expert kernels compute in for activations ``t``:
    autocast's (see ``_amp_dtype``), else ``t``'s own when it is bf16, fp16 or
    fp32, else fp32 (e.g. an fp64 tensor, computed in fp32 and cast back).
    bf16 and fp16 run on the 16-bit MFMAs with fp32 accumulation, as the
    reference's ``F.grouped_mm`` runs them (moe.py:113-119)."""
    amp = _amp_dtype(t)
    if amp is not None:
        return amp
    return t.dtype if t.dtype in (torch.bfloat16, torch.float16, torch.float32) else torch.float32


def _router_x(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """The router's input as its kernels take it beside the weight operand
    ``w`` (from ``_router_operand``): fp32 or bf16 as given, fp16 when the
    weight is fp16 too (the fp16 MFMAs, as the reference's ``F.linear`` on
    fp16 tensors), else an fp16 input in fp32 (exact). The logits are fp32
    arithmetic in every case."""
    return x.float() if x.dtype == torch.float16 and w.dtype != torch.float16 else x


def _router_operand(w: torch.Tensor, amp: torch.dtype | None, x_dtype: torch.dtype) -> torch.Tensor:
    """The router weight as the kernels take it beside activations of
    ``x_dtype``: bf16 under bf16 autocast and fp16 under fp16 autocast (as the
    reference's ``F.linear`` there), else fp32, bf16 or fp16 as given, except
    that an fp16 weight beside non-fp16 activations (a pairing the kernels do
    not take) and any other dtype are taken in fp32 (exact)."""
    if amp == torch.bfloat16:
        w = w.to(torch.bfloat16)
    elif amp == torch.float16:
        w = w.to(torch.float16)
    elif w.dtype == torch.float16 and x_dtype != torch.float16:
        w = w.float()
    elif w.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        w = w.float()
    return w.contiguous()


# Hidden and intermediate sizes reach the kernels as multiples of 8 (16-byte
# rows). Other sizes are zero-padded on the way in and sliced on the way out:
# the zero columns add nothing to any product, the SwiGLU of a zero gate and
# up column is zero, and autograd carries the gradients back through the pad.
def _pad8(n: int) -> int:
    return (n + 7) // 8 * 8


def _pad_last(t: torch.Tensor, n: int) -> torch.Tensor:
    return t if t.shape[-1] == n else F.pad(t, (0, n - t.shape[-1]))


def _pad_experts(gate_up_proj: torch.Tensor, down_proj: torch.Tensor, Hp: int, Ip: int):
    """(E, 2I, H), (E, H, I) -> (E, 2Ip, Hp), (E, Hp, Ip), gate rows [0, I) then up rows at [Ip, Ip + I)."""
    E, I2, H = gate_up_proj.shape
    I = I2 // 2
    gate, up = gate_up_proj[:, :I], gate_up_proj[:, I:]
    gate = F.pad(gate, (0, Hp - H, 0, Ip - I))
    up = F.pad(up, (0, Hp - H, 0, Ip - I))
    return torch.cat([gate, up], dim=1), F.pad(down_proj, (0, Ip - I, 0, Hp - H))


# 16-bit copies of fp32 master weights kept across calls (see weight_cast_cache):
# (id(master), tag) -> (weakref to the master, (version, data_ptr, shape, stride), copy);
# the tag is the copy's dtype, or "router_pieces" for a router weight's bf16 pieces
_cast_cache: dict[int, tuple] = {}
_cast_cache_on = False


@contextlib.contextmanager
def weight_cast_cache(enabled: bool = True):
    """Reuse the bf16 (or fp16) copies of fp32 master expert weights across calls.

    Under bf16 autocast the kernels take bf16 copies of fp32 master weights,
    as the reference casts them on every call (moe.py:110-112); its trainer
    runs several micro-batches per optimizer step (trainer.py:466-486), each
    casting again (2.4 GB read, 1.2 GB written per layer at the
    Qwen3-30B-A3B shape). Inside this context a master's copy is made once
    and reused while the master is unchanged: while its version counter,
    storage and layout are those of the cached copy. Optimizer steps,
    ``load_state_dict`` and in-place writes under ``torch.no_grad()`` bump the
    version and so recast. Writes through ``.data`` do not bump it and are not
    seen: inside the context, change masters through the tensor itself (or
    leave the context). The copies stay alive as long as their masters (half
    the masters' bytes). Eager mode only: under ``torch.compile`` every call
    casts, as without the context. The bf16 pieces of an fp32 router weight
    beside bf16 activations (``_router_pieces``) are kept the same way.
    """
    global _cast_cache_on
    prev, _cast_cache_on = _cast_cache_on, bool(enabled)
    try:
        yield
    finally:
        _cast_cache_on = prev
        if not _cast_cache_on:
            _cast_cache.clear()


def _cached(w: torch.Tensor, tag, make) -> torch.Tensor:
    """``make(w)`` (a tensor derived from ``w``), kept under ``(id(w), tag)``
    while ``w`` is unchanged (version counter, storage and layout)."""
    key = (id(w), tag)
    state = (w._version, w.data_ptr(), tuple(w.shape), tuple(w.stride()))
    hit = _cast_cache.get(key)
    if hit is not None and hit[0]() is w and hit[1] == state:
        return hit[2]
    with torch.no_grad():
        val = make(w.detach())
    _cast_cache[key] = (weakref.ref(w, lambda _r, k=key: _cast_cache.pop(k, None)), state, val)
    return val


def _cached_copy(w: torch.Tensor, dt: torch.dtype) -> torch.Tensor:
    return _cached(w, dt, lambda t: t.to(dt).contiguous())


def _router_pieces(x_dtype: torch.dtype, rw: torch.Tensor, source: torch.Tensor | None = None):
    """The bf16 pieces (``ops.split_router_weight``) of the fp32 router weight
    operand ``rw`` beside bf16 activations, the three-piece logits GEMM's
    operand: the forward splits the weight once and its backward reuses the
    pieces instead of splitting it again. Inside ``weight_cast_cache`` they are
    kept across calls while ``rw`` is unchanged, when ``rw`` is the parameter
    ``source`` itself. None for other pairings, for E not a multiple of 8 and
    under ``torch.compile``; the kernels then split the weight inside each call,
    with the same bits."""
    if (x_dtype != torch.bfloat16 or rw.dtype != torch.float32 or rw.shape[0] % 8 or not rw.is_cuda
            or torch.compiler.is_compiling()):
        return None
    def split(w):
        with _stage("router_split"):
            return ops.split_router_weight(w)

    if _cast_cache_on and source is rw and rw.is_leaf:
        return _cached(rw, "router_pieces", split)
    with torch.no_grad():
        return split(rw.detach().contiguous())


def _compute_weight(w: torch.Tensor, dt: torch.dtype) -> tuple[torch.Tensor, torch.Tensor | None]:
    """-> (the weight in the kernels' dtype, its fp32 master or None).

    An fp32 master weight that feeds 16-bit kernels (autocast training) is
    cast outside autograd and passed to the op beside its bf16 (or fp16) copy.
    The op's backward then writes the master's gradient in fp32 straight from
    the weight-gradient GEMM, with no 16-bit gradient and no cast kernel
    between.
    Inside ``weight_cast_cache`` the copy of a leaf master is reused while
    the master is unchanged. Otherwise the cast, if any, is an ordinary
    differentiable one.
    """
    half = dt in (torch.bfloat16, torch.float16)
    if w.dtype == torch.float32 and half and w.requires_grad and torch.is_grad_enabled():
        if _cast_cache_on and w.is_leaf and not torch.compiler.is_compiling():
            return _cached_copy(w, dt), w
        with torch.no_grad():
            return w.detach().to(dt).contiguous(), w
    return w.to(dtype=dt).contiguous(), None


def _expert_weights(gate_up_proj: torch.Tensor, down_proj: torch.Tensor, dt: torch.dtype, Hp: int, Ip: int):
    """-> gu, gu_master, dn, dn_master: the expert weights in the kernels'
    dtype (``_compute_weight``), zero-padded to the kernels' multiples of 8
    first when needed. The pad happens in the weights' own dtype, so fp32
    masters keep their fp32 weight gradients (autograd slices them back)."""
    if (Hp, Ip) != (gate_up_proj.shape[2], gate_up_proj.shape[1] // 2):
        gate_up_proj, down_proj = _pad_experts(gate_up_proj, down_proj, Hp, Ip)
    gu, gu_master = _compute_weight(gate_up_proj, dt)
    dn, dn_master = _compute_weight(down_proj, dt)
    return gu, gu_master, dn, dn_master


def _needs(ctx, n: int) -> tuple[bool, ...]:
    """ctx.needs_input_grad over all n schema arguments: the dispatcher drops
    trailing arguments left at their defaults (absent masters), and those need
    no gradient."""
    need = tuple(ctx.needs_input_grad)
    return need + (False,) * (n - len(need))


def _f32_wgrads(gate_up_master, down_master) -> list[bool]:
    """Which weight gradients the backward writes in fp32: those of fp32 masters."""
    return [m is not None and m.dtype == torch.float32 for m in (gate_up_master, down_master)]


# ------------------------------------------------------------------ router


def _none_if_empty(t: torch.Tensor) -> torch.Tensor | None:
    """Custom ops cannot return None: an absent gradient travels as the 1-D
    empty stand-in of ``_empty_like_none``. A real gradient of an empty batch,
    e.g. (0, H) for no tokens, keeps its shape and is returned as is."""
    return None if (t.dim() == 1 and t.numel() == 0) else t


def _empty_like_none(ref: torch.Tensor) -> torch.Tensor:
    """The empty stand-in for an absent output (same dtype and device as ref; 1-D,
    which no gradient of these ops can be: every tensor argument with a
    gradient has at least two dimensions or a nonzero size)."""
    return ref.new_empty(0)


@torch.library.custom_op("pmoe::router_fwd", mutates_args=(),
                         schema="(Tensor x, Tensor weight, int top_k, bool norm_topk_prob, Tensor? logit_bias, "
                                "Tensor? pieces=None) -> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)")
def _router_fwd(x, weight, top_k, norm_topk_prob, logit_bias, pieces=None):
    """``pieces``: the fp32 weight's bf16 pieces (``_router_pieces``) or None."""
    with _stage("router_fwd"):
        return ops.router_forward(x, weight, top_k, norm_topk_prob, logit_bias, pieces=pieces)


@_router_fwd.register_fake
def _(x, weight, top_k, norm_topk_prob, logit_bias, pieces=None):
    T, E, K = x.shape[0], weight.shape[0], top_k
    f32 = torch.float32
    return (x.new_empty(T, E, dtype=f32), x.new_empty(T, K), x.new_empty(T, K, dtype=torch.int64),
            x.new_empty(T, K, dtype=f32), x.new_empty(E, dtype=torch.int32), x.new_empty(E, dtype=f32),
            x.new_empty(1, dtype=f32))


@torch.library.custom_op("pmoe::router_bwd", mutates_args=(),
                         schema="(Tensor x, Tensor weight, Tensor logits, Tensor top_i, Tensor top_w32, "
                                "Tensor? grad_top_w, Tensor? grad_logits, bool norm_topk_prob, Tensor? pieces=None) "
                                "-> (Tensor, Tensor)")
def _router_bwd(x, weight, logits, top_i, top_w32, grad_top_w, grad_logits, norm_topk_prob, pieces=None):
    _refuse_capture("router_bwd")
    with _stage("router_bwd"):
        return ops.router_backward(x, weight, logits, top_i, top_w32, grad_top_w, grad_logits, norm_topk_prob,
                                   pieces=pieces)


@_router_bwd.register_fake
def _(x, weight, logits, top_i, top_w32, grad_top_w, grad_logits, norm_topk_prob, pieces=None):
    return torch.empty_like(x), torch.empty_like(weight)


def _router_setup(ctx, inputs, output):
    x, weight, top_k, norm_topk_prob, logit_bias, pieces = inputs
    logits, top_w, top_i, top_w32, counts, psum, lse2 = output
    ctx.save_for_backward(x, weight, logits, top_i, top_w32, pieces)
    ctx.norm_topk_prob = bool(norm_topk_prob)
    ctx.mark_non_differentiable(top_i, top_w32, counts, psum, lse2)
    ctx.set_materialize_grads(False)  # absent gradients stay None (no zero-filled tensors)


def _router_backward(ctx, g_logits, g_w, _gi, _gw32, _gc, _gp, _gl):
    x, weight, logits, top_i, top_w32, pieces = ctx.saved_tensors
    need = ctx.needs_input_grad
    if not (need[0] or need[1]) or (g_logits is None and g_w is None):
        return None, None, None, None, None, None
    if g_logits is not None:
        g_logits = g_logits.float().contiguous()
    if g_w is not None:
        g_w = g_w.contiguous()
    gx, gW = torch.ops.pmoe.router_bwd(x, weight, logits, top_i, top_w32, g_w, g_logits, ctx.norm_topk_prob, pieces)
    return (gx if need[0] else None), (gW if need[1] else None), None, None, None, None


_router_fwd.register_autograd(_router_backward, setup_context=_router_setup)


def router_topk(hidden: torch.Tensor, weight: torch.Tensor, top_k: int, norm_topk_prob: bool = True,
                logit_bias: torch.Tensor | None = None, return_stats: bool = False):
    """Fused router: fp32 logits, softmax, top-k (ties -> lower id), renormalise.

    Returns ``(router_logits (T,E) fp32, top_weights (T,K) hidden.dtype,
    top_indices (T,K) int64)`` and, with ``return_stats``, a ``RouterStats``.
    Gradients flow to ``hidden`` and ``weight`` through both the logits (for
    aux losses) and the top weights. Under CUDA autocast both operands are
    taken in bf16, as the reference's ``F.linear`` takes them there.
    """
    assert hidden.dim() == 2, "router expects (T, H) hidden states"
    assert weight.dim() == 2 and weight.shape[1] == hidden.shape[1]
    assert 1 <= top_k <= weight.shape[0]
    require_gpu(hidden, weight, logit_bias)
    amp = _amp_dtype(hidden)
    H = hidden.shape[1]
    cdt = _compute_dtype(hidden)
    w = _pad_last(_router_operand(weight, amp, cdt), _pad8(H)).contiguous()
    x = _pad_last(_router_x(hidden.to(cdt), w), _pad8(H)).contiguous()
    if logit_bias is not None:
        logit_bias = logit_bias.float().contiguous()
    logits, top_w, top_i, _w32, counts, psum, lse2 = torch.ops.pmoe.router_fwd(
        x, w, int(top_k), bool(norm_topk_prob), logit_bias, _router_pieces(x.dtype, w, weight))
    top_w = top_w.to(hidden.dtype)  # the reference returns them in x.dtype (qwen3_moe.py:177)
    if return_stats:
        return logits, top_w, top_i, RouterStats(counts, psum, lse2, x.shape[0])
    return logits, top_w, top_i


# -------------------------------------------------------------- expert FFN


def _ffn_forward(hidden, top_indices, top_weights, gate_up_proj, down_proj):
    """-> out and what the backward reads: offs, inv_pos, sorted_token, sorted_w, gu, mid.

    The expert-sorted copy of the hidden rows (moe.py:104) is never built: the
    gate_up GEMM gathers row sorted_token[p] of ``hidden`` in its operand loads,
    and its SwiGLU epilogue multiplies the activation by the routing weight
    (moe.py:120), so the down projection's rows come out weighted and the
    combine is a plain sum of each token's K rows."""
    E = gate_up_proj.shape[0]
    K = top_indices.shape[1]
    with _stage("permute"):
        _, offs, _sorted_pair, inv_pos, sorted_token, sorted_w = ops.permute_rows(top_indices, top_weights, E)
    with _stage("gate_up_fwd"):
        gu, mid = ops.gate_up_swiglu(hidden, gate_up_proj, offs, sorted_token, sorted_w)
    with _stage("down_fwd"):
        y = ops.down_proj(mid, down_proj, offs)
    with _stage("combine"):
        out = ops.combine(y, None, inv_pos, K)
    return out, offs, inv_pos, sorted_token, sorted_w, gu, mid


def _ffn_fake_saved(hidden, K, E, I):
    T, H = hidden.shape
    P = T * K
    i32 = torch.int32
    return (hidden.new_empty(E, dtype=i32), hidden.new_empty(P, dtype=i32), hidden.new_empty(P, dtype=i32),
            hidden.new_empty(P, dtype=torch.float32), hidden.new_empty(P, 2 * I), hidden.new_empty(P, I))


# Check caller-supplied expert ids before routing (moe_expert_ffn). The
# reference raises on an id outside [0, E) (F.one_hot at moe.py:50, bincount at
# moe.py:107); the kernels would clamp it into range instead. The check reads
# one int32 back, i.e. it synchronises the host once per call, as the
# reference's own bincount and .tolist() do; set False to skip it.
VALIDATE_EXPERT_IDS = True


def _check_expert_ids(top_indices: torch.Tensor, num_experts: int) -> None:
    bad = int(ops.count_invalid_ids(top_indices, num_experts).item())
    if bad:
        raise RuntimeError(f"moe_expert_ffn: {bad} expert id(s) outside [0, {num_experts})")


@torch.library.custom_op("pmoe::expert_ffn_fwd", mutates_args=(),
                         schema="(Tensor hidden, Tensor top_indices, Tensor top_weights, Tensor gate_up_proj, "
                                "Tensor down_proj, Tensor? gate_up_master=None, Tensor? down_master=None) -> "
                                "(Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)")
def _expert_ffn_fwd(hidden, top_indices, top_weights, gate_up_proj, down_proj, gate_up_master=None,
                    down_master=None):
    """The masters, when given, are the differentiable fp32 weights whose bf16
    copies gate_up_proj / down_proj are; the forward does not read them."""
    if VALIDATE_EXPERT_IDS:
        _check_expert_ids(top_indices, gate_up_proj.shape[0])
    return _ffn_forward(hidden, top_indices, top_weights, gate_up_proj, down_proj)


@_expert_ffn_fwd.register_fake
def _(hidden, top_indices, top_weights, gate_up_proj, down_proj, gate_up_master=None, down_master=None):
    E, I2 = gate_up_proj.shape[0], gate_up_proj.shape[1]
    return (torch.empty_like(hidden),) + _ffn_fake_saved(hidden, top_indices.shape[1], E, I2 // 2)


@torch.library.custom_op("pmoe::expert_bwd_dgrad", mutates_args=(),
                         schema="(Tensor grad_out, Tensor down_proj, Tensor offs, Tensor inv_pos, Tensor sorted_token, "
                                "Tensor sorted_w, Tensor gu, int top_k, bool need_top_w) -> (Tensor, Tensor)")
def _expert_bwd_dgrad(grad_out, down_proj, offs, inv_pos, sorted_token, sorted_w, gu, top_k, need_top_w):
    """The down projection's input gradient through the SwiGLU: -> grad_gate_up_out
    (P, 2I) and, with need_top_w, the routing weights' gradient (T, K) fp32
    (an empty stand-in otherwise). grad_out (T, H) is the layer's output
    gradient; its rows are gathered by sorted_token."""
    _refuse_capture("expert_bwd_dgrad")
    with _stage("down_dgrad"):
        g_gu, part = ops.down_proj_dgrad(grad_out, gu, down_proj, offs, sorted_token, sorted_w,
                                         need_part=need_top_w)
    if not need_top_w:
        return g_gu, _empty_like_none(sorted_w)
    with _stage("pair_wgrad"):
        return g_gu, ops.pair_weight_grad(part, inv_pos, top_k)


@_expert_bwd_dgrad.register_fake
def _(grad_out, down_proj, offs, inv_pos, sorted_token, sorted_w, gu, top_k, need_top_w):
    P = sorted_token.shape[0]
    return (gu.new_empty(P, gu.shape[1]),
            grad_out.new_empty(P // top_k, top_k, dtype=torch.float32) if need_top_w else _empty_like_none(sorted_w))


def _expert_gemms_backward(g_gu, grad_out, hidden, gate_up, down, offs, sorted_token, mid, need_rows, need_gu,
                           need_dn, reduce_rows, f32_wgrads=(False, False)):
    """The expert GEMMs' backward after the down dgrad (g_gu = grad_gate_up_out).
    With need_rows, the (P, H) input gradient of the sorted rows goes to
    ``reduce_rows`` (which sums each token's K rows) before the weight
    gradients are computed, so it is freed early. f32_wgrads (gate_up, down):
    write that weight gradient in fp32.
    -> (reduce_rows result or None, grad_gate_up or None, grad_down or None)."""
    E = gate_up.shape[0]
    f32 = torch.float32
    reduced = g_gu_w = g_dn_w = None
    if need_rows:
        with _stage("gate_up_dgrad"):
            g_xp = ops.gate_up_dgrad(g_gu, gate_up, offs)
        reduced = reduce_rows(g_xp)
        del g_xp
    if need_gu:
        with _stage("gate_up_wgrad"):
            g_gu_w = ops.gate_up_wgrad(g_gu, hidden, offs, E, f32 if f32_wgrads[0] else None, row_index=sorted_token)
    if need_dn:
        with _stage("down_wgrad"):
            g_dn_w = ops.down_proj_wgrad(grad_out, mid, offs, E, f32 if f32_wgrads[1] else None,
                                         row_index=sorted_token)
    return reduced, g_gu_w, g_dn_w


@torch.library.custom_op("pmoe::expert_bwd", mutates_args=(),
                         schema="(Tensor g_gu, Tensor grad_out, Tensor hidden, Tensor gate_up_proj, Tensor down_proj, "
                                "Tensor offs, Tensor inv_pos, Tensor sorted_token, Tensor mid, Tensor? grad_hidden_add, "
                                "int top_k, bool[] needs, bool[] f32_wgrads) -> (Tensor, Tensor, Tensor)")
def _expert_bwd(g_gu, grad_out, hidden, gate_up, down, offs, inv_pos, sorted_token, mid, grad_hidden_add, top_k,
                needs, f32_wgrads):
    """The expert GEMMs' backward after the down dgrad: -> grad_hidden (+
    grad_hidden_add), grad_gate_up, grad_down; an empty tensor where needs[i] is
    false (needs: hidden, gate_up, down). f32_wgrads (gate_up, down): that weight
    gradient is fp32 (an fp32 master's) instead of the operands' dtype."""
    _refuse_capture("expert_bwd")

    def reduce_rows(g_xp):
        with _stage("dispatch_bwd"):
            return ops.dispatch_backward(g_xp, inv_pos, hidden.shape[0], top_k, add=grad_hidden_add)

    g_hidden, g_gu_w, g_dn_w = _expert_gemms_backward(g_gu, grad_out, hidden, gate_up, down, offs, sorted_token, mid,
                                                      needs[0], needs[1], needs[2], reduce_rows, f32_wgrads)
    e = _empty_like_none
    return (g_hidden if g_hidden is not None else e(hidden), g_gu_w if g_gu_w is not None else e(gate_up),
            g_dn_w if g_dn_w is not None else e(down))


def _wgrad_fake(w, f32):
    return torch.empty_like(w, dtype=torch.float32 if f32 else w.dtype)


@_expert_bwd.register_fake
def _(g_gu, grad_out, hidden, gate_up, down, offs, inv_pos, sorted_token, mid, grad_hidden_add, top_k, needs,
      f32_wgrads):
    e = _empty_like_none
    return (torch.empty_like(hidden) if needs[0] else e(hidden),
            _wgrad_fake(gate_up, f32_wgrads[0]) if needs[1] else e(gate_up),
            _wgrad_fake(down, f32_wgrads[1]) if needs[2] else e(down))


def _ffn_setup(ctx, inputs, output):
    hidden, top_indices, top_weights, gate_up_proj, down_proj, gate_up_master, down_master = inputs
    ctx.f32_wgrads = _f32_wgrads(gate_up_master, down_master)
    out, offs, inv_pos, sorted_token, sorted_w, gu, mid = output
    ctx.save_for_backward(hidden, gate_up_proj, down_proj, offs, inv_pos, sorted_token, sorted_w, gu, mid)
    ctx.top_k = top_indices.shape[1]
    ctx.tw_dtype = top_weights.dtype
    ctx.mark_non_differentiable(offs, inv_pos, sorted_token, sorted_w, gu, mid)
    ctx.set_materialize_grads(False)


def _ffn_backward(ctx, grad_out, *_saved_grads):
    if grad_out is None:
        return (None,) * 7
    hidden, gate_up, down, offs, inv_pos, sorted_token, sorted_w, gu, mid = ctx.saved_tensors
    K = ctx.top_k
    need = _needs(ctx, 7)  # hidden, indices, weights, gate_up, down, gate_up_master, down_master
    need_gu, need_dn = need[3] or need[5], need[4] or need[6]
    if not (need[0] or need[2] or need_gu or need_dn):
        return (None,) * 7
    grad_out = grad_out.contiguous()
    if grad_out.dtype != hidden.dtype:
        grad_out = grad_out.to(hidden.dtype)
    g_gu, g_w = torch.ops.pmoe.expert_bwd_dgrad(grad_out, down, offs, inv_pos, sorted_token, sorted_w, gu, K,
                                                bool(need[2]))
    g_hidden = g_gu_w = g_dn_w = None
    if need[0] or need_gu or need_dn:
        g_hidden, g_gu_w, g_dn_w = torch.ops.pmoe.expert_bwd(g_gu, grad_out, hidden, gate_up, down, offs, inv_pos,
                                                             sorted_token, mid, None, K,
                                                             [bool(need[0]), bool(need_gu), bool(need_dn)],
                                                             ctx.f32_wgrads)
        g_hidden, g_gu_w, g_dn_w = (_none_if_empty(t) for t in (g_hidden, g_gu_w, g_dn_w))
    g_w = g_w.to(ctx.tw_dtype) if need[2] else None
    return (g_hidden if need[0] else None, None, g_w, g_gu_w if need[3] else None, g_dn_w if need[4] else None,
            g_gu_w if need[5] else None, g_dn_w if need[6] else None)


_expert_ffn_fwd.register_autograd(_ffn_backward, setup_context=_ffn_setup)


# ------------------------------------------------- whole sparse MLP block


@torch.library.custom_op("pmoe::sparse_moe_fwd", mutates_args=(),
                         schema="(Tensor x, Tensor router_weight, Tensor gate_up_proj, Tensor down_proj, int top_k, "
                                "bool norm_topk_prob, Tensor? logit_bias, Tensor? gate_up_master=None, "
                                "Tensor? down_master=None, Tensor? router_pieces=None) -> (Tensor, Tensor, Tensor, "
                                "Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, "
                                "Tensor)")
def _sparse_moe_fwd(x, router_weight, gate_up_proj, down_proj, top_k, norm_topk_prob, logit_bias,
                    gate_up_master=None, down_master=None, router_pieces=None):
    """Router + dropless experts (Qwen3MoeSparseMLP.forward) as one op.

    -> out, router_logits, counts, prob_sum, lse_sq_sum, then what the backward
    reads: top_i, top_w32, top_w, offs, inv_pos, sorted_token, sorted_w, gu,
    mid. The masters, when given, are the differentiable fp32 weights whose
    bf16 copies gate_up_proj / down_proj are (their gradients are written in
    fp32). router_pieces: the router weight's bf16 pieces (``_router_pieces``),
    reused by the backward, or None.
    """
    with _stage("router_fwd"):
        logits, top_w, top_i, top_w32, counts, psum, lse2 = ops.router_forward(
            _router_x(x, router_weight), router_weight, top_k, norm_topk_prob, logit_bias, tw_dtype=x.dtype,
            pieces=router_pieces)
    out, offs, inv_pos, stok, sw, gu, mid = _ffn_forward(x, top_i, top_w, gate_up_proj, down_proj)
    return out, logits, counts, psum, lse2, top_i, top_w32, top_w, offs, inv_pos, stok, sw, gu, mid


@_sparse_moe_fwd.register_fake
def _(x, router_weight, gate_up_proj, down_proj, top_k, norm_topk_prob, logit_bias, gate_up_master=None,
      down_master=None, router_pieces=None):
    T, E, K = x.shape[0], router_weight.shape[0], top_k
    I = gate_up_proj.shape[1] // 2
    f32 = torch.float32
    return ((torch.empty_like(x), x.new_empty(T, E, dtype=f32), x.new_empty(E, dtype=torch.int32),
             x.new_empty(E, dtype=f32), x.new_empty(1, dtype=f32), x.new_empty(T, K, dtype=torch.int64),
             x.new_empty(T, K, dtype=f32), x.new_empty(T, K))
            + _ffn_fake_saved(x, K, E, I))


def _sparse_setup(ctx, inputs, output):
    (x, router_weight, gate_up_proj, down_proj, top_k, norm_topk_prob, logit_bias, gu_master, dn_master,
     router_pieces) = inputs
    (out, logits, counts, psum, lse2, top_i, top_w32, top_w, offs, inv_pos, stok, sw, gu, mid) = output
    ctx.f32_wgrads = _f32_wgrads(gu_master, dn_master)
    ctx.save_for_backward(x, router_weight, logits, top_i, top_w32, gate_up_proj, down_proj, offs, inv_pos, stok,
                          sw, gu, mid, router_pieces)
    ctx.norm_topk_prob = bool(norm_topk_prob)
    ctx.dims = (x.shape[0], int(top_k))
    ctx.mark_non_differentiable(counts, psum, lse2, top_i, top_w32, top_w, offs, inv_pos, stok, sw, gu, mid)
    ctx.set_materialize_grads(False)


def _sparse_backward(ctx, g_out, g_logits, *_rest):
    """The down dgrad comes first (it yields the routing weights' gradient), then
    the router's backward, whose input gradient is added inside the dispatch
    backward, so the two input gradients are never summed by a separate pass."""
    (x, rw, logits, top_i, top_w32, gate_up, down, offs, inv_pos, stok, sw, gu, mid, pieces) = ctx.saved_tensors
    T, K = ctx.dims
    # x, router_weight, gate_up, down, top_k, norm, bias, gate_up_master, down_master, router_pieces
    need = _needs(ctx, 10)
    need_gu, need_dn = need[2] or need[7], need[3] or need[8]
    if g_out is None and g_logits is None:
        return (None,) * 10
    if g_logits is not None:
        g_logits = g_logits.float().contiguous()
    g_x = g_rw = g_gu_w = g_dn_w = None
    g_gu = g_tw = None
    if g_out is not None:
        g_out = g_out.contiguous()
        if g_out.dtype != gu.dtype:
            g_out = g_out.to(gu.dtype)
        g_gu, g_tw = torch.ops.pmoe.expert_bwd_dgrad(g_out, down, offs, inv_pos, stok, sw, gu, K,
                                                     bool(need[0] or need[1]))
        g_tw = _none_if_empty(g_tw)
    gx_router = None
    if need[0] or need[1]:
        gx_router, g_rw = torch.ops.pmoe.router_bwd(_router_x(x, rw), rw, logits, top_i, top_w32, g_tw, g_logits,
                                                    ctx.norm_topk_prob, pieces)
        gx_router = gx_router.to(x.dtype)  # fp32 when fp16 x met a non-fp16 weight
    if g_gu is not None and (need[0] or need_gu or need_dn):
        g_hidden, g_gu_w, g_dn_w = torch.ops.pmoe.expert_bwd(
            g_gu, g_out, x, gate_up, down, offs, inv_pos, stok, mid, gx_router if need[0] else None, K,
            [bool(need[0]), bool(need_gu), bool(need_dn)], ctx.f32_wgrads)
        g_x = _none_if_empty(g_hidden)
        g_gu_w = _none_if_empty(g_gu_w)
        g_dn_w = _none_if_empty(g_dn_w)
    elif need[0]:
        g_x = gx_router
    return ((g_x if need[0] else None), (g_rw if need[1] else None), g_gu_w if need[2] else None,
            g_dn_w if need[3] else None, None, None, None, g_gu_w if need[7] else None, g_dn_w if need[8] else None,
            None)


_sparse_moe_fwd.register_autograd(_sparse_backward, setup_context=_sparse_setup)


def sparse_moe_block(hidden: torch.Tensor, router_weight: torch.Tensor, gate_up_proj: torch.Tensor,
                     down_proj: torch.Tensor, top_k: int, norm_topk_prob: bool = True,
                     logit_bias: torch.Tensor | None = None):
    """Router + experts of ``Qwen3MoeSparseMLP.forward`` (qwen3_moe.py:233-239) on HIP.

    ``hidden`` (T, H). Returns ``(out (T,H), router_logits (T,E) fp32,
    RouterStats)``; the logits carry the gradient of any aux loss. Same
    arithmetic as ``router_topk`` followed by ``moe_expert_ffn``, including
    their bf16 operands under CUDA autocast (``out`` keeps ``hidden.dtype``).
    """
    assert hidden.dim() == 2 and router_weight.dim() == 2 and router_weight.shape[1] == hidden.shape[1]
    assert gate_up_proj.dim() == 3 and down_proj.dim() == 3
    assert 1 <= top_k <= router_weight.shape[0]
    require_gpu(hidden, router_weight, gate_up_proj, down_proj, logit_bias)
    amp = _amp_dtype(hidden)
    dt = _compute_dtype(hidden)
    T, H = hidden.shape
    I = gate_up_proj.shape[1] // 2
    Hp, Ip = _pad8(H), _pad8(I)
    x = _pad_last(hidden.to(dt), Hp).contiguous()
    rw = _pad_last(_router_operand(router_weight, amp, dt), Hp).contiguous()
    gu, gu_master, dn, dn_master = _expert_weights(gate_up_proj, down_proj, dt, Hp, Ip)
    if logit_bias is not None:
        logit_bias = logit_bias.float().contiguous()
    pieces = _router_pieces(dt, rw, router_weight)
    out, logits, counts, psum, lse2 = torch.ops.pmoe.sparse_moe_fwd(x, rw, gu, dn, int(top_k), bool(norm_topk_prob),
                                                                     logit_bias, gu_master, dn_master, pieces)[:5]
    return out[:, :H].to(hidden.dtype), logits, RouterStats(counts, psum, lse2, T)


def moe_expert_ffn(
    hidden: torch.Tensor,        # (T, H)
    top_indices: torch.Tensor,   # (T, K) int64
    top_weights: torch.Tensor,   # (T, K)
    gate_up_proj: torch.Tensor,  # (E, 2I, H)
    down_proj: torch.Tensor,     # (E, H, I)
    *,
    use_grouped_mm: bool | None = None,
) -> torch.Tensor:
    """Dropless top-k expert FFN on MI355X (drop-in for moe.py:127-168).

    ``out[t] = sum_k w[t,k] * down[e](silu(gate[e] x_t) * up[e] x_t)`` with
    e = top_indices[t,k]. Weights are cast to ``hidden.dtype`` first, as the
    reference does (moe.py:110-112), and to bf16 under CUDA autocast, with the
    output in ``hidden.dtype``. The permutation, both grouped GEMMs and the
    fp32-accumulating combine run as HIP kernels; there is no CPU path.
    """
    assert hidden.dim() == 2
    assert top_indices.shape == top_weights.shape
    assert top_indices.shape[0] == hidden.shape[0]
    assert gate_up_proj.dim() == 3 and down_proj.dim() == 3
    del use_grouped_mm  # one code path: the HIP grouped kernels
    require_gpu(hidden, top_indices, top_weights, gate_up_proj, down_proj)
    dt = _compute_dtype(hidden)
    H = hidden.shape[1]
    I = gate_up_proj.shape[1] // 2
    Hp, Ip = _pad8(H), _pad8(I)
    gu, gu_master, dn, dn_master = _expert_weights(gate_up_proj, down_proj, dt, Hp, Ip)
    tw = top_weights if top_weights.dtype in (torch.float32, torch.bfloat16, torch.float16) else top_weights.float()
    out = torch.ops.pmoe.expert_ffn_fwd(_pad_last(hidden.to(dt), Hp).contiguous(),
                                        top_indices.to(torch.int64).contiguous(), tw.contiguous(), gu, dn,
                                        gu_master, dn_master)[0]
    return out[:, :H].to(hidden.dtype)


# ------------------------------- MoE half of the block: RMSNorm -> MLP -> add


@torch.library.custom_op("pmoe::moe_sublayer_fwd", mutates_args=(),
                         schema="(Tensor x, Tensor norm_weight, float eps, Tensor router_weight, Tensor gate_up_proj, "
                                "Tensor down_proj, int top_k, bool norm_topk_prob, Tensor? logit_bias, "
                                "Tensor? gate_up_master=None, Tensor? down_master=None, Tensor? router_pieces=None) "
                                "-> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, "
                                "Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)")
def _moe_sublayer_fwd(x, norm_weight, eps, router_weight, gate_up_proj, down_proj, top_k, norm_topk_prob,
                      logit_bias, gate_up_master=None, down_master=None, router_pieces=None):
    """x + SparseMLP(RMSNorm(x)) with the norm and the residual add in the row kernels.

    The kernels compute in gate_up_proj's dtype; x is the residual stream (its
    own dtype). -> out, router_logits, counts, prob_sum, lse_sq_sum, then what
    the backward reads: normed, rstd, top_i, top_w32, top_w, offs, inv_pos,
    sorted_token, sorted_w, gu, mid. The masters, when given, are the
    differentiable fp32 weights whose bf16 copies gate_up_proj / down_proj are;
    router_pieces, the router weight's bf16 pieces (``_router_pieces``) or None.
    """
    with _stage("rmsnorm"):
        normed, rstd = ops.rmsnorm_forward(x, norm_weight, eps, gate_up_proj.dtype)
    with _stage("router_fwd"):
        logits, top_w, top_i, top_w32, counts, psum, lse2 = ops.router_forward(
            normed, router_weight, top_k, norm_topk_prob, logit_bias, pieces=router_pieces)
    with _stage("permute"):
        _, offs, _sorted_pair, inv_pos, stok, sw = ops.permute_rows(top_i, top_w, gate_up_proj.shape[0])
    with _stage("gate_up_fwd"):
        gu, mid = ops.gate_up_swiglu(normed, gate_up_proj, offs, stok, sw)
    with _stage("down_fwd"):
        y = ops.down_proj(mid, down_proj, offs)
    with _stage("combine"):
        out = ops.combine_residual(y, None, inv_pos, x, top_k)
    return out, logits, counts, psum, lse2, normed, rstd, top_i, top_w32, top_w, offs, inv_pos, stok, sw, gu, mid


@_moe_sublayer_fwd.register_fake
def _(x, norm_weight, eps, router_weight, gate_up_proj, down_proj, top_k, norm_topk_prob, logit_bias,
      gate_up_master=None, down_master=None, router_pieces=None):
    T, H = x.shape
    E, K, I = router_weight.shape[0], top_k, gate_up_proj.shape[1] // 2
    cdt = gate_up_proj.dtype
    f32, i32 = torch.float32, torch.int32
    P = T * K
    return (torch.empty_like(x), x.new_empty(T, E, dtype=f32), x.new_empty(E, dtype=i32), x.new_empty(E, dtype=f32),
            x.new_empty(1, dtype=f32), x.new_empty(T, H, dtype=cdt), x.new_empty(T, dtype=f32),
            x.new_empty(T, K, dtype=torch.int64), x.new_empty(T, K, dtype=f32), x.new_empty(T, K, dtype=cdt),
            x.new_empty(E, dtype=i32), x.new_empty(P, dtype=i32), x.new_empty(P, dtype=i32),
            x.new_empty(P, dtype=f32), x.new_empty(P, 2 * I, dtype=cdt), x.new_empty(P, I, dtype=cdt))


@torch.library.custom_op("pmoe::sublayer_bwd", mutates_args=(),
                         schema="(Tensor? g_gu, Tensor? grad_out_c, Tensor normed, Tensor gate_up_proj, "
                                "Tensor down_proj, Tensor offs, Tensor inv_pos, Tensor sorted_token, Tensor mid, "
                                "Tensor? grad_normed_add, Tensor x, Tensor norm_weight, Tensor rstd, "
                                "Tensor? grad_residual, int top_k, bool[] needs, bool[] f32_wgrads) -> "
                                "(Tensor, Tensor, Tensor, Tensor)")
def _sublayer_bwd(g_gu, grad_out_c, normed, gate_up, down, offs, inv_pos, sorted_token, mid, grad_normed_add, x,
                  norm_weight, rstd, grad_residual, top_k, needs, f32_wgrads):
    """Expert GEMM backward after the down dgrad, then the dispatch, RMSNorm and
    residual backward in one row pass: -> grad_x, grad_norm_weight,
    grad_gate_up, grad_down (empty where needs[i] is false; needs: x,
    norm_weight, gate_up, down). grad_out_c is the output gradient in the
    compute dtype (the down wgrad gathers its rows). f32_wgrads (gate_up,
    down): that weight gradient is fp32 (an fp32 master's)."""
    _refuse_capture("sublayer_bwd")
    need_x = needs[0] or needs[1]

    def reduce_rows(g_xp):
        with _stage("dispatch_bwd"):
            return ops.dispatch_rmsnorm_backward(g_xp, inv_pos, grad_normed_add, x, norm_weight, rstd, grad_residual,
                                                 top_k, need_weight=needs[1])

    reduced = g_gu_w = g_dn_w = None
    if g_gu is not None:
        reduced, g_gu_w, g_dn_w = _expert_gemms_backward(g_gu, grad_out_c, normed, gate_up, down, offs, sorted_token,
                                                         mid, need_x, needs[2], needs[3], reduce_rows, f32_wgrads)
    elif need_x:
        reduced = reduce_rows(None)
    g_x, g_nw = reduced if reduced is not None else (None, None)
    e = _empty_like_none
    return (g_x if g_x is not None and needs[0] else e(x), g_nw if g_nw is not None else e(norm_weight),
            g_gu_w if g_gu_w is not None else e(gate_up), g_dn_w if g_dn_w is not None else e(down))


@_sublayer_bwd.register_fake
def _(g_gu, grad_out_c, normed, gate_up, down, offs, inv_pos, sorted_token, mid, grad_normed_add, x, norm_weight,
      rstd, grad_residual, top_k, needs, f32_wgrads):
    e = _empty_like_none
    return (torch.empty_like(x) if needs[0] else e(x), torch.empty_like(norm_weight) if needs[1] else e(norm_weight),
            _wgrad_fake(gate_up, f32_wgrads[0]) if needs[2] else e(gate_up),
            _wgrad_fake(down, f32_wgrads[1]) if needs[3] else e(down))


def _sublayer_setup(ctx, inputs, output):
    (x, norm_weight, eps, router_weight, gate_up_proj, down_proj, top_k, norm_topk_prob, logit_bias, gu_master,
     dn_master, router_pieces) = inputs
    ctx.f32_wgrads = _f32_wgrads(gu_master, dn_master)
    (out, logits, counts, psum, lse2, normed, rstd, top_i, top_w32, top_w, offs, inv_pos, stok, sw, gu,
     mid) = output
    ctx.save_for_backward(x, norm_weight, rstd, normed, router_weight, logits, top_i, top_w32, gate_up_proj,
                          down_proj, offs, inv_pos, stok, sw, gu, mid, router_pieces)
    ctx.norm_topk_prob = bool(norm_topk_prob)
    ctx.top_k = int(top_k)
    ctx.mark_non_differentiable(counts, psum, lse2, normed, rstd, top_i, top_w32, top_w, offs, inv_pos, stok, sw, gu,
                                mid)
    ctx.set_materialize_grads(False)


def _sublayer_backward(ctx, g_out, g_logits, *_rest):
    """d out / d x is the identity (the residual) plus the norm-and-MLP path;
    the residual term, the router's share and the K expert rows are all summed
    inside the one row pass of the dispatch backward."""
    (x, nw, rstd, normed, rw, logits, top_i, top_w32, gate_up, down, offs, inv_pos, stok, sw, gu,
     mid, pieces) = ctx.saved_tensors
    # x, norm_weight, eps, router_weight, gate_up, down, top_k, norm, bias, gate_up_master, down_master,
    # router_pieces
    need = _needs(ctx, 12)
    need_gu, need_dn = need[4] or need[9], need[5] or need[10]
    nones = (None,) * 12
    if g_out is None and g_logits is None:
        return nones
    if g_logits is not None:
        g_logits = g_logits.float().contiguous()
    g_gu = g_tw = g_out_c = None
    if g_out is not None:
        g_out = g_out.contiguous()
        # the expert GEMMs gather rows of the output gradient in the compute dtype
        g_out_c = g_out if g_out.dtype == gu.dtype else g_out.to(gu.dtype)
        g_gu, g_tw = torch.ops.pmoe.expert_bwd_dgrad(g_out_c, down, offs, inv_pos, stok, sw, gu, ctx.top_k,
                                                     bool(need[0] or need[1] or need[3]))
        g_tw = _none_if_empty(g_tw)
    gx_router = g_rw = None
    if need[0] or need[1] or need[3]:
        gx_router, g_rw = torch.ops.pmoe.router_bwd(normed, rw, logits, top_i, top_w32, g_tw, g_logits,
                                                    ctx.norm_topk_prob, pieces)
    needs = [bool(need[0]), bool(need[1]), bool(need_gu) and g_gu is not None, bool(need_dn) and g_gu is not None]
    g_x = g_nw = g_gu_w = g_dn_w = None
    if any(needs):
        g_x, g_nw, g_gu_w, g_dn_w = torch.ops.pmoe.sublayer_bwd(
            g_gu, g_out_c, normed, gate_up, down, offs, inv_pos, stok, mid,
            gx_router if (need[0] or need[1]) else None, x, nw, rstd, g_out if need[0] else None, ctx.top_k, needs,
            ctx.f32_wgrads)
        g_x, g_nw, g_gu_w, g_dn_w = (_none_if_empty(t) for t in (g_x, g_nw, g_gu_w, g_dn_w))
    return (g_x if need[0] else None, g_nw if need[1] else None, None, g_rw if need[3] else None,
            g_gu_w if need[4] else None, g_dn_w if need[5] else None, None, None, None, g_gu_w if need[9] else None,
            g_dn_w if need[10] else None, None)


_moe_sublayer_fwd.register_autograd(_sublayer_backward, setup_context=_sublayer_setup)


def moe_sublayer(x: torch.Tensor, norm: torch.nn.RMSNorm, mlp) -> torch.Tensor:
    """``x + mlp(norm(x))`` — the MoE half of ``Qwen3MoeTransformerBlock.forward``
    (qwen3_moe.py:281) — with the RMSNorm and the residual add fused into the
    block's row kernels.

    ``norm`` is the block's ``torch.nn.RMSNorm`` (elementwise weight; eps None
    means ``finfo(x.dtype).eps``, as torch), ``mlp`` a
    ``pluggy_amd.Qwen3MoeSparseMLP``, whose ``last_router_logits`` and router
    statistics are set as its own forward sets them. ``x`` (B, S, H) is the
    residual stream (fp32 or bf16); the experts and the router run in bf16
    under CUDA autocast, else in the expert weights' dtype (cast to x's dtype
    first, as ``moe_expert_ffn``). Same value as
    ``x + mlp(norm(x))`` up to the rounding of the normed rows and of the MLP
    output, which this path does not round to the compute dtype before the add.
    """
    B, S, H = x.shape
    require_gpu(x)
    assert isinstance(norm, torch.nn.RMSNorm) and tuple(norm.normalized_shape) == (H,) and norm.weight is not None
    I = mlp.experts.gate_up_proj.shape[1] // 2
    if (H > 16384 or H % 8 or I % 8 or x.dtype not in (torch.float32, torch.bfloat16)
            or _compute_dtype(x) == torch.float16):
        # the fused backward's row kernels take 16-byte rows of an fp32 or bf16
        # stream up to 16384 wide (beyond 4096 the rows are walked twice, with
        # the norm-weight partials in LDS) and bf16 or fp32 expert rows; other
        # shapes and fp16 experts take the unfused path
        return x + mlp(norm(x))
    r = mlp.router
    flat = x.reshape(B * S, H).contiguous()
    amp = _amp_dtype(flat)
    cdt = _compute_dtype(flat)
    eps = norm.eps if norm.eps is not None else torch.finfo(x.dtype).eps
    nw = norm.weight if norm.weight.dtype == torch.float32 else norm.weight.float()
    rw = _router_operand(r.weight, amp, cdt)
    gu, gu_master = _compute_weight(mlp.experts.gate_up_proj, cdt)
    dn, dn_master = _compute_weight(mlp.experts.down_proj, cdt)
    bias = r.logit_bias.float().contiguous() if r.logit_bias is not None else None
    out, logits, counts, psum, lse2 = torch.ops.pmoe.moe_sublayer_fwd(
        flat, nw.contiguous(), float(eps), rw, gu, dn, int(r.top_k), bool(r.norm_topk_prob), bias,
        gu_master, dn_master, _router_pieces(cdt, rw, r.weight))[:5]
    r.last_stats = RouterStats(counts, psum, lse2, flat.shape[0])
    mlp.last_router_logits = logits
    return out.reshape(B, S, H)
