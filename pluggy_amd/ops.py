"""Functional wrappers of each C-ABI entry point (no autograd).

One function per kernel stage of the MoE block, so every stage can be called,
tested and timed on its own. Shapes follow ``include/pmoe.h``; outputs are
freshly allocated on the input's device and stream.
"""

from __future__ import annotations

import torch

from ._lib import PMOE_BF16X3, call, dtype_code, ptr, require_gpu, size, stream_of, workspace


def _dims(gate_up_proj: torch.Tensor):
    E, two_i, H = gate_up_proj.shape
    return E, H, two_i // 2


def split_router_weight(weight):
    """-> the bf16 pieces (4E, H) of an fp32 router weight (E, H), which
    ``router_forward`` / ``router_backward`` take as ``pieces`` beside bf16 x."""
    require_gpu(weight)
    assert weight.dtype == torch.float32 and weight.dim() == 2 and weight.is_contiguous()
    E, H = weight.shape
    pieces = torch.empty(4 * E, H, dtype=torch.bfloat16, device=weight.device)
    call("pmoe_router_split_weight", ptr(weight), E, H, ptr(pieces), stream_of(weight))
    return pieces


def _router_weight_arg(weight, pieces):
    """(pointer, dtype code) of the router weight operand: the pieces of an
    fp32 weight when given, else the weight itself."""
    if pieces is not None:
        assert weight.dtype == torch.float32 and pieces.shape == (4 * weight.shape[0], weight.shape[1])
        return ptr(pieces), PMOE_BF16X3
    return ptr(weight), dtype_code(weight.dtype)


def router_forward(x, weight, top_k: int, norm_topk_prob: bool = True, logit_bias=None, tw_dtype=None,
                   pieces=None):
    """-> logits, top_w (tw_dtype, default x.dtype), top_i (int64), top_w_f32, counts (int32), prob_sum,
    lse_sq_sum. ``pieces``: ``split_router_weight(weight)``, for bf16 x beside an fp32 weight."""
    require_gpu(x, weight, logit_bias)
    T, H = x.shape
    E = weight.shape[0]
    dev = x.device
    tw_dtype = x.dtype if tw_dtype is None else tw_dtype
    logits = torch.empty(T, E, dtype=torch.float32, device=dev)
    top_w = torch.empty(T, top_k, dtype=tw_dtype, device=dev)
    top_i = torch.empty(T, top_k, dtype=torch.int64, device=dev)
    top_w32 = torch.empty(T, top_k, dtype=torch.float32, device=dev)
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    psum = torch.empty(E, dtype=torch.float32, device=dev)
    lse2 = torch.empty(1, dtype=torch.float32, device=dev)
    ws = workspace(size("pmoe_router_forward_workspace_size", T, H, E), dev)
    w_ptr, w_code = _router_weight_arg(weight, pieces)
    call("pmoe_router_forward", ptr(x), dtype_code(x.dtype), w_ptr, w_code, ptr(logit_bias),
         T, H, E, top_k, int(norm_topk_prob), ptr(logits), ptr(top_w), dtype_code(tw_dtype), ptr(top_i),
         ptr(top_w32), ptr(counts), ptr(psum), ptr(lse2), ptr(ws), ws.numel(), stream_of(x))
    return logits, top_w, top_i, top_w32, counts, psum, lse2


def router_backward(x, weight, logits, top_i, top_w32, grad_top_w=None, grad_logits=None,
                    norm_topk_prob: bool = True, pieces=None):
    """-> grad_x (x.dtype), grad_weight (weight.dtype). ``pieces`` as in
    ``router_forward`` (the forward's, so the weight is split once)."""
    T, H = x.shape
    E, K = weight.shape[0], top_i.shape[1]
    gx = torch.empty_like(x)
    gW = torch.empty_like(weight)
    gw_code = dtype_code(grad_top_w.dtype) if grad_top_w is not None else 0
    ws = workspace(size("pmoe_router_backward_workspace_size", T, H, E), x.device)
    w_ptr, w_code = _router_weight_arg(weight, pieces)
    call("pmoe_router_backward", ptr(x), dtype_code(x.dtype), w_ptr, w_code, ptr(logits),
         ptr(top_i), ptr(top_w32), ptr(grad_top_w), gw_code, ptr(grad_logits), T, H, E, K, int(norm_topk_prob),
         ptr(gx), ptr(gW), ptr(ws), ws.numel(), stream_of(x))
    return gx, gW


def permute(top_indices, num_experts: int):
    """-> counts (E,) int32, offs (E,) int32, sorted_pair (P,) int32, inv_pos (P,) int32."""
    require_gpu(top_indices)
    T, K = top_indices.shape
    dev = top_indices.device
    P = T * K
    counts = torch.empty(num_experts, dtype=torch.int32, device=dev)
    offs = torch.empty(num_experts, dtype=torch.int32, device=dev)
    sorted_pair = torch.empty(P, dtype=torch.int32, device=dev)
    inv_pos = torch.empty(P, dtype=torch.int32, device=dev)
    ws = workspace(size("pmoe_permute_workspace_size", T, K, num_experts), dev)
    call("pmoe_permute", ptr(top_indices), T, K, num_experts, ptr(counts), ptr(offs), ptr(sorted_pair),
         ptr(inv_pos), ptr(ws), ws.numel(), stream_of(top_indices))
    return counts, offs, sorted_pair, inv_pos


def permute_rows(top_indices, top_weights, num_experts: int):
    """``permute`` and ``sort_rows`` in one pass: -> counts, offs, sorted_pair, inv_pos,
    sorted_token (P,) int32, sorted_w (P,) fp32 (None when top_weights is None)."""
    require_gpu(top_indices)
    T, K = top_indices.shape
    dev = top_indices.device
    P = T * K
    i32 = torch.int32
    counts, offs = (torch.empty(num_experts, dtype=i32, device=dev) for _ in range(2))
    sorted_pair, inv_pos, tok = (torch.empty(P, dtype=i32, device=dev) for _ in range(3))
    sw = torch.empty(P, dtype=torch.float32, device=dev) if top_weights is not None else None
    wcode = dtype_code(top_weights.dtype) if top_weights is not None else 0
    ws = workspace(size("pmoe_permute_workspace_size", T, K, num_experts), dev)
    call("pmoe_permute_rows", ptr(top_indices), ptr(top_weights), wcode, T, K, num_experts, ptr(counts), ptr(offs),
         ptr(sorted_pair), ptr(inv_pos), ptr(tok), ptr(sw), ptr(ws), ws.numel(), stream_of(top_indices))
    return counts, offs, sorted_pair, inv_pos, tok, sw


def count_invalid_ids(top_indices, num_experts: int) -> torch.Tensor:
    """-> (1,) int32 device tensor: ids of top_indices outside [0, E)."""
    require_gpu(top_indices)
    count = torch.empty(1, dtype=torch.int32, device=top_indices.device)
    call("pmoe_count_invalid_ids", ptr(top_indices), top_indices.numel(), num_experts, ptr(count),
         stream_of(top_indices))
    return count


def dispatch(hidden, inv_pos, top_k: int):
    """x_perm[inv_pos[t*K + k]] = hidden[t] (the expert-sorted row gather)."""
    T, H = hidden.shape
    x_perm = torch.empty(T * top_k, H, dtype=hidden.dtype, device=hidden.device)
    call("pmoe_dispatch", ptr(hidden), dtype_code(hidden.dtype), ptr(inv_pos), T, top_k, H, ptr(x_perm),
         stream_of(hidden))
    return x_perm


def sort_rows(sorted_pair, top_weights, top_k: int):
    """-> sorted_token (P,) int32 = sorted_pair / K, sorted_w (P,) fp32 = top_weights.flatten()[sorted_pair]
    (sorted_w None when top_weights is None)."""
    P = sorted_pair.shape[0]
    dev = sorted_pair.device
    tok = torch.empty(P, dtype=torch.int32, device=dev)
    sw = torch.empty(P, dtype=torch.float32, device=dev) if top_weights is not None else None
    wcode = dtype_code(top_weights.dtype) if top_weights is not None else 0
    call("pmoe_sort_rows", ptr(sorted_pair), ptr(top_weights), wcode, P // top_k, top_k, ptr(tok), ptr(sw),
         stream_of(sorted_pair))
    return tok, sw


def gate_up_swiglu(x, gate_up_proj, offs, row_index=None, row_weight=None):
    """-> gate_up_out (P, 2I), mid (P, I) = row_weight * silu(gate) * up.

    Row p of the GEMM's input is x[row_index[p]] (gathered) or x[p] when
    row_index is None (x is then the expert-sorted (P, H) copy)."""
    E, H, I = _dims(gate_up_proj)
    P = row_index.shape[0] if row_index is not None else x.shape[0]
    gu = torch.empty(P, 2 * I, dtype=x.dtype, device=x.device)
    mid = torch.empty(P, I, dtype=x.dtype, device=x.device)
    call("pmoe_gate_up_swiglu", ptr(x), ptr(row_index), ptr(row_weight), x.shape[0], ptr(gate_up_proj), ptr(offs),
         dtype_code(x.dtype), P, E, H, I, ptr(gu), ptr(mid), stream_of(x))
    return gu, mid


def down_proj(mid, down_proj_w, offs):
    E, H, I = down_proj_w.shape
    P = mid.shape[0]
    y = torch.empty(P, H, dtype=mid.dtype, device=mid.device)
    call("pmoe_down_proj", ptr(mid), ptr(down_proj_w), ptr(offs), dtype_code(mid.dtype), P, E, H, I, ptr(y),
         stream_of(mid))
    return y


def combine(y, top_weights, inv_pos, top_k: int | None = None):
    """out[t] = sum_k w[t,k] * y[inv_pos[t*K + k]]; top_weights None: unit weights (then give top_k)."""
    T, K = (top_weights.shape if top_weights is not None else (inv_pos.shape[0] // top_k, top_k))
    H = y.shape[1]
    out = torch.empty(T, H, dtype=y.dtype, device=y.device)
    wcode = dtype_code(top_weights.dtype) if top_weights is not None else 0
    call("pmoe_combine", ptr(y), ptr(top_weights), wcode, ptr(inv_pos), dtype_code(y.dtype), T, K, H, ptr(out),
         stream_of(y))
    return out


def combine_backward(grad_out, y, top_weights, inv_pos):
    T, K = top_weights.shape
    H = y.shape[1]
    gy = torch.empty_like(y)
    gw = torch.empty_like(top_weights)
    call("pmoe_combine_backward", ptr(grad_out), ptr(y), ptr(top_weights), dtype_code(top_weights.dtype),
         ptr(inv_pos), dtype_code(y.dtype), T, K, H, ptr(gy), ptr(gw), stream_of(y))
    return gy, gw


def part_cols(inter: int) -> int:
    """Routing-weight partials per sorted row: one per 64-column block of I."""
    return (inter + 63) // 64


def down_proj_backward(grad, mid, gate_up_out, down_proj_w, offs, row_index=None, row_weight=None,
                       need_part=False):
    """-> grad_gate_up_out (P, 2I), grad_down_proj, partials (P, ceil(I/64)) fp32 or None.

    The GEMMs' rows of ``grad`` are grad[row_index[p]] (gathered) or grad[p];
    with row_weight (mid = w * silu(g) * u), grad is the gradient of the
    weighted rows and the partials sum to the routing weights' gradient."""
    E, H, I = down_proj_w.shape
    P = row_index.shape[0] if row_index is not None else grad.shape[0]
    ggu = torch.empty(P, 2 * I, dtype=grad.dtype, device=grad.device)
    gdn = torch.empty_like(down_proj_w)
    part = torch.empty(P, part_cols(I), dtype=torch.float32, device=grad.device) if need_part else None
    call("pmoe_down_proj_backward", ptr(grad), ptr(row_index), ptr(row_weight), grad.shape[0], ptr(mid),
         ptr(gate_up_out), ptr(down_proj_w), ptr(offs), dtype_code(grad.dtype), P, E, H, I, ptr(ggu), ptr(gdn),
         dtype_code(gdn.dtype), ptr(part), part_cols(I), stream_of(grad))
    return ggu, gdn, part


def down_proj_dgrad(grad, gate_up_out, down_proj_w, offs, row_index=None, row_weight=None, need_part=False):
    """grad_gate_up_out = SwiGLU'(gate_up_out) * (w *) (G . down_proj[e]) (one kernel), and with
    need_part the routing-weight partials (P, ceil(I/64)) fp32 (else None)."""
    E, H, I = down_proj_w.shape
    P = row_index.shape[0] if row_index is not None else grad.shape[0]
    ggu = torch.empty(P, 2 * I, dtype=grad.dtype, device=grad.device)
    part = torch.empty(P, part_cols(I), dtype=torch.float32, device=grad.device) if need_part else None
    call("pmoe_down_proj_backward", ptr(grad), ptr(row_index), ptr(row_weight), grad.shape[0], None,
         ptr(gate_up_out), ptr(down_proj_w), ptr(offs), dtype_code(grad.dtype), P, E, H, I, ptr(ggu), None,
         dtype_code(grad.dtype), ptr(part), part_cols(I), stream_of(grad))
    return ggu, part


def down_proj_wgrad(grad, mid, offs, num_experts: int, out_dtype=None, row_index=None):
    """grad_down_proj[e] = G_e^T . mid_e (one kernel), G_p = grad[row_index[p]] or grad[p], in
    `out_dtype` (default the operands'; fp32 from bf16 operands for an fp32 master weight)."""
    H = grad.shape[1]
    P, I = mid.shape
    gdn = torch.empty(num_experts, H, I, dtype=out_dtype or grad.dtype, device=grad.device)
    call("pmoe_down_proj_backward", ptr(grad), ptr(row_index), None, grad.shape[0], ptr(mid), None, None, ptr(offs),
         dtype_code(grad.dtype), P, num_experts, H, I, None, ptr(gdn), dtype_code(gdn.dtype), None, 0,
         stream_of(grad))
    return gdn


def gate_up_dgrad(grad_gate_up_out, gate_up_proj, offs):
    """grad_x_perm = grad_gate_up_out . gate_up_proj[e] (one kernel; the sorted rows' input gradient)."""
    E, H, I = _dims(gate_up_proj)
    P = grad_gate_up_out.shape[0]
    gx = torch.empty(P, H, dtype=grad_gate_up_out.dtype, device=grad_gate_up_out.device)
    call("pmoe_gate_up_backward", ptr(grad_gate_up_out), None, None, P, ptr(gate_up_proj), ptr(offs),
         dtype_code(gx.dtype), P, E, H, I, ptr(gx), None, dtype_code(gx.dtype), stream_of(gx))
    return gx


def gate_up_wgrad(grad_gate_up_out, x, offs, num_experts: int, out_dtype=None, row_index=None):
    """grad_gate_up_proj[e] = grad_gate_up_out_e^T . X_e, X_p = x[row_index[p]] or x[p] (one kernel),
    in `out_dtype` (default the operands'; fp32 from bf16 operands for an fp32 master)."""
    H = x.shape[1]
    P = grad_gate_up_out.shape[0]
    I = grad_gate_up_out.shape[1] // 2
    gw = torch.empty(num_experts, 2 * I, H, dtype=out_dtype or x.dtype, device=x.device)
    call("pmoe_gate_up_backward", ptr(grad_gate_up_out), ptr(x), ptr(row_index), x.shape[0], None, ptr(offs),
         dtype_code(x.dtype), P, num_experts, H, I, None, ptr(gw), dtype_code(gw.dtype), stream_of(x))
    return gw


def gate_up_backward(grad_gate_up_out, x, gate_up_proj, offs, row_index=None):
    E, H, I = _dims(gate_up_proj)
    P = grad_gate_up_out.shape[0]
    gx = torch.empty(P, H, dtype=x.dtype, device=x.device)
    gw = torch.empty_like(gate_up_proj)
    call("pmoe_gate_up_backward", ptr(grad_gate_up_out), ptr(x), ptr(row_index), x.shape[0], ptr(gate_up_proj),
         ptr(offs), dtype_code(x.dtype), P, E, H, I, ptr(gx), ptr(gw), dtype_code(gw.dtype), stream_of(x))
    return gx, gw


def pair_weight_grad(part, inv_pos, top_k: int, out_dtype=torch.float32):
    """grad_top_weights (T, K) = the sum of each pair's row partials (from down_proj_backward)."""
    P, ld = part.shape
    T = P // top_k
    gw = torch.empty(T, top_k, dtype=out_dtype, device=part.device)
    call("pmoe_pair_weight_grad", ptr(part), ld, ld, ptr(inv_pos), T, top_k, ptr(gw), dtype_code(out_dtype),
         stream_of(part))
    return gw


def dispatch_backward(grad_x_perm, inv_pos, tokens: int, top_k: int, add=None):
    """grad_hidden[t] = add[t] + sum_k grad_x_perm[inv_pos[t*K + k]] (add may be None)."""
    H = grad_x_perm.shape[1]
    gh = torch.empty(tokens, H, dtype=grad_x_perm.dtype, device=grad_x_perm.device)
    if add is not None:
        assert add.shape == gh.shape and add.dtype == gh.dtype and add.is_contiguous()
    call("pmoe_dispatch_backward", ptr(grad_x_perm), ptr(inv_pos), ptr(add), dtype_code(grad_x_perm.dtype), tokens,
         top_k, H, ptr(gh), stream_of(grad_x_perm))
    return gh


# --------------------------------------------- block neighbours (norm2, residual)


def rmsnorm_forward(x, weight, eps: float, out_dtype):
    """torch.nn.RMSNorm in fp32 arithmetic -> out (T,H) out_dtype, rstd (T,) fp32. weight (H,) fp32."""
    require_gpu(x, weight)
    T, H = x.shape
    out = torch.empty(T, H, dtype=out_dtype, device=x.device)
    rstd = torch.empty(T, dtype=torch.float32, device=x.device)
    call("pmoe_rmsnorm_forward", ptr(x), dtype_code(x.dtype), ptr(weight), float(eps), T, H, ptr(out),
         dtype_code(out_dtype), ptr(rstd), stream_of(x))
    return out, rstd


def combine_residual(y, top_weights, inv_pos, residual, top_k: int | None = None):
    """out (residual.dtype) = residual + the (weighted) K-sum of the expert rows; top_weights None: unit weights."""
    T = residual.shape[0]
    K = top_weights.shape[1] if top_weights is not None else top_k
    H = y.shape[1]
    out = torch.empty_like(residual)
    wcode = dtype_code(top_weights.dtype) if top_weights is not None else 0
    call("pmoe_combine_residual", ptr(y), ptr(top_weights), wcode, ptr(inv_pos), dtype_code(y.dtype), ptr(residual),
         dtype_code(residual.dtype), T, K, H, ptr(out), stream_of(y))
    return out


def combine_residual_backward(grad_out, y, top_weights, inv_pos):
    """-> grad_y (y.dtype), grad_top_weights; grad_out in the residual stream's dtype."""
    T, K = top_weights.shape
    H = y.shape[1]
    gy = torch.empty_like(y)
    gw = torch.empty_like(top_weights)
    call("pmoe_combine_residual_backward", ptr(grad_out), dtype_code(grad_out.dtype), ptr(y), ptr(top_weights),
         dtype_code(top_weights.dtype), ptr(inv_pos), dtype_code(y.dtype), T, K, H, ptr(gy), ptr(gw), stream_of(y))
    return gy, gw


def dispatch_rmsnorm_backward(grad_x_perm, inv_pos, grad_normed_add, x, weight, rstd, grad_residual, top_k: int,
                              need_weight: bool = True, weight_dtype=torch.float32):
    """-> grad_x (x.dtype), grad_weight (weight_dtype, or None).

    grad_x = grad_residual + RMSNorm-backward(grad_normed_add + K-sum of grad_x_perm);
    grad_x_perm, grad_normed_add and grad_residual may each be None.
    """
    T, H = x.shape
    g = grad_x_perm if grad_x_perm is not None else grad_normed_add
    gdt = g.dtype if g is not None else torch.bfloat16
    gx = torch.empty_like(x)
    gw = torch.empty(H, dtype=weight_dtype, device=x.device) if need_weight else None
    ws = workspace(size("pmoe_dispatch_rmsnorm_backward_workspace_size", T, H) if need_weight else 0, x.device)
    call("pmoe_dispatch_rmsnorm_backward", ptr(grad_x_perm), ptr(inv_pos), ptr(grad_normed_add), dtype_code(gdt),
         ptr(x), dtype_code(x.dtype), ptr(weight), ptr(rstd), ptr(grad_residual), T, top_k, H, ptr(gx), ptr(gw),
         dtype_code(weight_dtype), ptr(ws), ws.numel(), stream_of(x))
    return gx, gw
