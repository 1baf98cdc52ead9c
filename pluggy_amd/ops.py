"""Functional wrappers of each C-ABI entry point (no autograd).

One function per kernel stage of the MoE block, so every stage can be called,
tested and timed on its own. Shapes follow ``include/pmoe.h``; outputs are
freshly allocated on the input's device and stream.
"""

from __future__ import annotations

import torch

from ._lib import call, dtype_code, ptr, require_gpu, size, stream_of, workspace


def _dims(gate_up_proj: torch.Tensor):
    E, two_i, H = gate_up_proj.shape
    return E, H, two_i // 2


def router_forward(x, weight, top_k: int, norm_topk_prob: bool = True, logit_bias=None):
    """-> logits, top_w (x.dtype), top_i (int64), top_w_f32, counts (int32), prob_sum, lse_sq_sum."""
    require_gpu(x, weight, logit_bias)
    T, H = x.shape
    E = weight.shape[0]
    dev = x.device
    logits = torch.empty(T, E, dtype=torch.float32, device=dev)
    top_w = torch.empty(T, top_k, dtype=x.dtype, device=dev)
    top_i = torch.empty(T, top_k, dtype=torch.int64, device=dev)
    top_w32 = torch.empty(T, top_k, dtype=torch.float32, device=dev)
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    psum = torch.empty(E, dtype=torch.float32, device=dev)
    lse2 = torch.empty(1, dtype=torch.float32, device=dev)
    ws = workspace(size("pmoe_router_forward_workspace_size", T, H, E), dev)
    call("pmoe_router_forward", ptr(x), dtype_code(x.dtype), ptr(weight), dtype_code(weight.dtype), ptr(logit_bias),
         T, H, E, top_k, int(norm_topk_prob), ptr(logits), ptr(top_w), dtype_code(x.dtype), ptr(top_i),
         ptr(top_w32), ptr(counts), ptr(psum), ptr(lse2), ptr(ws), ws.numel(), stream_of(x))
    return logits, top_w, top_i, top_w32, counts, psum, lse2


def router_backward(x, weight, logits, top_i, top_w32, grad_top_w=None, grad_logits=None,
                    norm_topk_prob: bool = True):
    """-> grad_x (x.dtype), grad_weight (weight.dtype)."""
    T, H = x.shape
    E, K = weight.shape[0], top_i.shape[1]
    gx = torch.empty_like(x)
    gW = torch.empty_like(weight)
    gw_code = dtype_code(grad_top_w.dtype) if grad_top_w is not None else 0
    ws = workspace(size("pmoe_router_backward_workspace_size", T, H, E), x.device)
    call("pmoe_router_backward", ptr(x), dtype_code(x.dtype), ptr(weight), dtype_code(weight.dtype), ptr(logits),
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


def gate_up_swiglu(x_perm, gate_up_proj, offs):
    E, H, I = _dims(gate_up_proj)
    P = x_perm.shape[0]
    gu = torch.empty(P, 2 * I, dtype=x_perm.dtype, device=x_perm.device)
    mid = torch.empty(P, I, dtype=x_perm.dtype, device=x_perm.device)
    call("pmoe_gate_up_swiglu", ptr(x_perm), ptr(gate_up_proj), ptr(offs), dtype_code(x_perm.dtype), P, E, H, I,
         ptr(gu), ptr(mid), stream_of(x_perm))
    return gu, mid


def down_proj(mid, down_proj_w, offs):
    E, H, I = down_proj_w.shape
    P = mid.shape[0]
    y = torch.empty(P, H, dtype=mid.dtype, device=mid.device)
    call("pmoe_down_proj", ptr(mid), ptr(down_proj_w), ptr(offs), dtype_code(mid.dtype), P, E, H, I, ptr(y),
         stream_of(mid))
    return y


def combine(y, top_weights, inv_pos):
    T, K = top_weights.shape
    H = y.shape[1]
    out = torch.empty(T, H, dtype=y.dtype, device=y.device)
    call("pmoe_combine", ptr(y), ptr(top_weights), dtype_code(top_weights.dtype), ptr(inv_pos), dtype_code(y.dtype),
         T, K, H, ptr(out), stream_of(y))
    return out


def combine_backward(grad_out, y, top_weights, inv_pos):
    T, K = top_weights.shape
    H = y.shape[1]
    gy = torch.empty_like(y)
    gw = torch.empty_like(top_weights)
    call("pmoe_combine_backward", ptr(grad_out), ptr(y), ptr(top_weights), dtype_code(top_weights.dtype),
         ptr(inv_pos), dtype_code(y.dtype), T, K, H, ptr(gy), ptr(gw), stream_of(y))
    return gy, gw


def down_proj_backward(grad_y, mid, gate_up_out, down_proj_w, offs):
    E, H, I = down_proj_w.shape
    P = grad_y.shape[0]
    ggu = torch.empty(P, 2 * I, dtype=grad_y.dtype, device=grad_y.device)
    gdn = torch.empty_like(down_proj_w)
    call("pmoe_down_proj_backward", ptr(grad_y), ptr(mid), ptr(gate_up_out), ptr(down_proj_w), ptr(offs),
         dtype_code(grad_y.dtype), P, E, H, I, ptr(ggu), ptr(gdn), dtype_code(gdn.dtype), stream_of(grad_y))
    return ggu, gdn


def down_proj_dgrad(grad_y, gate_up_out, down_proj_w, offs):
    """grad_gate_up_out = SwiGLU'(gate_up_out) * (grad_y . down_proj[e]) (one kernel)."""
    E, H, I = down_proj_w.shape
    P = grad_y.shape[0]
    ggu = torch.empty(P, 2 * I, dtype=grad_y.dtype, device=grad_y.device)
    call("pmoe_down_proj_backward", ptr(grad_y), None, ptr(gate_up_out), ptr(down_proj_w), ptr(offs),
         dtype_code(grad_y.dtype), P, E, H, I, ptr(ggu), None, dtype_code(grad_y.dtype), stream_of(grad_y))
    return ggu


def down_proj_wgrad(grad_y, mid, offs, num_experts: int, out_dtype=None):
    """grad_down_proj[e] = grad_y_e^T . mid_e (one kernel), in `out_dtype`
    (default the operands'; fp32 from bf16 operands for an fp32 master weight)."""
    P, H = grad_y.shape
    I = mid.shape[1]
    gdn = torch.empty(num_experts, H, I, dtype=out_dtype or grad_y.dtype, device=grad_y.device)
    call("pmoe_down_proj_backward", ptr(grad_y), ptr(mid), None, None, ptr(offs), dtype_code(grad_y.dtype), P,
         num_experts, H, I, None, ptr(gdn), dtype_code(gdn.dtype), stream_of(grad_y))
    return gdn


def gate_up_dgrad(grad_gate_up_out, gate_up_proj, offs):
    """grad_x_perm = grad_gate_up_out . gate_up_proj[e] (one kernel)."""
    E, H, I = _dims(gate_up_proj)
    P = grad_gate_up_out.shape[0]
    gx = torch.empty(P, H, dtype=grad_gate_up_out.dtype, device=grad_gate_up_out.device)
    call("pmoe_gate_up_backward", ptr(grad_gate_up_out), None, ptr(gate_up_proj), ptr(offs),
         dtype_code(gx.dtype), P, E, H, I, ptr(gx), None, dtype_code(gx.dtype), stream_of(gx))
    return gx


def gate_up_wgrad(grad_gate_up_out, x_perm, offs, num_experts: int, out_dtype=None):
    """grad_gate_up_proj[e] = grad_gate_up_out_e^T . x_perm_e (one kernel), in
    `out_dtype` (default the operands'; fp32 from bf16 operands for an fp32 master)."""
    P, H = x_perm.shape
    I = grad_gate_up_out.shape[1] // 2
    gw = torch.empty(num_experts, 2 * I, H, dtype=out_dtype or x_perm.dtype, device=x_perm.device)
    call("pmoe_gate_up_backward", ptr(grad_gate_up_out), ptr(x_perm), None, ptr(offs), dtype_code(x_perm.dtype),
         P, num_experts, H, I, None, ptr(gw), dtype_code(gw.dtype), stream_of(x_perm))
    return gw


def gate_up_backward(grad_gate_up_out, x_perm, gate_up_proj, offs):
    E, H, I = _dims(gate_up_proj)
    P = x_perm.shape[0]
    gx = torch.empty_like(x_perm)
    gw = torch.empty_like(gate_up_proj)
    call("pmoe_gate_up_backward", ptr(grad_gate_up_out), ptr(x_perm), ptr(gate_up_proj), ptr(offs),
         dtype_code(x_perm.dtype), P, E, H, I, ptr(gx), ptr(gw), dtype_code(gw.dtype), stream_of(x_perm))
    return gx, gw


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


def combine_residual(y, top_weights, inv_pos, residual):
    """out (residual.dtype) = residual + the weighted K-sum of the expert rows."""
    T, K = top_weights.shape
    H = y.shape[1]
    out = torch.empty_like(residual)
    call("pmoe_combine_residual", ptr(y), ptr(top_weights), dtype_code(top_weights.dtype), ptr(inv_pos),
         dtype_code(y.dtype), ptr(residual), dtype_code(residual.dtype), T, K, H, ptr(out), stream_of(y))
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
