/*
 * pmoe: MI355X-native (gfx950) kernels for pluggy's Qwen3-MoE sparse FFN block.
 *
 * C ABI. Conventions shared by every entry point:
 *  - Pointers are device pointers (HBM) unless stated; tensors are dense
 *    row-major. Sizes are element counts.
 *  - dtype codes: PMOE_F32 (fp32), PMOE_BF16 (bf16 stored as uint16) or
 *    PMOE_F16 (IEEE fp16). fp16 is taken by the expert path (permutation row
 *    tables, row movers, expert GEMMs, the whole-FFN entry points), which
 *    computes it on the fp16 MFMAs with fp32 accumulation as the reference's
 *    F.grouped_mm does for fp16 tensors; so is the router when its x and
 *    weight are both fp16. The RMSNorm and residual neighbours take fp32 or
 *    bf16.
 *  - `stream` is a hipStream_t (NULL = the default stream). Work is enqueued
 *    asynchronously; no entry point synchronises the host or allocates
 *    memory. Scratch memory comes from the caller through `workspace`, sized by
 *    the matching *_workspace_size query.
 *  - Return 0 on success, a negative PMOE_ERR_* code for a rejected argument,
 *    or a positive hipError_t from the runtime. pmoe_last_error_string()
 *    describes the most recent failure of the calling thread.
 *  - Inputs are never modified (except `logits` of pmoe_router_forward, which
 *    is an output). Outputs are overwritten, never accumulated into.
 *  - Requirements: H and I are multiples of 8; 1 <= K <= E <= 1024; K <= 64.
 *
 * Citations name the reference function each entry point replaces
 * (sonnetx/pluggy, paths relative to the repository root).
 */
#ifndef PMOE_H
#define PMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PMOE_API __attribute__((visibility("default")))

/* PMOE_BF16X3: a router weight that is fp32, given as the bf16 pieces
 * pmoe_router_split_weight writes (router entry points only, beside bf16 x). */
enum { PMOE_F32 = 0, PMOE_BF16 = 1, PMOE_F16 = 2, PMOE_BF16X3 = 3 };
enum {
  PMOE_OK = 0,
  PMOE_ERR_INVALID = -1,     /* bad shape, dtype or null pointer */
  PMOE_ERR_UNSUPPORTED = -2, /* a valid request outside what is built */
  PMOE_ERR_WORKSPACE = -3    /* workspace smaller than the size query */
};

PMOE_API const char* pmoe_version(void);
PMOE_API const char* pmoe_last_error_string(void);

/* ---------------------------------------------------------------- router ---
 * Replaces Qwen3MoeTopKRouter.forward (pluggy/models/qwen3_moe/qwen3_moe.py:168-178):
 *   logits = x . W^T (+ logit_bias)  [fp32 arithmetic; for bf16 x the fp32 W is
 *   split into three bf16 pieces whose products with x are exact; fp16 x and
 *   fp16 W multiply exactly on the fp16 MFMAs]
 *   p = softmax(logits) (fp32); top-k of logits (ties -> lower expert id)
 *   w = p[top] (/ sum p[top] when norm_topk_prob), written as tw_dtype and fp32.
 * Also emits the additive aux statistics of load_balancing_loss / router_z_loss
 * (qwen3_moe.py:285-316) and the per-expert counts of _update_expert_counts
 * (qwen3_moe.py:417-426): expert_counts[e] (int32), prob_sum[e] = sum_t p[t,e],
 * lse_sq_sum = sum_t logsumexp(logits[t])^2. Any of the three may be NULL.
 * x: (T,H) x_dtype; weight: (E,H) w_dtype (each fp32 or bf16, or both fp16:
 * the reference's F.linear under fp16 takes fp16 x and W, qwen3_moe.py:172;
 * or, beside bf16 x, PMOE_BF16X3: the pieces of an fp32 weight from
 * pmoe_router_split_weight, which spare the call its own split);
 * logit_bias: (E,) fp32 or NULL; logits: (T,E) fp32; top_weights: (T,K)
 * tw_dtype (fp32, bf16 or fp16, rounded as the reference's
 * .to(hidden_states.dtype), qwen3_moe.py:177);
 * top_indices: (T,K) int64; top_weights_f32: (T,K) fp32 (kept for the
 * backward). */
PMOE_API size_t pmoe_router_forward_workspace_size(int64_t T, int64_t H, int64_t E);
PMOE_API int pmoe_router_forward(const void* x, int x_dtype, const void* weight, int w_dtype,
                                 const float* logit_bias, int64_t T, int64_t H, int64_t E, int64_t K,
                                 int norm_topk_prob, float* logits, void* top_weights, int tw_dtype,
                                 int64_t* top_indices, float* top_weights_f32, int32_t* expert_counts,
                                 float* prob_sum, float* lse_sq_sum, void* workspace, size_t workspace_bytes,
                                 void* stream);

/* Autograd of pmoe_router_forward (torch derivatives of qwen3_moe.py:172-177):
 *   dl = d(top_weights) through renorm/softmax/top-k (+ grad_logits)
 *   grad_x = dl . W  (x_dtype, overwritten),  grad_weight = dl^T . x (w_dtype).
 * dl is fp32; its products with x and W are formed exactly from 16-bit
 * pieces of dl (two bf16 pieces; for fp16 x and W, grad_weight from two fp16
 * pieces, which carry fp16's exponent range as the reference's fp16 dl does).
 * grad_top_weights (T,K) gw_dtype (fp32, bf16 or fp16) and grad_logits (T,E)
 * fp32 may be NULL (zero); grad_x / grad_weight may be NULL (not needed).
 * A weight given as PMOE_BF16X3 pieces (E a multiple of 8) gets its gradient
 * in fp32. */
PMOE_API size_t pmoe_router_backward_workspace_size(int64_t T, int64_t H, int64_t E);
/* The bf16 pieces of an fp32 router weight (E,H) that pmoe_router_forward and
 * pmoe_router_backward take as w_dtype PMOE_BF16X3, so that a forward and its
 * backward (or the micro-batches of one optimizer step) split the weight once
 * instead of on every call: pieces (4,E,H) bf16 = [lo; hi; mid; hi], hi =
 * bf16(W), mid = bf16(W - hi), lo = bf16(W - hi - mid); hi + mid + lo = W to
 * 2^-24 relative. Part of the split inside pmoe_router_forward (the per-call
 * copy of qwen3_moe.py:172's weight operand), exposed; no reference
 * counterpart of its own. */
PMOE_API int pmoe_router_split_weight(const float* weight, int64_t E, int64_t H, void* pieces, void* stream);
PMOE_API int pmoe_router_backward(const void* x, int x_dtype, const void* weight, int w_dtype,
                                  const float* logits, const int64_t* top_indices, const float* top_weights_f32,
                                  const void* grad_top_weights, int gw_dtype, const float* grad_logits, int64_t T,
                                  int64_t H, int64_t E, int64_t K, int norm_topk_prob, void* grad_x,
                                  void* grad_weight, void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------- permutation ---
 * Replaces the flatten / argsort(stable) / bincount / cumsum of
 * _expert_ffn_grouped (pluggy/kernels/moe.py:89-108): a stable counting sort of
 * the P = T*K pairs q = t*K + k by expert top_indices[q].
 * counts (E,) int32; offs (E,) int32 inclusive end offsets (moe.py:108);
 * sorted_pair (P,) int32 (token = sorted_pair / K); inv_pos (P,) int32 with
 * inv_pos[sorted_pair[p]] = p.
 * Ids outside [0,E) are not rejected here (no entry point syncs the host):
 * they are clamped into range, so such a pair is routed to expert 0 or E-1,
 * where the reference raises (F.one_hot at moe.py:50 on its loop path,
 * bincount and the offs length on its grouped path, moe.py:106-108). Callers
 * whose indices do not come from pmoe_router_forward check them first with
 * pmoe_count_invalid_ids (the Python operator moe_expert_ffn does, and
 * raises). */
PMOE_API size_t pmoe_permute_workspace_size(int64_t T, int64_t K, int64_t E);
PMOE_API int pmoe_permute(const int64_t* top_indices, int64_t T, int64_t K, int64_t E, int32_t* counts,
                          int32_t* offs, int32_t* sorted_pair, int32_t* inv_pos, void* workspace,
                          size_t workspace_bytes, void* stream);

/* Number of ids in top_indices[0..n) outside [0, E), written to count[0]
 * (int32, device memory): the check behind the RuntimeError that the
 * reference's F.one_hot (moe.py:50) and bincount (moe.py:107) raise on such
 * ids. One small kernel; the caller reads the count. */
PMOE_API int pmoe_count_invalid_ids(const int64_t* top_indices, int64_t n, int64_t E, int32_t* count, void* stream);

/* Row gather hidden[sorted_token] (moe.py:104), done in scatter form:
 * x_perm[inv_pos[t*K + k]] = hidden[t] for every token t and slot k (each
 * hidden row is read once), which equals x_perm[p] = hidden[sorted_pair[p] / K]. */
PMOE_API int pmoe_dispatch(const void* hidden, int dtype, const int32_t* inv_pos, int64_t T, int64_t K, int64_t H,
                           void* x_perm, void* stream);

/* pmoe_permute and pmoe_sort_rows in one pass (moe.py:89-108): the
 * permutation, and for each sorted row p the expert GEMMs' row tables
 * sorted_token[p] = sorted_pair[p] / K and sorted_w[p] = float(top_weights[
 * sorted_pair[p]]) (sorted_w may be NULL, then top_weights too). Workspace as
 * pmoe_permute_workspace_size. */
PMOE_API int pmoe_permute_rows(const int64_t* top_indices, const void* top_weights, int w_dtype, int64_t T,
                               int64_t K, int64_t E, int32_t* counts, int32_t* offs, int32_t* sorted_pair,
                               int32_t* inv_pos, int32_t* sorted_token, float* sorted_w, void* workspace,
                               size_t workspace_bytes, void* stream);

/* Per sorted row p of the permutation (pair q = sorted_pair[p]):
 * sorted_token[p] = q / K, the token whose row the expert GEMMs gather (the
 * reference's sorted_token, moe.py:90-101), and sorted_w[p] = top_weights[q]
 * as fp32 (its sorted_w, moe.py:103). top_weights / sorted_w may be NULL
 * together (no weights). sorted_pair, sorted_token, sorted_w: (T*K,). */
PMOE_API int pmoe_sort_rows(const int32_t* sorted_pair, const void* top_weights, int w_dtype, int64_t T, int64_t K,
                            int32_t* sorted_token, float* sorted_w, void* stream);

/* Grouped gate_up GEMM + SwiGLU (moe.py:104, :113-118, :120; swiglu.py:14-16):
 * with A_p = x[row_index[p]] (the row gather hidden[sorted_token] done inside
 * the GEMM's operand loads; x holds x_rows rows) or A_p = x[p] when row_index
 * is NULL (x_rows = P),
 *   gate_up_out[p] = A_p . gate_up_proj[e(p)]^T  (P, 2I), rounded to dtype;
 *   mid[p] = row_weight[p] * silu(gate) * up  (P, I)  (row_weight NULL: 1),
 * i.e. the routing weight of moe.py:120 applied to the activation, so that
 * the down projection's rows come out weighted. gate_up_proj: (E, 2I, H).
 * A gathered x must stay below 2 GiB (PMOE_ERR_UNSUPPORTED beyond). */
PMOE_API int pmoe_gate_up_swiglu(const void* x, const int32_t* row_index, const float* row_weight, int64_t x_rows,
                                 const void* gate_up_proj, const int32_t* offs, int dtype, int64_t P, int64_t E,
                                 int64_t H, int64_t I, void* gate_up_out, void* mid, void* stream);

/* Grouped down GEMM (moe.py:119): y[p] = mid[p] . down_proj[e(p)]^T  (P, H);
 * down_proj: (E, H, I). y is the unweighted expert output. */
PMOE_API int pmoe_down_proj(const void* mid, const void* down_proj, const int32_t* offs, int dtype, int64_t P,
                            int64_t E, int64_t H, int64_t I, void* y, void* stream);

/* Weighted combine (moe.py:120-123, in gather form, fp32 accumulation, k ascending):
 * out[t] = sum_k top_weights[t,k] * y[inv_pos[t*K+k]]; top_weights NULL: unit
 * weights (rows that already carry their routing weight). */
PMOE_API int pmoe_combine(const void* y, const void* top_weights, int w_dtype, const int32_t* inv_pos, int dtype,
                          int64_t T, int64_t K, int64_t H, void* out, void* stream);

/* Backward of pmoe_combine: grad_y[p] = w * grad_out[t]; grad_top_weights[t,k] =
 * <grad_out[t], y[inv_pos[t*K+k]]>. */
PMOE_API int pmoe_combine_backward(const void* grad_out, const void* y, const void* top_weights, int w_dtype,
                                   const int32_t* inv_pos, int dtype, int64_t T, int64_t K, int64_t H,
                                   void* grad_y, void* grad_top_weights, void* stream);

/* Backward of pmoe_down_proj and the SwiGLU. G_p = grad[row_index[p]] (grad
 * holds grad_rows rows: the layer's output gradient, gathered as the
 * reference's grad of hidden[sorted_token] flows, moe.py:104/123) or
 * G_p = grad[p] when row_index is NULL (grad_rows = P). acc_p = G_p .
 * down_proj[e(p)].
 *   Without row_weight, G is the gradient of y and acc of mid:
 *     grad_gate_up_out = SwiGLU'(gate_up_out) * acc.
 *   With row_weight (mid = w * silu(g) * up from pmoe_gate_up_swiglu), acc is
 *   the gradient of that weighted mid:
 *     grad_gate_up_out = SwiGLU'(gate_up_out) * (w * acc), and when part is not
 *     NULL, part[p * part_ld + c] = sum over the 64 columns of block c of
 *     acc * silu(g) * up (part_ld >= ceil(I / 64)); row p's partials sum to the
 *     gradient of its routing weight (pmoe_pair_weight_grad).
 *   grad_down_proj[e] = G_e^T . mid_e (zeros for an empty expert).
 * Either output may be NULL. grad_weight_dtype is grad_down_proj's dtype:
 * `dtype`, or PMOE_F32 with 16-bit operands (the gradient of an fp32 master
 * weight that the forward cast to 16 bits, written without a separate cast). */
PMOE_API int pmoe_down_proj_backward(const void* grad, const int32_t* row_index, const float* row_weight,
                                     int64_t grad_rows, const void* mid, const void* gate_up_out,
                                     const void* down_proj, const int32_t* offs, int dtype, int64_t P, int64_t E,
                                     int64_t H, int64_t I, void* grad_gate_up_out, void* grad_down_proj,
                                     int grad_weight_dtype, float* part, int64_t part_ld, void* stream);

/* Backward of the gate_up GEMM: grad_x_perm = grad_gate_up_out . gate_up_proj[e]
 * (the sorted rows' input gradient; pmoe_dispatch_backward sums a token's K
 * rows); grad_gate_up_proj[e] = grad_gate_up_out_e^T . X_e with X_p =
 * x[row_index[p]] (x holds x_rows rows) or x[p] when row_index is NULL.
 * Either output may be NULL. grad_weight_dtype as for pmoe_down_proj_backward. */
PMOE_API int pmoe_gate_up_backward(const void* grad_gate_up_out, const void* x, const int32_t* row_index,
                                   int64_t x_rows, const void* gate_up_proj, const int32_t* offs, int dtype, int64_t P,
                                   int64_t E, int64_t H, int64_t I, void* grad_x_perm, void* grad_gate_up_proj,
                                   int grad_weight_dtype, void* stream);

/* Gradient of the routing weights (the autograd of moe.py:120, and of
 * index_add_'s input there): grad_top_weights[q] = sum_j part[inv_pos[q] *
 * part_ld + j] over j < nparts (fp32, j ascending), in gw_dtype; q = t*K + k. */
PMOE_API int pmoe_pair_weight_grad(const float* part, int64_t part_ld, int64_t nparts, const int32_t* inv_pos,
                                   int64_t T, int64_t K, void* grad_top_weights, int gw_dtype, void* stream);

/* Backward of pmoe_dispatch: grad_hidden[t] = grad_hidden_add[t] + sum_k
 * grad_x_perm[inv_pos[t*K+k]] (fp32 sum, k ascending; grad_hidden_add (T,H)
 * may be NULL, e.g. the router's share of the input gradient). */
PMOE_API int pmoe_dispatch_backward(const void* grad_x_perm, const int32_t* inv_pos, const void* grad_hidden_add,
                                    int dtype, int64_t T, int64_t K, int64_t H, void* grad_hidden, void* stream);

/* ------------------------------------------------------ block neighbours ---
 * The RMSNorm in front of the sparse MLP and the residual add behind it, as
 * Qwen3MoeTransformerBlock.forward computes them (pluggy/models/qwen3_moe/
 * qwen3_moe.py:281, x = x + ffn(norm2(x)); norm2 = torch.nn.RMSNorm, :260),
 * fused into the row kernels of the block. */

/* torch.nn.RMSNorm forward (elementwise weight): out[t] = (x[t] * r_t) * weight,
 * r_t = 1 / sqrt(sum_j x[t,j]^2 / H + eps), fp32 arithmetic; rstd[t] = r_t.
 * x: (T,H) x_dtype; weight: (H,) fp32; out: (T,H) out_dtype (the operand of the
 * router and the dispatch, e.g. bf16 from an fp32 residual stream, so no
 * separate cast); rstd: (T,) fp32. torch's default eps is finfo(x.dtype).eps. */
PMOE_API int pmoe_rmsnorm_forward(const void* x, int x_dtype, const float* weight, float eps, int64_t T, int64_t H,
                                  void* out, int out_dtype, float* rstd, void* stream);

/* pmoe_combine with the residual add fused (moe.py:120-123 + qwen3_moe.py:281):
 * out[t] = residual[t] + sum_k top_weights[t,k] * y[inv_pos[t*K+k]], fp32
 * accumulation starting from the residual, k ascending. residual and out:
 * (T,H) res_dtype (e.g. an fp32 residual stream over bf16 expert rows). */
PMOE_API int pmoe_combine_residual(const void* y, const void* top_weights, int w_dtype, const int32_t* inv_pos,
                                   int dtype, const void* residual, int res_dtype, int64_t T, int64_t K, int64_t H,
                                   void* out, void* stream);

/* Backward of pmoe_combine_residual (the residual's gradient is grad_out
 * itself): grad_y[p] = w * grad_out[t]; grad_top_weights[t,k] = <grad_out[t],
 * y[inv_pos[t*K+k]]>. grad_out: (T,H) res_dtype; grad_y: (P,H) dtype. */
PMOE_API int pmoe_combine_residual_backward(const void* grad_out, int res_dtype, const void* y,
                                            const void* top_weights, int w_dtype, const int32_t* inv_pos, int dtype,
                                            int64_t T, int64_t K, int64_t H, void* grad_y, void* grad_top_weights,
                                            void* stream);

/* Backward of the dispatch, the RMSNorm and the residual add in one row pass
 * (autograd of qwen3_moe.py:281 through moe.py:104 and torch.nn.RMSNorm):
 *   g[t]      = grad_normed_add[t] + sum_k grad_x_perm[inv_pos[t*K+k]]  (dL/d norm output)
 *   grad_x[t] = grad_residual[t] + r_t * weight * g[t] - (r_t^3 / H) <g[t] * weight, x[t]> x[t]
 *   grad_weight = sum_t g[t] * x[t] * r_t  (fixed-order partial sums; deterministic)
 * grad_x_perm (T*K,H) and grad_normed_add (T,H) have dtype `dtype`; x,
 * grad_residual and grad_x are (T,H) x_dtype; weight and rstd (from
 * pmoe_rmsnorm_forward) fp32; grad_weight (H,) w_dtype. grad_x_perm,
 * grad_normed_add, grad_residual and grad_weight may each be NULL (no term /
 * not wanted). H <= 16384 (PMOE_ERR_UNSUPPORTED beyond): rows up to 4096 are
 * held in registers, wider ones walked twice (twice the grad_x_perm reads). */
PMOE_API size_t pmoe_dispatch_rmsnorm_backward_workspace_size(int64_t T, int64_t H);
PMOE_API int pmoe_dispatch_rmsnorm_backward(const void* grad_x_perm, const int32_t* inv_pos,
                                            const void* grad_normed_add, int dtype, const void* x, int x_dtype,
                                            const float* weight, const float* rstd, const void* grad_residual,
                                            int64_t T, int64_t K, int64_t H, void* grad_x, void* grad_weight,
                                            int w_dtype, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------ whole expert FFN ---
 * Replaces moe_expert_ffn / _expert_ffn_grouped (pluggy/kernels/moe.py:68-168):
 * permute, sort_rows, gate_up+SwiGLU over the gathered hidden rows with the
 * routing weight in the activation, down, and an unweighted combine. The
 * expert-sorted copy of hidden (moe.py:104) is never materialised. The saved
 * tensors (counts, offs, sorted_pair, inv_pos, sorted_token, sorted_w,
 * gate_up_out, mid) are caller-owned outputs that pmoe_expert_ffn_backward
 * consumes; y (P, H), the weighted expert rows, is only needed by the combine.
 * hidden (T,H), top_indices (T,K) int64, top_weights (T,K) w_dtype,
 * gate_up_proj (E,2I,H), down_proj (E,H,I), out (T,H); sorted_token (P,)
 * int32; sorted_w (P,) fp32; gate_up_out (P,2I), mid (P,I), y (P,H) dtype.
 * top_weights and sorted_w are required when T > 0 (the weights reach the
 * output only through sorted_w); NULL returns PMOE_ERR_INVALID before any
 * launch. */
PMOE_API size_t pmoe_expert_ffn_forward_workspace_size(int64_t T, int64_t K, int64_t E);
PMOE_API int pmoe_expert_ffn_forward(const void* hidden, const int64_t* top_indices, const void* top_weights,
                                     int w_dtype, const void* gate_up_proj, const void* down_proj, int dtype,
                                     int64_t T, int64_t K, int64_t E, int64_t H, int64_t I, void* out,
                                     int32_t* counts, int32_t* offs, int32_t* sorted_pair, int32_t* inv_pos,
                                     int32_t* sorted_token, float* sorted_w, void* gate_up_out, void* mid, void* y,
                                     void* workspace, size_t workspace_bytes, void* stream);

/* pmoe_expert_ffn_forward without the workspace arguments. No counterpart in
 * the reference: it is for callers that cannot allocate memory (code under HIP
 * graph capture, serving loops, harnesses that forbid allocation). The
 * permutation's scratch lives in a 256 KiB static device array, one per
 * device, so T*K <= 2048 * floor(65536 / E) pairs (PMOE_ERR_UNSUPPORTED
 * beyond; e.g. 1 048 576 pairs at E = 128). Outputs and saved tensors are the
 * caller's, as for pmoe_expert_ffn_forward. Calls that overlap on one device
 * share that array and race; calls on different devices do not. */
PMOE_API int pmoe_expert_ffn_forward_noalloc(const void* hidden, const int64_t* top_indices, const void* top_weights,
                                             int w_dtype, const void* gate_up_proj, const void* down_proj,
                                             int dtype, int64_t T, int64_t K, int64_t E, int64_t H, int64_t I,
                                             void* out, int32_t* counts, int32_t* offs, int32_t* sorted_pair,
                                             int32_t* inv_pos, int32_t* sorted_token, float* sorted_w,
                                             void* gate_up_out, void* mid, void* y, void* stream);

/* Autograd of pmoe_expert_ffn_forward from grad_out (T,H) dtype. Any of
 * grad_hidden, grad_top_weights (T,K) w_dtype, grad_gate_up_proj,
 * grad_down_proj may be NULL. grad_weight_dtype is the dtype of the two weight
 * gradients: `dtype`, or PMOE_F32 with 16-bit operands (fp32 master weights).
 * Workspace holds grad_gate_up_out, the sorted rows' input gradient and the
 * routing-weight partials. sorted_w (the forward's) is required when T > 0. */
PMOE_API size_t pmoe_expert_ffn_backward_workspace_size(int64_t T, int64_t K, int64_t H, int64_t I, int dtype);
PMOE_API int pmoe_expert_ffn_backward(const void* grad_out, const void* hidden, int w_dtype, const void* gate_up_proj,
                                      const void* down_proj, int dtype, int64_t T, int64_t K, int64_t E, int64_t H,
                                      int64_t I, const int32_t* offs, const int32_t* inv_pos,
                                      const int32_t* sorted_token, const float* sorted_w, const void* gate_up_out,
                                      const void* mid, void* grad_hidden, void* grad_top_weights,
                                      void* grad_gate_up_proj, void* grad_down_proj, int grad_weight_dtype,
                                      void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------- engine queries ---
 * No counterpart in the reference (which has no kernels of its own): which
 * tile the grouped-GEMM engine gives an expert GEMM, for tests and tuning.
 * kind: PMOE_GEMM_* below; dtype: the operands' (PMOE_BF16 and PMOE_F16 take the
 * persistent DMA engine: 32-row tiles for the forward GEMMs of few-token
 * batches, 128 or 256 otherwise; PMOE_F32 the register-staged one: 64 rows);
 * num_cus <= 0: the current device's compute units. Returns the tile's rows,
 * or a negative PMOE_ERR_* code. Host-only: launches nothing. */
enum {
  PMOE_GEMM_GATE_UP_FWD = 0,
  PMOE_GEMM_DOWN_FWD = 1,
  PMOE_GEMM_DOWN_DGRAD = 2,
  PMOE_GEMM_DOWN_WGRAD = 3,
  PMOE_GEMM_GATE_UP_DGRAD = 4,
  PMOE_GEMM_GATE_UP_WGRAD = 5
};
PMOE_API int pmoe_expert_gemm_tile_rows(int kind, int64_t P, int64_t E, int64_t H, int64_t I, int dtype,
                                        int num_cus);

#ifdef __cplusplus
}
#endif

#endif /* PMOE_H */
