// Internal launchers of the pmoe kernels (C++; the C ABI lives in api.hip).
// Every launcher enqueues on `s`, allocates nothing and never synchronises.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "common.h"

namespace pmoe {

// ---- grouped expert GEMMs (gemm.hip). T = bf16_t, f16_t or float
// (activation dtype); Tw: the weight gradients' type (EG_*_WGRAD; fp32 with
// 16-bit operands for fp32 master weights). offs: (E,) int32 inclusive end row of each
// expert in the sorted order. Operands per kind (see ExpertGemm): A, B, aux,
// C, C2 (gate_up forward: mid), Cw (weight gradients); xg: gathers and
// routing weights.
template <typename T, typename Tw>
hipError_t expert_gemm_run(int kind, const T* A, const T* B, const T* aux, T* C, T* C2, Tw* Cw, const int32_t* offs,
                           int P, int E, int H, int I, const ExpertGather& xg, hipStream_t s);

// Rows of the tiles expert_gemm_run gives GEMM `kind` (32, 128 or 256 for
// 16-bit operands, half = true; the register-staged engine's for fp32) on `cus`
// compute units (<= 0: the current device's).
int expert_gemm_tile_rows(int kind, int P, int E, int H, int I, bool half, int cus);

// ---- router GEMMs in fp32 arithmetic (gemm.hip). TX: x dtype, TW: router weight dtype.
template <typename TX, typename TW>
hipError_t router_logits_gemm(const TX* x, const TW* w, int T, int H, int E, float* logits, hipStream_t s);
// dx = dl . W   (dl: (T, ldl) fp32, columns >= E are ignored)
template <typename TX, typename TW>
hipError_t router_dx_gemm(const float* dl, int ldl, const TW* w, int T, int H, int E, TX* dx, hipStream_t s);
// partial[g] = dl[chunk g]^T . x[chunk g]  -> (splits, E, H) fp32
template <typename TX>
hipError_t router_dw_gemm(const float* dl, int ldl, const TX* x, int T, int H, int E, int split_chunk,
                          float* partial, hipStream_t s);

// ---- routing, permutation and row movement (route.hip).
// logits = the fixed-order sum of nsplit split-K planes (plane s of (t, e) at
// parts[s*split_stride + t*ldp + e]) plus the optional bias, then softmax /
// top-k / renormalisation and the per-block statistics of rows_per_block
// (<= 16) rows per block: four rows per wave when E <= 256 and rows_per_block
// is a multiple of 4, else one wave per row.
template <typename TW>
hipError_t router_topk(const float* parts, int nsplit, int64_t split_stride, int64_t ldp, float* logits,
                       const float* logit_bias, int T, int E, int K, int norm_topk, TW* top_w, int64_t* top_idx,
                       float* top_w_f32, float* blk_psum, float* blk_lse2, int* blk_counts, int rows_per_block,
                       hipStream_t s);
// fp32 w (n values) -> bf16 planes [lo; hi; mid] (planes 3) or [lo; hi; mid; hi] (planes 4).
hipError_t split_bf16x3(const float* w, int64_t n, int planes, bf16_t* out, hipStream_t s);
// parts (T, npieces*E) fp32 = x . [w3[0]; w3[1]; ...]^T: one GEMM over the stacked pieces, so x is
// read once; x (T,H) bf16, w3 (npieces,E,H) bf16. splits > 1: split-K over H
// into `splits` planes of (T, npieces*E) each.
hipError_t router_logits_bf16_pieces(const bf16_t* x, const bf16_t* w3, int npieces, int T, int H, int E,
                                     int splits, float* parts, hipStream_t s);
// parts (T, E) planes fp32 = x . w^T from fp16 x (T,H) and fp16 w (E,H), split-K as above.
hipError_t router_logits_f16(const f16_t* x, const f16_t* w, int T, int H, int E, int splits, float* parts,
                             hipStream_t s);
hipError_t router_stats_reduce(const float* blk_psum, const float* blk_lse2, const int* blk_counts, int nblk, int E,
                               float* prob_sum, float* lse_sq_sum, int32_t* counts, hipStream_t s);
// dl (T, ldl) fp32, or with dl3 != nullptr the bf16 planes [dl_hi | dl_hi | dl_lo] (T, 3*ldl),
// and with dl2 != nullptr also the fp16 planes [dl_hi | dl_lo] (T, 2*ldl).
template <typename TG>
hipError_t router_dlogits(const float* logits, const int64_t* top_idx, const float* top_w_f32, const TG* grad_w,
                          const float* grad_logits, int T, int E, int K, int norm_topk, float* dl, bf16_t* dl3,
                          f16_t* dl2, int ldl, hipStream_t s);
// w3t = [W_hi; W_mid; W_hi] with rows E..ldl-1 of each plane zero (3*ldl, H)
template <typename TW>
hipError_t split_router_weight_bwd(const TW* w, int E, int H, int ldl, bf16_t* w3t, hipStream_t s);
template <typename TO>
hipError_t router_dx_bf16(const bf16_t* dl3, int ldl, const bf16_t* w3t, int T, int H, TO* dx, hipStream_t s);
hipError_t router_dw_f16(const f16_t* dl2, int ldl, const f16_t* x, int T, int H, int E, int split_chunk,
                         float* partial, hipStream_t s);
hipError_t router_dw_bf16(const bf16_t* dl3, int ldl, const bf16_t* x, int T, int H, int E, int split_chunk,
                          float* partial, hipStream_t s);
template <typename TO>
hipError_t reduce_partials(const float* partial, int splits, int64_t n, TO* out, hipStream_t s);

template <typename TW>
hipError_t sort_rows(const int32_t* sorted_pair, const TW* w, int P, int K, int32_t* sorted_token, float* sorted_w,
                     hipStream_t s);
template <typename TG>
hipError_t pair_weight_grad(const float* part, int ld, int nparts, const int32_t* inv_pos, int P, TG* grad_w,
                            hipStream_t s);
hipError_t count_invalid_ids(const int64_t* idx, int64_t n, int64_t E, int32_t* count, hipStream_t s);
// Stable counting-sort permutation of the T*K pairs by expert; with
// sorted_token non-null it also writes the expert GEMMs' row tables
// (sorted_token[p] = sorted_pair[p] / K, sorted_w[p] = float(w[sorted_pair[p]]),
// w fp32, bf16 or fp16 for w_code 0, 1, 2; sorted_w may be null).
hipError_t permute_pairs(const int64_t* top_idx, int T, int K, int E, int32_t* counts, int32_t* offs,
                         int32_t* sorted_pair, int32_t* inv_pos, int32_t* chunk_hist, int chunk, hipStream_t s,
                         int32_t* sorted_token = nullptr, float* sorted_w = nullptr, const void* w = nullptr,
                         int w_code = 0);
template <typename T>
hipError_t dispatch_rows(const T* x, const int32_t* inv_pos, int T_, int K, int H, T* x_perm, hipStream_t s);
template <typename T, typename TW>
hipError_t combine_rows(const T* y, const TW* w, const int32_t* inv_pos, int T_, int K, int H, T* out,
                        hipStream_t s);
template <typename T, typename TW>
hipError_t combine_rows_bwd(const T* dout, const T* y, const TW* w, const int32_t* inv_pos, int T_, int K, int H,
                            T* dy, TW* dw, hipStream_t s);
template <typename T>
// dx = (add +) the K-sum; add (T_,H) may be NULL
hipError_t dispatch_rows_bwd(const T* dx_perm, const int32_t* inv_pos, const T* add, int T_, int K, int H, T* dx,
                             hipStream_t s);

// out = res + the weighted K-sum (the block's residual add fused into the combine)
template <typename T, typename TW, typename TR>
hipError_t combine_rows_residual(const T* y, const TW* w, const int32_t* inv_pos, const TR* res, int T_, int K, int H,
                                 TR* out, hipStream_t s);
// combine backward with the upstream gradient in its own dtype TD
template <typename T, typename TW, typename TD>
hipError_t combine_rows_residual_bwd(const TD* dout, const T* y, const TW* w, const int32_t* inv_pos, int T_, int K,
                                     int H, T* dy, TW* dw, hipStream_t s);

// ---- RMSNorm neighbours (norm.hip). w: (H,) fp32 norm weight; rstd: (T,) fp32.
template <typename TX, typename TO>
hipError_t rmsnorm_fwd(const TX* x, const float* w, float eps, int T_, int H, TO* out, float* rstd, hipStream_t s);
// gx = res + RMSNorm-backward(add + K-sum of gxp); gw_partial: (rmsnorm_bwd_blocks(T), H) fp32 or NULL.
template <typename T, typename TX>
hipError_t dispatch_rmsnorm_bwd(const T* gxp, const int32_t* inv_pos, const T* add, const TX* x, const float* w,
                                const float* rstd, const TX* res, int T_, int K, int H, TX* gx, float* gw_partial,
                                hipStream_t s);
// rows up to kRmsnormRegH are held in registers by the backward; wider rows
// (up to kRmsnormMaxH: two waves' norm-weight partials of 2 * H floats in LDS)
// are walked twice in chunks
constexpr int kRmsnormRegH = 4096;
constexpr int kRmsnormMaxH = 16384;
constexpr int kRmsnormBwdMaxBlocks = 1024;
int rmsnorm_bwd_blocks(int T_);
// Tall partial matrices (rows x n) are reduced in two passes: groups of
// kRowGroup rows into tmp (rmsnorm_bwd_groups(T) x n), then reduce_partials.
constexpr int kRowGroup = 32;
int rmsnorm_bwd_groups(int T_);
hipError_t sum_row_groups(const float* partial, int rows, int n, float* tmp, hipStream_t s);

// Chunk size (pairs) of the permutation histogram and the workspace it needs.
constexpr int kPermuteChunk = 2048;
// Most split-K planes of the bf16-pieces router logits GEMM (the top-k kernel
// loads all of a row's planes at once).
constexpr int kRouterMaxSplits = 8;
inline int64_t permute_chunks(int64_t P) { return (P + kPermuteChunk - 1) / kPermuteChunk; }

}  // namespace pmoe
