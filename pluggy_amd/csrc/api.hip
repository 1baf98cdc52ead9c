// C ABI of pmoe (declared in include/pmoe.h): argument checks, dtype dispatch,
// workspace carving and the multi-kernel sequences of each entry point.
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "../../include/pmoe.h"
#include "kernels.h"

using namespace pmoe;

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_status(hipError_t e, const char* where) {
  if (e == hipSuccess) return PMOE_OK;
  return fail((int)e, "%s: %s", where, hipGetErrorString(e));
}

#define PMOE_TRY(expr, where)                        \
  do {                                               \
    hipError_t e_ = (expr);                          \
    if (e_ != hipSuccess) return hip_status(e_, where); \
  } while (0)

#define PMOE_REQUIRE(cond, ...)                               \
  do {                                                        \
    if (!(cond)) return fail(PMOE_ERR_INVALID, __VA_ARGS__); \
  } while (0)

constexpr size_t kAlign = 256;
size_t align_up(size_t n) { return (n + kAlign - 1) / kAlign * kAlign; }

// Bump allocator over the caller's workspace.
struct Carver {
  char* base;
  size_t used = 0;
  explicit Carver(void* p) : base(static_cast<char*>(p)) {}
  template <typename T>
  T* take(size_t count) {
    T* p = reinterpret_cast<T*>(base + used);
    used += align_up(count * sizeof(T));
    return p;
  }
};

// The router, the RMSNorm neighbours and the residual combine take fp32 and
// bf16; the expert path (row tables, row movers, expert GEMMs) also fp16.
bool dtype_ok(int d) { return d == PMOE_F32 || d == PMOE_BF16; }
bool dtype16_ok(int d) { return dtype_ok(d) || d == PMOE_F16; }
// The router's (x, weight) pairings: each fp32 or bf16, both fp16, or bf16 x
// beside an fp32 weight given as its bf16 pieces (pmoe_router_split_weight).
bool router_pair_ok(int x, int w) {
  return (dtype_ok(x) && dtype_ok(w)) || (x == PMOE_F16 && w == PMOE_F16) || (x == PMOE_BF16 && w == PMOE_BF16X3);
}
size_t elem_bytes(int d) { return d == PMOE_F32 ? 4 : 2; }
hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Tokens per split-K chunk of the router weight-gradient GEMM (fp32 partials
// summed in order by reduce_partials).
constexpr int kRouterSplitChunk = 1024;
constexpr int64_t kMaxIndex = 0x7fffffffLL;

// Rows per block of the router top-k kernel: 16 when there are enough rows to
// fill the GPU, else 4 (a wave takes four rows for E <= 256, else one).
int router_rows(int64_t T) { return T >= 2048 ? 16 : 4; }
int64_t router_blocks(int64_t T) { return (T + router_rows(T) - 1) / router_rows(T); }
// Split-K planes of the router logits GEMM: its output tiles (128 x 128 for
// the three bf16 pieces of an fp32 weight, 64 x 64 for a bf16 weight) fall
// short of the 256 CUs unless tokens are many, so the reduction over H is
// split (chunks of at least 256) until there are about 256 blocks; the top-k
// kernel sums the planes in order.
int router_logit_splits(int64_t T, int64_t H, int64_t E, bool pieces) {
  if (T <= 0) return 1;
  const int64_t tiles = pieces ? ((T + 127) / 128) * ((E + 127) / 128) : ((T + 63) / 64) * ((E + 63) / 64);
  int64_t s = (256 + tiles - 1) / tiles;
  s = std::min<int64_t>(s, std::min<int64_t>(kRouterMaxSplits, std::max<int64_t>(1, H / 256)));
  return (int)std::max<int64_t>(1, s);
}
int64_t router_splits(int64_t T) { return std::max<int64_t>(1, (T + kRouterSplitChunk - 1) / kRouterSplitChunk); }
int64_t ldl_of(int64_t E) { return (E + 7) / 8 * 8; }

int check_moe_dims(int64_t T, int64_t K, int64_t E, int64_t H, int64_t I) {
  PMOE_REQUIRE(T >= 0 && H > 0 && E > 0 && K > 0, "sizes must be positive (T=%lld H=%lld E=%lld K=%lld)",
               (long long)T, (long long)H, (long long)E, (long long)K);
  PMOE_REQUIRE(K <= E, "top_k=%lld exceeds num_experts=%lld", (long long)K, (long long)E);
  PMOE_REQUIRE(E <= 1024, "num_experts=%lld > 1024 is not supported", (long long)E);
  PMOE_REQUIRE(K <= 64, "top_k=%lld > 64 is not supported", (long long)K);
  PMOE_REQUIRE(H % 8 == 0, "hidden size %lld must be a multiple of 8", (long long)H);
  PMOE_REQUIRE(I >= 0 && I % 8 == 0, "moe intermediate size %lld must be a multiple of 8", (long long)I);
  PMOE_REQUIRE(T * K <= kMaxIndex && T * K * std::max<int64_t>(H, 2 * I) <= (int64_t)1 << 40,
               "problem too large (T*K=%lld)", (long long)(T * K));
  return PMOE_OK;
}

// Calls f with a null pointer of the element type of a dtype code (fp32 or
// bf16; by_dtype16 also fp16).
template <class F>
hipError_t by_dtype(int code, F&& f) {
  if (code == PMOE_BF16) return f(static_cast<bf16_t*>(nullptr));
  return f(static_cast<float*>(nullptr));
}
template <class F>
hipError_t by_dtype16(int code, F&& f) {
  if (code == PMOE_F16) return f(static_cast<f16_t*>(nullptr));
  return by_dtype(code, f);
}
#define PMOE_ELEM(p) std::remove_pointer_t<decltype(p)>

}  // namespace

extern "C" {

PMOE_API const char* pmoe_version(void) { return "pmoe 0.1.0 gfx950"; }
PMOE_API const char* pmoe_last_error_string(void) { return g_err; }

// ------------------------------------------------------------------ router

PMOE_API size_t pmoe_router_forward_workspace_size(int64_t T, int64_t H, int64_t E) {
  const int64_t nb = router_blocks(T);
  return align_up(nb * E * sizeof(float)) + align_up(nb * E * sizeof(int)) + align_up(nb * sizeof(float)) +
         align_up(3 * E * H * sizeof(bf16_t)) +
         align_up(std::max(router_logit_splits(T, H, E, true), router_logit_splits(T, H, E, false)) * T * E *
                  sizeof(float));
}

PMOE_API int pmoe_router_forward(const void* x, int x_dtype, const void* weight, int w_dtype,
                                 const float* logit_bias, int64_t T, int64_t H, int64_t E, int64_t K,
                                 int norm_topk_prob, float* logits, void* top_weights, int tw_dtype,
                                 int64_t* top_indices, float* top_weights_f32, int32_t* expert_counts,
                                 float* prob_sum, float* lse_sq_sum, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  if (int rc = check_moe_dims(T, K, E, H, 0)) return rc;
  PMOE_REQUIRE(router_pair_ok(x_dtype, w_dtype) && dtype16_ok(tw_dtype),
               "router_forward: x and weight dtype codes must be PMOE_F32 or PMOE_BF16, both PMOE_F16, or "
               "PMOE_BF16 and PMOE_BF16X3");
  PMOE_REQUIRE(T == 0 || (x && weight && logits && top_weights && top_indices && top_weights_f32),
               "router_forward: null tensor");
  const size_t need = pmoe_router_forward_workspace_size(T, H, E);
  if (workspace_bytes < need || (need > 0 && !workspace))
    return fail(PMOE_ERR_WORKSPACE, "router_forward: workspace %zu < %zu bytes", workspace_bytes, need);
  hipStream_t s = as_stream(stream);
  const int t = (int)T, h = (int)H, e = (int)E, k = (int)K;
  Carver cv(workspace);
  const int64_t nb = router_blocks(T);
  float* blk_psum = cv.take<float>(nb * E);
  int* blk_cnt = cv.take<int>(nb * E);
  float* blk_lse2 = cv.take<float>(nb);
  bf16_t* w3 = cv.take<bf16_t>(3 * E * H);
  const bool pieces = x_dtype == PMOE_BF16 && (w_dtype == PMOE_F32 || w_dtype == PMOE_BF16X3);
  const int splits = router_logit_splits(T, H, E, pieces);
  float* parts = cv.take<float>(splits * T * E);
  // Logits in fp32 arithmetic. bf16 x: x is exact in bf16, so splitting an fp32
  // weight into three bf16 pieces makes every MFMA product exact; the GEMM's
  // epilogue adds the three pieces' fp32 accumulators in a fixed order, and the
  // top-k kernel sums the split-K planes in order. fp16 x and weight: fp16
  // products are exact in fp32, one piece on the fp16 MFMAs.
  const float* lparts = logits;
  int nsplit = 1;
  int64_t sstride = 0;
  if (T > 0) {
    if (x_dtype == PMOE_F16) {
      PMOE_TRY(router_logits_f16((const f16_t*)x, (const f16_t*)weight, t, h, e, splits, parts, s),
               "router logits GEMM");
      lparts = parts;
      nsplit = splits;
      sstride = (int64_t)T * E;
    } else if (x_dtype == PMOE_BF16) {
      const bf16_t* wb = (const bf16_t*)weight;
      int npieces = 1;
      if (w_dtype == PMOE_F32) {
        PMOE_TRY(split_bf16x3((const float*)weight, E * H, 3, w3, s), "router weight split");
        wb = w3;
        npieces = 3;
      } else if (w_dtype == PMOE_BF16X3) {
        npieces = 3;  // planes 0..2 of the caller's pieces
      }
      // the pieces are summed in the GEMM's epilogue: one (T, E) plane per split
      PMOE_TRY(router_logits_bf16_pieces((const bf16_t*)x, wb, npieces, t, h, e, splits, parts, s),
               "router logits GEMM");
      lparts = parts;
      nsplit = splits;
      sstride = (int64_t)T * E;
    } else {
      hipError_t st = w_dtype == PMOE_F32
                          ? router_logits_gemm<float, float>((const float*)x, (const float*)weight, t, h, e, logits, s)
                          : router_logits_gemm<float, bf16_t>((const float*)x, (const bf16_t*)weight, t, h, e, logits,
                                                              s);
      PMOE_TRY(st, "router logits GEMM");
    }
    hipError_t st = by_dtype16(tw_dtype, [&](auto wp) {
      typedef PMOE_ELEM(wp) W;
      return router_topk<W>(lparts, nsplit, sstride, E, logits, logit_bias, t, e, k, norm_topk_prob, (W*)top_weights,
                            top_indices, top_weights_f32, blk_psum, blk_lse2, blk_cnt, router_rows(T), s);
    });
    PMOE_TRY(st, "router top-k");
  }
  if (expert_counts || prob_sum || lse_sq_sum)
    PMOE_TRY(router_stats_reduce(blk_psum, blk_lse2, blk_cnt, (int)nb, e, prob_sum, lse_sq_sum, expert_counts, s),
             "router statistics");
  return PMOE_OK;
}

PMOE_API int pmoe_router_split_weight(const float* weight, int64_t E, int64_t H, void* pieces, void* stream) {
  if (int rc = check_moe_dims(1, 1, E, H, 0)) return rc;
  PMOE_REQUIRE(weight && pieces, "router_split_weight: null tensor");
  PMOE_TRY(split_bf16x3(weight, E * H, 4, (bf16_t*)pieces, as_stream(stream)), "router weight split");
  return PMOE_OK;
}

PMOE_API size_t pmoe_router_backward_workspace_size(int64_t T, int64_t H, int64_t E) {
  const int64_t ldl = ldl_of(E);
  const size_t fp32_path = align_up(T * ldl * sizeof(float)) + align_up(router_splits(T) * E * H * sizeof(float));
  const size_t bf16_path = align_up(T * 3 * ldl * sizeof(bf16_t)) + align_up(3 * ldl * H * sizeof(bf16_t)) +
                           align_up(2 * router_splits(T) * E * H * sizeof(float));
  const size_t f16_path = bf16_path + align_up(T * 2 * ldl * sizeof(f16_t));
  return std::max(fp32_path, f16_path);
}

PMOE_API int pmoe_router_backward(const void* x, int x_dtype, const void* weight, int w_dtype,
                                  const float* logits, const int64_t* top_indices, const float* top_weights_f32,
                                  const void* grad_top_weights, int gw_dtype, const float* grad_logits, int64_t T,
                                  int64_t H, int64_t E, int64_t K, int norm_topk_prob, void* grad_x,
                                  void* grad_weight, void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = check_moe_dims(T, K, E, H, 0)) return rc;
  PMOE_REQUIRE(router_pair_ok(x_dtype, w_dtype) && dtype16_ok(gw_dtype),
               "router_backward: x and weight dtype codes must be PMOE_F32 or PMOE_BF16, both PMOE_F16, or "
               "PMOE_BF16 and PMOE_BF16X3");
  PMOE_REQUIRE(w_dtype != PMOE_BF16X3 || E % 8 == 0,
               "router_backward: a weight given as pieces needs E a multiple of 8");
  PMOE_REQUIRE(T == 0 || (x && weight && logits && top_indices && top_weights_f32),
               "router_backward: null tensor");
  const size_t need = pmoe_router_backward_workspace_size(T, H, E);
  if (workspace_bytes < need || !workspace)
    return fail(PMOE_ERR_WORKSPACE, "router_backward: workspace %zu < %zu bytes", workspace_bytes, need);
  hipStream_t s = as_stream(stream);
  const int t = (int)T, h = (int)H, e = (int)E, k = (int)K;
  const int ldl = (int)ldl_of(E);
  const int splits = (int)router_splits(T);
  Carver cv(workspace);
  if (T == 0) {
    // no tokens: dW = 0, written by the reduction kernel over zero partial
    // planes (a kernel write, not hipMemsetAsync, so a captured graph replays it)
    if (grad_weight) {
      hipError_t st = by_dtype16(w_dtype == PMOE_BF16X3 ? PMOE_F32 : w_dtype, [&](auto wp) {
        typedef PMOE_ELEM(wp) W;
        return reduce_partials<W>(nullptr, 0, E * H, (W*)grad_weight, s);
      });
      PMOE_TRY(st, "router dW zero");
    }
    return PMOE_OK;
  }
  auto dlogits = [&](float* dl, bf16_t* dl3, f16_t* dl2) {
    return by_dtype16(gw_dtype, [&](auto gp) {
      typedef PMOE_ELEM(gp) G;
      return router_dlogits<G>(logits, top_indices, top_weights_f32, (const G*)grad_top_weights, grad_logits, t, e,
                               k, norm_topk_prob, dl, dl3, dl2, ldl, s);
    });
  };
  if (x_dtype == PMOE_F16) {
    // fp16 x and weight: dx from the bf16 planes of dl and the weight's bf16
    // pieces W = W_hi + W_lo (exact for fp16), as below; dW from fp16 planes
    // dl = dl_hi + dl_lo and the fp16 x on the fp16 MFMAs, every product exact.
    bf16_t* dl3 = cv.take<bf16_t>((size_t)T * 3 * ldl);
    bf16_t* w3t = cv.take<bf16_t>((size_t)3 * ldl * H);
    float* partial = cv.take<float>((size_t)2 * splits * E * H);
    f16_t* dl2 = cv.take<f16_t>((size_t)T * 2 * ldl);
    PMOE_TRY(dlogits(nullptr, dl3, grad_weight ? dl2 : nullptr), "router dlogits");
    if (grad_x) {
      PMOE_TRY(split_router_weight_bwd<f16_t>((const f16_t*)weight, e, h, ldl, w3t, s), "router weight split");
      PMOE_TRY(router_dx_bf16<f16_t>(dl3, ldl, w3t, t, h, (f16_t*)grad_x, s), "router dx GEMM");
    }
    if (grad_weight) {
      PMOE_TRY(router_dw_f16(dl2, ldl, (const f16_t*)x, t, h, e, kRouterSplitChunk, partial, s), "router dW GEMM");
      PMOE_TRY(reduce_partials<f16_t>(partial, 2 * splits, E * H, (f16_t*)grad_weight, s), "router dW reduce");
    }
    return PMOE_OK;
  }
  if (x_dtype == PMOE_BF16) {
    // bf16 x: dl is split into bf16 planes hi + lo; dx = [hi|hi|lo].[W_hi;W_mid;W_hi]
    // and dW = hi^T x + lo^T x, all products exact, fp32 accumulation.
    bf16_t* dl3 = cv.take<bf16_t>((size_t)T * 3 * ldl);
    bf16_t* w3t = cv.take<bf16_t>((size_t)3 * ldl * H);
    float* partial = cv.take<float>((size_t)2 * splits * E * H);
    PMOE_TRY(dlogits(nullptr, dl3, nullptr), "router dlogits");
    hipError_t st;
    if (grad_x) {
      const bf16_t* wt = w3t;
      if (w_dtype == PMOE_BF16X3) {
        wt = (const bf16_t*)weight + (size_t)E * H;  // planes 1..3 = [hi; mid; hi] (ldl == E)
      } else {
        st = w_dtype == PMOE_F32 ? split_router_weight_bwd<float>((const float*)weight, e, h, ldl, w3t, s)
                                 : split_router_weight_bwd<bf16_t>((const bf16_t*)weight, e, h, ldl, w3t, s);
        PMOE_TRY(st, "router weight split");
      }
      PMOE_TRY(router_dx_bf16<bf16_t>(dl3, ldl, wt, t, h, (bf16_t*)grad_x, s), "router dx GEMM");
    }
    if (grad_weight) {
      PMOE_TRY(router_dw_bf16(dl3, ldl, (const bf16_t*)x, t, h, e, kRouterSplitChunk, partial, s), "router dW GEMM");
      // an fp32 weight, whole or as pieces, gets its gradient in fp32
      st = w_dtype == PMOE_BF16 ? reduce_partials<bf16_t>(partial, 2 * splits, E * H, (bf16_t*)grad_weight, s)
                                : reduce_partials<float>(partial, 2 * splits, E * H, (float*)grad_weight, s);
      PMOE_TRY(st, "router dW reduce");
    }
    return PMOE_OK;
  }
  // fp32 x: fp32 MFMA GEMMs on the fp32 dl
  float* dl = cv.take<float>((size_t)T * ldl);
  float* partial = cv.take<float>((size_t)splits * E * H);
  PMOE_TRY(dlogits(dl, nullptr, nullptr), "router dlogits");
  hipError_t st;
  if (grad_x) {
    st = w_dtype == PMOE_F32
             ? router_dx_gemm<float, float>(dl, ldl, (const float*)weight, t, h, e, (float*)grad_x, s)
             : router_dx_gemm<float, bf16_t>(dl, ldl, (const bf16_t*)weight, t, h, e, (float*)grad_x, s);
    PMOE_TRY(st, "router dx GEMM");
  }
  if (grad_weight) {
    PMOE_TRY(router_dw_gemm<float>(dl, ldl, (const float*)x, t, h, e, kRouterSplitChunk, partial, s),
             "router dW GEMM");
    st = w_dtype == PMOE_BF16 ? reduce_partials<bf16_t>(partial, splits, E * H, (bf16_t*)grad_weight, s)
                              : reduce_partials<float>(partial, splits, E * H, (float*)grad_weight, s);
    PMOE_TRY(st, "router dW reduce");
  }
  return PMOE_OK;
}

// ------------------------------------------------------------- permutation

PMOE_API size_t pmoe_permute_workspace_size(int64_t T, int64_t K, int64_t E) {
  return align_up(std::max<int64_t>(1, permute_chunks(T * K)) * E * sizeof(int32_t));
}

PMOE_API int pmoe_permute(const int64_t* top_indices, int64_t T, int64_t K, int64_t E, int32_t* counts,
                          int32_t* offs, int32_t* sorted_pair, int32_t* inv_pos, void* workspace,
                          size_t workspace_bytes, void* stream) {
  if (int rc = check_moe_dims(T, K, E, 8, 0)) return rc;
  PMOE_REQUIRE(counts && offs && (T == 0 || (top_indices && sorted_pair && inv_pos)), "permute: null tensor");
  const size_t need = pmoe_permute_workspace_size(T, K, E);
  if (workspace_bytes < need || !workspace)
    return fail(PMOE_ERR_WORKSPACE, "permute: workspace %zu < %zu bytes", workspace_bytes, need);
  PMOE_TRY(permute_pairs(top_indices, (int)T, (int)K, (int)E, counts, offs, sorted_pair, inv_pos,
                         static_cast<int32_t*>(workspace), kPermuteChunk, as_stream(stream)),
           "permute");
  return PMOE_OK;
}

PMOE_API int pmoe_permute_rows(const int64_t* top_indices, const void* top_weights, int w_dtype, int64_t T,
                               int64_t K, int64_t E, int32_t* counts, int32_t* offs, int32_t* sorted_pair,
                               int32_t* inv_pos, int32_t* sorted_token, float* sorted_w, void* workspace,
                               size_t workspace_bytes, void* stream) {
  if (int rc = check_moe_dims(T, K, E, 8, 0)) return rc;
  PMOE_REQUIRE(dtype16_ok(w_dtype), "unknown dtype code");
  PMOE_REQUIRE(counts && offs &&
                   (T == 0 || (top_indices && sorted_pair && inv_pos && sorted_token && (!sorted_w || top_weights))),
               "permute_rows: null tensor");
  const size_t need = pmoe_permute_workspace_size(T, K, E);
  if (workspace_bytes < need || !workspace)
    return fail(PMOE_ERR_WORKSPACE, "permute_rows: workspace %zu < %zu bytes", workspace_bytes, need);
  PMOE_TRY(permute_pairs(top_indices, (int)T, (int)K, (int)E, counts, offs, sorted_pair, inv_pos,
                         static_cast<int32_t*>(workspace), kPermuteChunk, as_stream(stream), sorted_token, sorted_w,
                         top_weights, w_dtype == PMOE_BF16 ? 1 : w_dtype == PMOE_F16 ? 2 : 0),
           "permute_rows");
  return PMOE_OK;
}

PMOE_API int pmoe_count_invalid_ids(const int64_t* top_indices, int64_t n, int64_t E, int32_t* count,
                                    void* stream) {
  PMOE_REQUIRE(n >= 0 && E >= 1, "count_invalid_ids: n %lld, E %lld", (long long)n, (long long)E);
  PMOE_REQUIRE(count && (n == 0 || top_indices), "count_invalid_ids: null tensor");
  PMOE_TRY(count_invalid_ids(top_indices, n, E, count, as_stream(stream)), "count_invalid_ids");
  return PMOE_OK;
}

PMOE_API int pmoe_dispatch(const void* hidden, int dtype, const int32_t* inv_pos, int64_t T, int64_t K, int64_t H,
                           void* x_perm, void* stream) {
  if (int rc = check_moe_dims(T, K, K, H, 0)) return rc;
  PMOE_REQUIRE(dtype16_ok(dtype), "unknown dtype code");
  if (T == 0) return PMOE_OK;
  PMOE_REQUIRE(hidden && inv_pos && x_perm, "dispatch: null tensor");
  hipError_t st = by_dtype16(dtype, [&](auto tp) {
    typedef PMOE_ELEM(tp) E;
    return dispatch_rows<E>((const E*)hidden, inv_pos, (int)T, (int)K, (int)H, (E*)x_perm, as_stream(stream));
  });
  return hip_status(st, "dispatch");
}

PMOE_API int pmoe_dispatch_backward(const void* grad_x_perm, const int32_t* inv_pos, const void* grad_hidden_add,
                                    int dtype, int64_t T, int64_t K, int64_t H, void* grad_hidden, void* stream) {
  if (int rc = check_moe_dims(T, K, K, H, 0)) return rc;
  PMOE_REQUIRE(dtype16_ok(dtype), "unknown dtype code");
  if (T == 0) return PMOE_OK;
  PMOE_REQUIRE(grad_x_perm && inv_pos && grad_hidden, "dispatch_backward: null tensor");
  hipError_t st = by_dtype16(dtype, [&](auto tp) {
    typedef PMOE_ELEM(tp) E;
    return dispatch_rows_bwd<E>((const E*)grad_x_perm, inv_pos, (const E*)grad_hidden_add, (int)T, (int)K, (int)H,
                                (E*)grad_hidden, as_stream(stream));
  });
  return hip_status(st, "dispatch_backward");
}

// ------------------------------------------------------------ expert GEMMs

extern "C++" {
namespace {

// A gathered operand is addressed through one buffer descriptor, whose byte
// offsets are 32-bit: its storage must stay below 2 GiB.
int check_gather(const int32_t* index, int64_t rows, int64_t cols, int dtype, int64_t P, const char* what) {
  if (index == nullptr) {
    PMOE_REQUIRE(rows == P, "%s: without a row index the operand has the P = %lld sorted rows (got %lld)", what,
                 (long long)P, (long long)rows);
    return PMOE_OK;
  }
  PMOE_REQUIRE(rows > 0, "%s: a gathered operand needs rows > 0", what);
  const int64_t bytes = rows * cols * (int64_t)elem_bytes(dtype);
  if (bytes >= ((int64_t)1 << 31) - 16)
    return fail(PMOE_ERR_UNSUPPORTED, "%s: gathered operand of %lld bytes exceeds the 2 GiB a descriptor addresses",
                what, (long long)bytes);
  return PMOE_OK;
}

template <typename T, typename Tw>
hipError_t run_expert(int kind, const void* A, const void* B, const void* aux, void* C, void* C2, void* Cw,
                      const int32_t* offs, int64_t P, int64_t E, int64_t H, int64_t I, const ExpertGather& xg,
                      hipStream_t s) {
  return expert_gemm_run<T, Tw>(kind, (const T*)A, (const T*)B, (const T*)aux, (T*)C, (T*)C2, (Tw*)Cw, offs, (int)P,
                                (int)E, (int)H, (int)I, xg, s);
}

// dtype: the operands'; wdt: the weight gradient's (wgrad kinds).
hipError_t dispatch_expert(int kind, int dtype, int wdt, const void* A, const void* B, const void* aux, void* C,
                           void* C2, void* Cw, const int32_t* offs, int64_t P, int64_t E, int64_t H, int64_t I,
                           const ExpertGather& xg, hipStream_t s) {
  if (dtype == PMOE_F32) return run_expert<float, float>(kind, A, B, aux, C, C2, Cw, offs, P, E, H, I, xg, s);
  if (dtype == PMOE_F16) {
    if (wdt == PMOE_F32) return run_expert<f16_t, float>(kind, A, B, aux, C, C2, Cw, offs, P, E, H, I, xg, s);
    return run_expert<f16_t, f16_t>(kind, A, B, aux, C, C2, Cw, offs, P, E, H, I, xg, s);
  }
  if (wdt == PMOE_F32) return run_expert<bf16_t, float>(kind, A, B, aux, C, C2, Cw, offs, P, E, H, I, xg, s);
  return run_expert<bf16_t, bf16_t>(kind, A, B, aux, C, C2, Cw, offs, P, E, H, I, xg, s);
}

}  // namespace
}  // extern "C++"

PMOE_API int pmoe_sort_rows(const int32_t* sorted_pair, const void* top_weights, int w_dtype, int64_t T, int64_t K,
                            int32_t* sorted_token, float* sorted_w, void* stream) {
  PMOE_REQUIRE(T >= 0 && K > 0 && T * K <= kMaxIndex, "sort_rows: bad sizes");
  PMOE_REQUIRE(dtype16_ok(w_dtype), "unknown dtype code");
  if (T == 0) return PMOE_OK;
  PMOE_REQUIRE(sorted_pair && sorted_token && (sorted_w == nullptr || top_weights), "sort_rows: null tensor");
  const int P = (int)(T * K);
  hipError_t st = by_dtype16(w_dtype, [&](auto wp) {
    typedef PMOE_ELEM(wp) W;
    return sort_rows<W>(sorted_pair, (const W*)top_weights, P, (int)K, sorted_token, sorted_w, as_stream(stream));
  });
  return hip_status(st, "sort_rows");
}

PMOE_API int pmoe_gate_up_swiglu(const void* x, const int32_t* row_index, const float* row_weight, int64_t x_rows,
                                 const void* gate_up_proj, const int32_t* offs, int dtype, int64_t P, int64_t E,
                                 int64_t H, int64_t I, void* gate_up_out, void* mid, void* stream) {
  if (int rc = check_moe_dims(P, 1, E, H, I)) return rc;
  PMOE_REQUIRE(dtype16_ok(dtype) && I > 0, "gate_up_swiglu: bad dtype or I");
  if (int rc = check_gather(row_index, x_rows, H, dtype, P, "gate_up_swiglu")) return rc;
  if (P == 0) return PMOE_OK;
  PMOE_REQUIRE(x && gate_up_proj && offs && gate_up_out && mid, "gate_up_swiglu: null tensor");
  ExpertGather xg;
  xg.index = row_index;
  xg.rows = x_rows;
  xg.row_w = row_weight;
  PMOE_TRY(dispatch_expert(EG_GATE_UP_FWD, dtype, dtype, x, gate_up_proj, nullptr, gate_up_out, mid, nullptr, offs, P,
                           E, H, I, xg, as_stream(stream)),
           "gate_up_swiglu");
  return PMOE_OK;
}

PMOE_API int pmoe_down_proj(const void* mid, const void* down_proj, const int32_t* offs, int dtype, int64_t P,
                            int64_t E, int64_t H, int64_t I, void* y, void* stream) {
  if (int rc = check_moe_dims(P, 1, E, H, I)) return rc;
  PMOE_REQUIRE(dtype16_ok(dtype) && I > 0, "down_proj: bad dtype or I");
  if (P == 0) return PMOE_OK;
  PMOE_REQUIRE(mid && down_proj && offs && y, "down_proj: null tensor");
  PMOE_TRY(dispatch_expert(EG_DOWN_FWD, dtype, dtype, mid, down_proj, nullptr, y, nullptr, nullptr, offs, P, E, H, I,
                           ExpertGather(), as_stream(stream)),
           "down_proj");
  return PMOE_OK;
}

PMOE_API int pmoe_down_proj_backward(const void* grad, const int32_t* row_index, const float* row_weight,
                                     int64_t grad_rows, const void* mid, const void* gate_up_out,
                                     const void* down_proj, const int32_t* offs, int dtype, int64_t P, int64_t E,
                                     int64_t H, int64_t I, void* grad_gate_up_out, void* grad_down_proj,
                                     int grad_weight_dtype, float* part, int64_t part_ld, void* stream) {
  if (int rc = check_moe_dims(P, 1, E, H, I)) return rc;
  PMOE_REQUIRE(dtype16_ok(dtype) && I > 0, "down_proj_backward: bad dtype or I");
  PMOE_REQUIRE(grad_weight_dtype == dtype || (dtype != PMOE_F32 && grad_weight_dtype == PMOE_F32),
               "down_proj_backward: grad_down_proj dtype must be the operands' or fp32");
  if (int rc = check_gather(row_index, grad_rows, H, dtype, P, "down_proj_backward")) return rc;
  PMOE_REQUIRE(part == nullptr || (row_weight != nullptr && part_ld >= (I + 63) / 64),
               "down_proj_backward: routing-weight partials need row_weight and part_ld >= ceil(I / 64)");
  PMOE_REQUIRE(offs && (P == 0 || grad), "down_proj_backward: null tensor");
  hipStream_t s = as_stream(stream);
  ExpertGather xg;
  xg.index = row_index;
  xg.rows = grad_rows;
  if (grad_gate_up_out && P > 0) {
    PMOE_REQUIRE(down_proj && gate_up_out, "down_proj_backward: null tensor");
    ExpertGather xd = xg;
    xd.row_w = row_weight;
    xd.part = part;
    xd.part_ld = (int)part_ld;
    PMOE_TRY(dispatch_expert(EG_DOWN_DGRAD, dtype, dtype, grad, down_proj, gate_up_out, grad_gate_up_out, nullptr,
                             nullptr, offs, P, E, H, I, xd, s),
             "down dgrad");
  } else {
    PMOE_REQUIRE(part == nullptr, "down_proj_backward: routing-weight partials come with grad_gate_up_out");
  }
  if (grad_down_proj) {
    PMOE_REQUIRE(P == 0 || mid, "down_proj_backward: null mid");
    PMOE_TRY(dispatch_expert(EG_DOWN_WGRAD, dtype, grad_weight_dtype, grad, mid, nullptr, nullptr, nullptr,
                             grad_down_proj, offs, P, E, H, I, xg, s),
             "down wgrad");
  }
  return PMOE_OK;
}

PMOE_API int pmoe_gate_up_backward(const void* grad_gate_up_out, const void* x, const int32_t* row_index,
                                   int64_t x_rows, const void* gate_up_proj, const int32_t* offs, int dtype, int64_t P,
                                   int64_t E, int64_t H, int64_t I, void* grad_x_perm, void* grad_gate_up_proj,
                                   int grad_weight_dtype, void* stream) {
  if (int rc = check_moe_dims(P, 1, E, H, I)) return rc;
  PMOE_REQUIRE(dtype16_ok(dtype) && I > 0, "gate_up_backward: bad dtype or I");
  PMOE_REQUIRE(grad_weight_dtype == dtype || (dtype != PMOE_F32 && grad_weight_dtype == PMOE_F32),
               "gate_up_backward: grad_gate_up_proj dtype must be the operands' or fp32");
  if (int rc = check_gather(row_index, x_rows, H, dtype, P, "gate_up_backward")) return rc;
  PMOE_REQUIRE(offs && (P == 0 || grad_gate_up_out), "gate_up_backward: null tensor");
  hipStream_t s = as_stream(stream);
  if (grad_x_perm && P > 0) {
    PMOE_REQUIRE(gate_up_proj, "gate_up_backward: null weight");
    PMOE_TRY(dispatch_expert(EG_GATE_UP_DGRAD, dtype, dtype, grad_gate_up_out, gate_up_proj, nullptr, grad_x_perm,
                             nullptr, nullptr, offs, P, E, H, I, ExpertGather(), s),
             "gate_up dgrad");
  }
  if (grad_gate_up_proj) {
    PMOE_REQUIRE(P == 0 || x, "gate_up_backward: null x");
    ExpertGather xg;
    xg.index = row_index;
    xg.rows = x_rows;
    PMOE_TRY(dispatch_expert(EG_GATE_UP_WGRAD, dtype, grad_weight_dtype, grad_gate_up_out, x, nullptr, nullptr,
                             nullptr, grad_gate_up_proj, offs, P, E, H, I, xg, s),
             "gate_up wgrad");
  }
  return PMOE_OK;
}

PMOE_API int pmoe_pair_weight_grad(const float* part, int64_t part_ld, int64_t nparts, const int32_t* inv_pos,
                                   int64_t T, int64_t K, void* grad_top_weights, int gw_dtype, void* stream) {
  PMOE_REQUIRE(T >= 0 && K > 0 && T * K <= kMaxIndex && nparts >= 0 && part_ld >= nparts && part_ld < (1 << 20),
               "pair_weight_grad: bad sizes");
  PMOE_REQUIRE(dtype16_ok(gw_dtype), "unknown dtype code");
  if (T == 0) return PMOE_OK;
  PMOE_REQUIRE(part && inv_pos && grad_top_weights, "pair_weight_grad: null tensor");
  const int P = (int)(T * K);
  hipError_t st = by_dtype16(gw_dtype, [&](auto gp) {
    typedef PMOE_ELEM(gp) G;
    return pair_weight_grad<G>(part, (int)part_ld, (int)nparts, inv_pos, P, (G*)grad_top_weights, as_stream(stream));
  });
  return hip_status(st, "pair_weight_grad");
}

// ---------------------------------------------------------------- combine

PMOE_API int pmoe_combine(const void* y, const void* top_weights, int w_dtype, const int32_t* inv_pos, int dtype,
                          int64_t T, int64_t K, int64_t H, void* out, void* stream) {
  if (int rc = check_moe_dims(T, K, K, H, 0)) return rc;
  PMOE_REQUIRE(dtype16_ok(dtype) && dtype16_ok(w_dtype), "unknown dtype code");
  if (T == 0) return PMOE_OK;
  PMOE_REQUIRE(y && inv_pos && out, "combine: null tensor");  // top_weights NULL: unit weights
  hipStream_t s = as_stream(stream);
  const int t = (int)T, k = (int)K, h = (int)H;
  hipError_t st = by_dtype16(dtype, [&](auto yp) {
    return by_dtype16(w_dtype, [&](auto wp) {
      typedef PMOE_ELEM(yp) Y;
      typedef PMOE_ELEM(wp) W;
      return combine_rows<Y, W>((const Y*)y, (const W*)top_weights, inv_pos, t, k, h, (Y*)out, s);
    });
  });
  return hip_status(st, "combine");
}

PMOE_API int pmoe_combine_backward(const void* grad_out, const void* y, const void* top_weights, int w_dtype,
                                   const int32_t* inv_pos, int dtype, int64_t T, int64_t K, int64_t H,
                                   void* grad_y, void* grad_top_weights, void* stream) {
  if (int rc = check_moe_dims(T, K, K, H, 0)) return rc;
  PMOE_REQUIRE(dtype16_ok(dtype) && dtype16_ok(w_dtype), "unknown dtype code");
  if (T == 0) return PMOE_OK;
  PMOE_REQUIRE(grad_out && y && top_weights && inv_pos && grad_y && grad_top_weights,
               "combine_backward: null tensor");
  hipStream_t s = as_stream(stream);
  const int t = (int)T, k = (int)K, h = (int)H;
  hipError_t st = by_dtype16(dtype, [&](auto yp) {
    return by_dtype16(w_dtype, [&](auto wp) {
      typedef PMOE_ELEM(yp) Y;
      typedef PMOE_ELEM(wp) W;
      return combine_rows_bwd<Y, W>((const Y*)grad_out, (const Y*)y, (const W*)top_weights, inv_pos, t, k, h,
                                    (Y*)grad_y, (W*)grad_top_weights, s);
    });
  });
  return hip_status(st, "combine_backward");
}

// ------------------------------------------------------- whole expert FFN

PMOE_API size_t pmoe_expert_ffn_forward_workspace_size(int64_t T, int64_t K, int64_t E) {
  return pmoe_permute_workspace_size(T, K, E);
}

PMOE_API int pmoe_expert_ffn_forward(const void* hidden, const int64_t* top_indices, const void* top_weights,
                                     int w_dtype, const void* gate_up_proj, const void* down_proj, int dtype,
                                     int64_t T, int64_t K, int64_t E, int64_t H, int64_t I, void* out,
                                     int32_t* counts, int32_t* offs, int32_t* sorted_pair, int32_t* inv_pos,
                                     int32_t* sorted_token, float* sorted_w, void* gate_up_out, void* mid, void* y,
                                     void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = check_moe_dims(T, K, E, H, I)) return rc;
  PMOE_REQUIRE(I > 0 && dtype16_ok(dtype) && dtype16_ok(w_dtype), "expert_ffn_forward: bad dtype or I");
  // The routing weights reach the output only through sorted_w (the SwiGLU
  // epilogue scales each sorted row by it; the combine is unweighted), so both
  // are required: without them the sum would silently be unweighted.
  PMOE_REQUIRE(T == 0 || (top_weights && sorted_w),
               "expert_ffn_forward: top_weights and sorted_w are required (the routing weights enter through "
               "sorted_w)");
  if (int rc = pmoe_permute_rows(top_indices, top_weights, w_dtype, T, K, E, counts, offs, sorted_pair, inv_pos,
                                 sorted_token, sorted_w, workspace, workspace_bytes, stream))
    return rc;
  if (T == 0) return PMOE_OK;
  const int64_t P = T * K;
  if (int rc = pmoe_gate_up_swiglu(hidden, sorted_token, sorted_w, T, gate_up_proj, offs, dtype, P, E, H, I,
                                   gate_up_out, mid, stream))
    return rc;
  if (int rc = pmoe_down_proj(mid, down_proj, offs, dtype, P, E, H, I, y, stream)) return rc;
  return pmoe_combine(y, nullptr, w_dtype, inv_pos, dtype, T, K, H, out, stream);
}

// ---- the whole-FFN forward without a workspace argument
//
// For callers that cannot allocate (code under HIP graph capture, serving
// loops, harnesses that forbid allocation): the permutation's chunk
// histograms, the only scratch memory of pmoe_expert_ffn_forward, live in a
// file-scope device array of kStaticScratchBytes. Each device holds its own
// copy until the process ends; its address is looked up once per device, with
// that device current, on the entry point's first call there. Every call on a
// device shares the array, so calls that overlap on one device race.
// Nothing in it has to start at zero: the histogram kernel writes every
// (chunk, expert) entry before the scan reads it.
constexpr size_t kStaticScratchBytes = 256 * 1024;
__device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

namespace {

constexpr int kMaxScratchDevices = 64;
std::once_flag g_scratch_once[kMaxScratchDevices];
void* g_scratch_ptr[kMaxScratchDevices];
hipError_t g_scratch_err[kMaxScratchDevices];

// Device address of `scratch` on the current device (the host-side name is
// only a stand-in and must never reach a kernel).
hipError_t static_scratch(void** out) {
  int dev = 0;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxScratchDevices) return hipErrorInvalidDevice;
  std::call_once(g_scratch_once[dev], [dev] {
    void* p = nullptr;
    g_scratch_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_scratch_ptr[dev] = g_scratch_err[dev] == hipSuccess ? p : nullptr;
  });
  if (g_scratch_err[dev] != hipSuccess) return g_scratch_err[dev];
  if (g_scratch_ptr[dev] == nullptr) return hipErrorInvalidSymbol;
  *out = g_scratch_ptr[dev];
  return hipSuccess;
}

}  // namespace

PMOE_API int pmoe_expert_ffn_forward_noalloc(const void* hidden, const int64_t* top_indices, const void* top_weights,
                                             int w_dtype, const void* gate_up_proj, const void* down_proj,
                                             int dtype, int64_t T, int64_t K, int64_t E, int64_t H, int64_t I,
                                             void* out, int32_t* counts, int32_t* offs, int32_t* sorted_pair,
                                             int32_t* inv_pos, int32_t* sorted_token, float* sorted_w,
                                             void* gate_up_out, void* mid, void* y, void* stream) {
  if (int rc = check_moe_dims(T, K, E, H, I)) return rc;
  PMOE_REQUIRE(T == 0 || (top_weights && sorted_w),
               "expert_ffn_forward_noalloc: top_weights and sorted_w are required (the routing weights enter "
               "through sorted_w)");
  const size_t need = pmoe_expert_ffn_forward_workspace_size(T, K, E);
  if (need > kStaticScratchBytes)
    return fail(PMOE_ERR_UNSUPPORTED,
                "expert_ffn_forward_noalloc: T*K = %lld pairs over %lld experts need %zu bytes of scratch; the "
                "static maximum is %zu (ceil(T*K / %d) * E * 4 bytes)",
                (long long)(T * K), (long long)E, need, kStaticScratchBytes, kPermuteChunk);
  void* ws = nullptr;
  PMOE_TRY(static_scratch(&ws), "expert_ffn_forward_noalloc: static scratch address");
  return pmoe_expert_ffn_forward(hidden, top_indices, top_weights, w_dtype, gate_up_proj, down_proj, dtype, T, K, E,
                                 H, I, out, counts, offs, sorted_pair, inv_pos, sorted_token, sorted_w, gate_up_out,
                                 mid, y, ws, kStaticScratchBytes, stream);
}

PMOE_API size_t pmoe_expert_ffn_backward_workspace_size(int64_t T, int64_t K, int64_t H, int64_t I, int dtype) {
  const size_t es = elem_bytes(dtype);
  const int64_t P = T * K;
  return align_up((size_t)P * 2 * I * es) + align_up((size_t)P * H * es) +
         align_up((size_t)P * ((I + 63) / 64) * sizeof(float));
}

PMOE_API int pmoe_expert_ffn_backward(const void* grad_out, const void* hidden, int w_dtype, const void* gate_up_proj,
                                      const void* down_proj, int dtype, int64_t T, int64_t K, int64_t E, int64_t H,
                                      int64_t I, const int32_t* offs, const int32_t* inv_pos,
                                      const int32_t* sorted_token, const float* sorted_w, const void* gate_up_out,
                                      const void* mid, void* grad_hidden, void* grad_top_weights,
                                      void* grad_gate_up_proj, void* grad_down_proj, int grad_weight_dtype,
                                      void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = check_moe_dims(T, K, E, H, I)) return rc;
  PMOE_REQUIRE(dtype16_ok(dtype) && dtype16_ok(w_dtype) && I > 0, "expert_ffn_backward: bad dtype or I");
  PMOE_REQUIRE(grad_weight_dtype == dtype || (dtype != PMOE_F32 && grad_weight_dtype == PMOE_F32),
               "expert_ffn_backward: weight gradient dtype must be the operands' or fp32");
  // sorted_w scales the gradient of every sorted row (the forward's weighted
  // rows); without it every gradient would be that of the unweighted sum
  PMOE_REQUIRE(T == 0 || sorted_w, "expert_ffn_backward: sorted_w (the routing weight of each sorted row) is required");
  const size_t need = pmoe_expert_ffn_backward_workspace_size(T, K, H, I, dtype);
  if (workspace_bytes < need || (need > 0 && !workspace))
    return fail(PMOE_ERR_WORKSPACE, "expert_ffn_backward: workspace %zu < %zu bytes", workspace_bytes, need);
  const int64_t P = T * K;
  const size_t es = elem_bytes(dtype);
  Carver c(workspace);
  void* g_gu = c.take<char>((size_t)P * 2 * I * es);
  void* g_xp = c.take<char>((size_t)P * H * es);
  const int64_t part_ld = (I + 63) / 64;
  float* part = c.take<float>((size_t)P * part_ld);
  const bool need_rows = grad_hidden != nullptr;
  const bool need_tw = grad_top_weights != nullptr;
  const bool need_dgu = need_rows || need_tw || grad_gate_up_proj != nullptr;
  if (T > 0 && need_dgu) {
    if (int rc = pmoe_down_proj_backward(grad_out, sorted_token, sorted_w, T, mid, gate_up_out, down_proj, offs, dtype,
                                         P, E, H, I, g_gu, nullptr, grad_weight_dtype, need_tw ? part : nullptr,
                                         part_ld, stream))
      return rc;
  }
  if (need_tw && T > 0) {
    if (int rc = pmoe_pair_weight_grad(part, part_ld, part_ld, inv_pos, T, K, grad_top_weights, w_dtype, stream))
      return rc;
  }
  if (need_rows) {
    if (int rc = pmoe_gate_up_backward(g_gu, hidden, sorted_token, T, gate_up_proj, offs, dtype, P, E, H, I, g_xp,
                                       nullptr, grad_weight_dtype, stream))
      return rc;
    if (int rc = pmoe_dispatch_backward(g_xp, inv_pos, nullptr, dtype, T, K, H, grad_hidden, stream)) return rc;
  }
  if (grad_gate_up_proj) {
    if (int rc = pmoe_gate_up_backward(g_gu, hidden, sorted_token, T, gate_up_proj, offs, dtype, P, E, H, I, nullptr,
                                       grad_gate_up_proj, grad_weight_dtype, stream))
      return rc;
  }
  if (grad_down_proj) {
    if (int rc = pmoe_down_proj_backward(grad_out, sorted_token, sorted_w, T, mid, gate_up_out, down_proj, offs,
                                         dtype, P, E, H, I, nullptr, grad_down_proj, grad_weight_dtype, nullptr, 0,
                                         stream))
      return rc;
  }
  return PMOE_OK;
}

// ------------------------------------------------------- engine queries

PMOE_API int pmoe_expert_gemm_tile_rows(int kind, int64_t P, int64_t E, int64_t H, int64_t I, int dtype,
                                        int num_cus) {
  PMOE_REQUIRE(kind >= EG_GATE_UP_FWD && kind <= EG_GATE_UP_WGRAD, "expert_gemm_tile_rows: unknown kind %d", kind);
  PMOE_REQUIRE(dtype16_ok(dtype), "unknown dtype code");
  PMOE_REQUIRE(P >= 0 && P <= kMaxIndex && E >= 1 && E <= 1024 && H > 0 && I > 0 && H <= INT32_MAX && I <= INT32_MAX,
               "expert_gemm_tile_rows: bad sizes");
  return expert_gemm_tile_rows(kind, (int)P, (int)E, (int)H, (int)I, dtype != PMOE_F32, num_cus);
}

// ------------------------------------------------------- block neighbours

PMOE_API int pmoe_rmsnorm_forward(const void* x, int x_dtype, const float* weight, float eps, int64_t T, int64_t H,
                                  void* out, int out_dtype, float* rstd, void* stream) {
  PMOE_REQUIRE(T >= 0 && H > 0 && H % 8 == 0 && T <= kMaxIndex, "rmsnorm_forward: bad sizes T=%lld H=%lld",
               (long long)T, (long long)H);
  PMOE_REQUIRE(dtype_ok(x_dtype) && dtype_ok(out_dtype),
               "rmsnorm_forward: dtype codes must be PMOE_F32 or PMOE_BF16");
  PMOE_REQUIRE(eps >= 0.0f, "rmsnorm_forward: eps must be non-negative");
  if (T == 0) return PMOE_OK;
  PMOE_REQUIRE(x && weight && out && rstd, "rmsnorm_forward: null tensor");
  hipError_t st = by_dtype(x_dtype, [&](auto xp) {
    return by_dtype(out_dtype, [&](auto op) {
      return rmsnorm_fwd<PMOE_ELEM(xp), PMOE_ELEM(op)>(static_cast<const PMOE_ELEM(xp)*>(x), weight, eps, (int)T,
                                                       (int)H, static_cast<PMOE_ELEM(op)*>(out), rstd,
                                                       as_stream(stream));
    });
  });
  return hip_status(st, "rmsnorm_forward");
}

PMOE_API int pmoe_combine_residual(const void* y, const void* top_weights, int w_dtype, const int32_t* inv_pos,
                                   int dtype, const void* residual, int res_dtype, int64_t T, int64_t K, int64_t H,
                                   void* out, void* stream) {
  if (int rc = check_moe_dims(T, K, K, H, 0)) return rc;
  PMOE_REQUIRE(dtype_ok(dtype) && dtype_ok(w_dtype) && dtype_ok(res_dtype),
               "combine_residual: dtype codes must be PMOE_F32 or PMOE_BF16");
  if (T == 0) return PMOE_OK;
  PMOE_REQUIRE(y && inv_pos && residual && out, "combine_residual: null tensor");  // top_weights NULL: unit weights
  hipError_t st = by_dtype(dtype, [&](auto yp) {
    return by_dtype(w_dtype, [&](auto wp) {
      return by_dtype(res_dtype, [&](auto rp) {
        return combine_rows_residual<PMOE_ELEM(yp), PMOE_ELEM(wp), PMOE_ELEM(rp)>(
            static_cast<const PMOE_ELEM(yp)*>(y), static_cast<const PMOE_ELEM(wp)*>(top_weights), inv_pos,
            static_cast<const PMOE_ELEM(rp)*>(residual), (int)T, (int)K, (int)H, static_cast<PMOE_ELEM(rp)*>(out),
            as_stream(stream));
      });
    });
  });
  return hip_status(st, "combine_residual");
}

PMOE_API int pmoe_combine_residual_backward(const void* grad_out, int res_dtype, const void* y,
                                            const void* top_weights, int w_dtype, const int32_t* inv_pos, int dtype,
                                            int64_t T, int64_t K, int64_t H, void* grad_y, void* grad_top_weights,
                                            void* stream) {
  if (int rc = check_moe_dims(T, K, K, H, 0)) return rc;
  PMOE_REQUIRE(dtype_ok(dtype) && dtype_ok(w_dtype) && dtype_ok(res_dtype),
               "combine_residual_backward: dtype codes must be PMOE_F32 or PMOE_BF16");
  if (T == 0) return PMOE_OK;
  PMOE_REQUIRE(grad_out && y && top_weights && inv_pos && grad_y && grad_top_weights,
               "combine_residual_backward: null tensor");
  hipError_t st = by_dtype(dtype, [&](auto yp) {
    return by_dtype(w_dtype, [&](auto wp) {
      return by_dtype(res_dtype, [&](auto rp) {
        return combine_rows_residual_bwd<PMOE_ELEM(yp), PMOE_ELEM(wp), PMOE_ELEM(rp)>(
            static_cast<const PMOE_ELEM(rp)*>(grad_out), static_cast<const PMOE_ELEM(yp)*>(y),
            static_cast<const PMOE_ELEM(wp)*>(top_weights), inv_pos, (int)T, (int)K, (int)H,
            static_cast<PMOE_ELEM(yp)*>(grad_y), static_cast<PMOE_ELEM(wp)*>(grad_top_weights), as_stream(stream));
      });
    });
  });
  return hip_status(st, "combine_residual_backward");
}

PMOE_API size_t pmoe_dispatch_rmsnorm_backward_workspace_size(int64_t T, int64_t H) {
  if (T <= 0 || H <= 0 || T > kMaxIndex) return 0;
  return align_up((size_t)rmsnorm_bwd_blocks((int)T) * (size_t)H * sizeof(float)) +
         align_up((size_t)rmsnorm_bwd_groups((int)T) * (size_t)H * sizeof(float));
}

PMOE_API int pmoe_dispatch_rmsnorm_backward(const void* grad_x_perm, const int32_t* inv_pos,
                                            const void* grad_normed_add, int dtype, const void* x, int x_dtype,
                                            const float* weight, const float* rstd, const void* grad_residual,
                                            int64_t T, int64_t K, int64_t H, void* grad_x, void* grad_weight,
                                            int w_dtype, void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = check_moe_dims(T, K, K, H, 0)) return rc;
  PMOE_REQUIRE(dtype_ok(dtype) && dtype_ok(x_dtype) && dtype_ok(w_dtype),
               "dispatch_rmsnorm_backward: dtype codes must be PMOE_F32 or PMOE_BF16");
  if (H > kRmsnormMaxH)
    return fail(PMOE_ERR_UNSUPPORTED, "dispatch_rmsnorm_backward: hidden size %lld > %d", (long long)H,
                kRmsnormMaxH);
  if (T == 0) return PMOE_OK;
  PMOE_REQUIRE(x && weight && rstd && grad_x, "dispatch_rmsnorm_backward: null tensor");
  PMOE_REQUIRE(!grad_x_perm || inv_pos, "dispatch_rmsnorm_backward: grad_x_perm without inv_pos");
  const size_t need = grad_weight ? pmoe_dispatch_rmsnorm_backward_workspace_size(T, H) : 0;
  if (workspace_bytes < need || (need > 0 && !workspace))
    return fail(PMOE_ERR_WORKSPACE, "dispatch_rmsnorm_backward: workspace %zu < %zu bytes", workspace_bytes, need);
  hipStream_t s = as_stream(stream);
  Carver cv(workspace);
  const int nb = rmsnorm_bwd_blocks((int)T), ng = rmsnorm_bwd_groups((int)T);
  float* partial = grad_weight ? cv.take<float>((size_t)nb * H) : nullptr;
  float* grouped = grad_weight ? cv.take<float>((size_t)ng * H) : nullptr;
  hipError_t st = by_dtype(dtype, [&](auto gp) {
    return by_dtype(x_dtype, [&](auto xp) {
      using TX = PMOE_ELEM(xp);
      return dispatch_rmsnorm_bwd<PMOE_ELEM(gp), TX>(
          static_cast<const PMOE_ELEM(gp)*>(grad_x_perm), inv_pos, static_cast<const PMOE_ELEM(gp)*>(grad_normed_add),
          static_cast<const TX*>(x), weight, rstd, static_cast<const TX*>(grad_residual), (int)T, (int)K, (int)H,
          static_cast<TX*>(grad_x), partial, s);
    });
  });
  PMOE_TRY(st, "dispatch_rmsnorm_backward");
  if (grad_weight) {
    PMOE_TRY(sum_row_groups(partial, nb, (int)H, grouped, s), "dispatch_rmsnorm_backward (weight)");
    st = w_dtype == PMOE_BF16 ? reduce_partials<bf16_t>(grouped, ng, H, static_cast<bf16_t*>(grad_weight), s)
                              : reduce_partials<float>(grouped, ng, H, static_cast<float*>(grad_weight), s);
    PMOE_TRY(st, "dispatch_rmsnorm_backward (weight)");
  }
  return PMOE_OK;
}

}  // extern "C"
