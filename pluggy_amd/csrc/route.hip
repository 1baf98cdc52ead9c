// Router top-k, routing statistics, the stable expert permutation, and the
// HBM-bound row movers (dispatch gather, weighted combine and their backward).
#include <limits.h>

#include <algorithm>
#include <type_traits>

#include "kernels.h"

namespace pmoe {

namespace {

__device__ __forceinline__ float nan_to_neg_inf(float v) { return v != v ? -INFINITY : v; }

// Top-k ranks larger logits first, equal logits -> lower expert id. Keys are
// the logits mapped to ints in the same order (-0 folded into +0, so the two
// zeros tie as they do as floats), so a wave-wide max is an integer max.
__device__ __forceinline__ int rank_key(float v) {
  const int b = __float_as_int(v + 0.0f);
  return b >= 0 ? b : b ^ 0x7fffffff;
}
__device__ __forceinline__ float key_value(int k) { return __int_as_float(k >= 0 ? k : k ^ 0x7fffffff); }

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int dpp_max(int v) {
  return max(v, __builtin_amdgcn_update_dpp(v, v, CTRL, ROW_MASK, 0xf, false));
}

// Max over the 64 lanes in six DPP steps (no LDS round trips): pairs, quads,
// half rows, rows, then rows 1 and 3 take lane 15 of the row before, rows 2
// and 3 take lane 31; lane 63 ends with the total.
__device__ __forceinline__ int wave_max_dpp(int v) {
  v = dpp_max<0xB1, 0xf>(v);   // quad_perm [1,0,3,2]
  v = dpp_max<0x4E, 0xf>(v);   // quad_perm [2,3,0,1]
  v = dpp_max<0x141, 0xf>(v);  // row_half_mirror
  v = dpp_max<0x140, 0xf>(v);  // row_mirror
  v = dpp_max<0x142, 0xa>(v);  // row_bcast:15
  v = dpp_max<0x143, 0xc>(v);  // row_bcast:31
  return __builtin_amdgcn_readlane(v, 63);
}

// fmaxf over the 64 lanes by the same DPP steps (fmaxf is order-free: the
// result equals the butterfly's, NaN lanes ignored as fmaxf ignores them).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_fmax(float v) {
  return fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, ROW_MASK,
                                                             0xf, false)));
}
__device__ __forceinline__ float wave_fmax_dpp(float v) {
  v = dpp_fmax<0xB1, 0xf>(v);
  v = dpp_fmax<0x4E, 0xf>(v);
  v = dpp_fmax<0x141, 0xf>(v);
  v = dpp_fmax<0x140, 0xf>(v);
  v = dpp_fmax<0x142, 0xa>(v);
  v = dpp_fmax<0x143, 0xc>(v);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// One wave per row. EPL = experts per lane (E <= 64 * EPL).
// W (E*H fp32) -> bf16 planes [lo; hi; mid] (and with planes == 4 a second
// hi after them) with hi + mid + lo == W to within 2^-24 relative (each
// residual is exact in fp32). The logits GEMM reads planes 0..2; the input
// gradient's GEMM reads planes 1..3 = [hi; mid; hi] against dl's bf16 planes
// [dl_hi | dl_hi | dl_lo].
__global__ void split_bf16x3_kernel(const float* __restrict__ w, int64_t n, int planes, bf16_t* __restrict__ out) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const float v = w[i];
    const bf16_t hi = f32_to_bf16(v);
    const float r1 = v - bf16_to_f32(hi);
    const bf16_t mid = f32_to_bf16(r1);
    const float r2 = r1 - bf16_to_f32(mid);
    out[i] = f32_to_bf16(r2);
    out[n + i] = hi;
    out[2 * n + i] = mid;
    if (planes == 4) out[3 * n + i] = hi;
  }
}

// Router top-k, one wave per row (the block's waves take consecutive rows).
// The logits of (row, e) are the in-order sum of nsplit split-K planes, plane
// sp at parts[sp * split_stride + row * ldp + e], plus the optional bias;
// parts may alias logits (nsplit 1, no bias: nothing is written back). Every
// plane's loads of a row are issued before the first is used (addresses are
// clamped into the row, so no lane branches), so a row costs one memory
// latency whatever nsplit is.
constexpr int kMaxSplits = kRouterMaxSplits;
template <int EPL, typename TW>
__global__ __launch_bounds__(1024) void router_topk_kernel(const float* __restrict__ parts, int nsplit,
                                                           int64_t split_stride, int64_t ldp, float* logits,
                                                           const float* __restrict__ bias,
                                                           int T, int E, int K, int norm_topk, TW* __restrict__ top_w,
                                                           int64_t* __restrict__ top_idx, float* __restrict__ top_w_f32,
                                                           float* __restrict__ blk_psum, float* __restrict__ blk_lse2,
                                                           int* __restrict__ blk_counts) {
  extern __shared__ float sh[];  // [NW][E] psum partials, then [E] int counts, then [NW] lse2
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nw = blockDim.x >> 6;
  float* s_psum = sh;
  int* s_cnt = reinterpret_cast<int*>(sh + nw * E);
  float* s_lse2 = sh + (nw + 1) * E;
  for (int e = tid; e < E; e += blockDim.x) s_cnt[e] = 0;
  __syncthreads();

  float psum[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) psum[j] = 0.0f;
  float lse2 = 0.0f;
  const int row = blockIdx.x * nw + wave;
  if (row < T) {
    // ---- logits of the row (the loads of up to 4 lane slots in one batch)
    constexpr int JB = EPL < 4 ? EPL : 4;
    const bool write_logits = nsplit > 1 || bias != nullptr || parts != logits;
    float v[EPL];
#pragma unroll
    for (int j0 = 0; j0 < EPL; j0 += JB) {
      float pl[kMaxSplits][JB];
#pragma unroll
      for (int sp = 0; sp < kMaxSplits; ++sp) {
        if (sp < nsplit) {  // uniform
#pragma unroll
          for (int jj = 0; jj < JB; ++jj)
            pl[sp][jj] = parts[sp * split_stride + (int64_t)row * ldp + min(lane + 64 * (j0 + jj), E - 1)];
        }
      }
#pragma unroll
      for (int jj = 0; jj < JB; ++jj) {
        const int e = lane + 64 * (j0 + jj);
        float x = pl[0][jj];
#pragma unroll
        for (int sp = 1; sp < kMaxSplits; ++sp)
          if (sp < nsplit) x += pl[sp][jj];
        if (bias != nullptr) x += bias[min(e, E - 1)];
        if (e < E && write_logits) logits[(int64_t)row * E + e] = x;
        v[j0 + jj] = e < E ? x : -INFINITY;
      }
    }
    // ---- softmax statistics
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < EPL; ++j) m = fmaxf(m, v[j]);
    m = wave_fmax_dpp(m);
    float ex[EPL];
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      ex[j] = (lane + 64 * j < E) ? expf(v[j] - m) : 0.0f;
      s += ex[j];
    }
    s = wave_sum(s);
    const float inv_s = 1.0f / s;
    const float lse = m + logf(s);
    lse2 = lse * lse;  // every lane holds the same value; lane 0's copy is used
#pragma unroll
    for (int j = 0; j < EPL; ++j) psum[j] = ex[j] * inv_s;

    // ---- top-k by (logit desc, id asc); NaN ranks as -inf so a valid id is
    // always found. Each pick: the wave max of the unpicked keys, then the
    // lowest id holding it (ballot over each lane slot in id order). Lane k
    // keeps pick k's logit; the probabilities follow the loop.
    int key[EPL];
#pragma unroll
    for (int j = 0; j < EPL; ++j) key[j] = rank_key(nan_to_neg_inf(v[j]));
    unsigned selmask = 0;
    float v_sel = -INFINITY;
    int e_sel = 0;
    for (int k = 0; k < K; ++k) {
      int lm = INT_MIN;
#pragma unroll
      for (int j = 0; j < EPL; ++j)
        if (lane + 64 * j < E && !((selmask >> j) & 1u)) lm = max(lm, key[j]);
      const int km = wave_max_dpp(lm);
      int be = -1;
#pragma unroll
      for (int j = 0; j < EPL; ++j) {
        const unsigned long long hit = __ballot(lane + 64 * j < E && !((selmask >> j) & 1u) && key[j] == km);
        if (be < 0 && hit != 0ull) be = 64 * j + __builtin_ctzll(hit);
      }
      if ((be & 63) == lane) selmask |= 1u << (be >> 6);
      if (lane == k) { v_sel = key_value(km); e_sel = be; }
    }
    // p of each pick on its own lane; their sum in pick order
    const float p_sel = lane < K ? expf(v_sel - m) * inv_s : 0.0f;
    float psum_sel = 0.0f;
    for (int k = 0; k < K; ++k)
      psum_sel += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p_sel), k));
    if (lane < K) {
      const float w = norm_topk ? p_sel / psum_sel : p_sel;
      const int64_t o = (int64_t)row * K + lane;
      top_idx[o] = e_sel;
      top_w_f32[o] = w;
      store_scalar<TW>(top_w + o, w);
      atomicAdd(&s_cnt[e_sel], 1);
    }
  }
  // fixed-order block reduction of the statistics (deterministic)
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = lane + 64 * j;
    if (e < E) s_psum[wave * E + e] = psum[j];
  }
  if (lane == 0) s_lse2[wave] = lse2;
  __syncthreads();
  for (int e = tid; e < E; e += blockDim.x) {
    float t = s_psum[e];
    for (int w = 1; w < nw; ++w) t += s_psum[w * E + e];
    blk_psum[(int64_t)blockIdx.x * E + e] = t;
    blk_counts[(int64_t)blockIdx.x * E + e] = s_cnt[e];
  }
  if (tid == 0) {
    float t = s_lse2[0];
    for (int w = 1; w < nw; ++w) t += s_lse2[w];
    blk_lse2[blockIdx.x] = t;
  }
}

// Reductions over one 16-lane DPP row (every lane of the row ends with the
// result; each step pairs lanes symmetrically, so all lanes hold the same
// bits): pairs, quads, half rows (row_half_mirror), the row (row_mirror).
__device__ __forceinline__ int row16_max(int v) {
  v = dpp_max<0xB1, 0xf>(v);
  v = dpp_max<0x4E, 0xf>(v);
  v = dpp_max<0x141, 0xf>(v);
  return dpp_max<0x140, 0xf>(v);
}
__device__ __forceinline__ float row16_fmax(float v) {
  v = dpp_fmax<0xB1, 0xf>(v);
  v = dpp_fmax<0x4E, 0xf>(v);
  v = dpp_fmax<0x141, 0xf>(v);
  return dpp_fmax<0x140, 0xf>(v);
}
template <int CTRL>
__device__ __forceinline__ float dpp_fadd(float v) {
  return v + __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float row16_sum(float v) {
  v = dpp_fadd<0xB1>(v);
  v = dpp_fadd<0x4E>(v);
  v = dpp_fadd<0x141>(v);
  return dpp_fadd<0x140>(v);
}

// Router top-k with four rows per wave: each 16-lane DPP row of the wave takes
// one token row, lane li holding experts li*V .. li*V+V-1 (E <= 16 V). The
// same results as router_topk_kernel (logits, ids, top weights, statistics),
// with the row reductions in 4 DPP steps instead of 6 and one ballot per pick:
// lower lanes hold lower ids, so the lowest lane of the row whose local
// maximum equals the row's maximum owns the pick (its lowest slot holding that
// key). Blocks of NWB waves take 4 NWB consecutive rows. VEC: E, ldp and
// split_stride multiples of 4 and V of 4, so a lane's loads and logit stores
// are 16-byte vectors. The sums of the softmax run in the DPP butterfly's
// fixed order.
template <int V, bool VEC, typename TW>
__global__ __launch_bounds__(256) void router_topk16_kernel(const float* __restrict__ parts, int nsplit,
                                                            int64_t split_stride, int64_t ldp, float* logits,
                                                            const float* __restrict__ bias, int T, int E, int K,
                                                            int norm_topk, TW* __restrict__ top_w,
                                                            int64_t* __restrict__ top_idx,
                                                            float* __restrict__ top_w_f32,
                                                            float* __restrict__ blk_psum,
                                                            float* __restrict__ blk_lse2,
                                                            int* __restrict__ blk_counts) {
  static_assert(!VEC || V % 4 == 0, "16-byte lane slices");
  // LDS: [R][E] psum partials, [E] counts, [R] lse2, then per row K picks (id, p)
  extern __shared__ float sh[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nwb = blockDim.x >> 6;
  const int R = 4 * nwb;  // rows of the block
  const int li = lane & 15, rg = lane >> 4;
  const int rb = wave * 4 + rg;  // row within the block
  float* s_psum = sh;
  int* s_cnt = reinterpret_cast<int*>(sh + R * E);
  float* s_lse2 = sh + (R + 1) * E;
  int* s_pid = reinterpret_cast<int*>(sh + (R + 1) * E + R);
  float* s_pp = sh + (R + 1) * E + R + R * K;
  for (int e = tid; e < E; e += blockDim.x) s_cnt[e] = 0;
  __syncthreads();

  const int row = blockIdx.x * R + rb;
  const bool live = row < T;
  const int64_t rowc = live ? row : T - 1;  // dead rows read a live row and write nothing
  const bool write_logits = nsplit > 1 || bias != nullptr || parts != logits;
  const int e0 = li * V;

  // ---- logits of the lane's V experts: every plane's loads, then the in-order sums
  float v[V];
  {
    float acc[V];
    if constexpr (VEC) {
      // chunks past E read the row's last chunk (E >= 4), whose values are masked below
      float4 pl[kMaxSplits][V / 4];
#pragma unroll
      for (int sp = 0; sp < kMaxSplits; ++sp)
        if (sp < nsplit) {
#pragma unroll
          for (int c = 0; c < V / 4; ++c) {
            const int ec = min(e0 + 4 * c, E - 4);
            pl[sp][c] = *reinterpret_cast<const float4*>(parts + sp * split_stride + rowc * ldp + ec);
          }
        }
#pragma unroll
      for (int c = 0; c < V / 4; ++c) {
        float4 x = pl[0][c];
#pragma unroll
        for (int sp = 1; sp < kMaxSplits; ++sp)
          if (sp < nsplit) {
            x.x += pl[sp][c].x; x.y += pl[sp][c].y; x.z += pl[sp][c].z; x.w += pl[sp][c].w;
          }
        acc[4 * c] = x.x; acc[4 * c + 1] = x.y; acc[4 * c + 2] = x.z; acc[4 * c + 3] = x.w;
      }
    } else {
      float pl[kMaxSplits][V];
#pragma unroll
      for (int sp = 0; sp < kMaxSplits; ++sp)
        if (sp < nsplit) {
#pragma unroll
          for (int j = 0; j < V; ++j) pl[sp][j] = parts[sp * split_stride + rowc * ldp + min(e0 + j, E - 1)];
        }
#pragma unroll
      for (int j = 0; j < V; ++j) {
        float x = pl[0][j];
#pragma unroll
        for (int sp = 1; sp < kMaxSplits; ++sp)
          if (sp < nsplit) x += pl[sp][j];
        acc[j] = x;
      }
    }
    if (bias != nullptr) {
#pragma unroll
      for (int j = 0; j < V; ++j) acc[j] += bias[min(e0 + j, E - 1)];
    }
    if (live && write_logits && e0 < E) {
      float* lrow = logits + (int64_t)row * E;
      if constexpr (VEC) {
#pragma unroll
        for (int c = 0; c < V / 4; ++c)
          if (e0 + 4 * c < E)
            *reinterpret_cast<float4*>(lrow + e0 + 4 * c) =
                make_float4(acc[4 * c], acc[4 * c + 1], acc[4 * c + 2], acc[4 * c + 3]);
      } else {
#pragma unroll
        for (int j = 0; j < V; ++j)
          if (e0 + j < E) lrow[e0 + j] = acc[j];
      }
    }
#pragma unroll
    for (int j = 0; j < V; ++j) v[j] = e0 + j < E ? acc[j] : -INFINITY;
  }

  // ---- softmax statistics of the row
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < V; ++j) m = fmaxf(m, v[j]);
  m = row16_fmax(m);
  float ex[V];
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < V; ++j) {
    ex[j] = e0 + j < E ? expf(v[j] - m) : 0.0f;
    s += ex[j];
  }
  s = row16_sum(s);
  const float inv_s = 1.0f / s;
  const float lse = m + logf(s);

  // ---- top-k by (logit desc, id asc); NaN ranks as -inf, picked and padding
  // slots hold INT_MIN (below every logit's key), so K <= E picks find valid ids
  int key[V];
#pragma unroll
  for (int j = 0; j < V; ++j) key[j] = e0 + j < E ? rank_key(nan_to_neg_inf(v[j])) : INT_MIN;
  int* pid = s_pid + rb * K;
  float* pp = s_pp + rb * K;
  for (int k = 0; k < K; ++k) {
    int lm = key[0];
#pragma unroll
    for (int j = 1; j < V; ++j) lm = max(lm, key[j]);
    const int km = row16_max(lm);
    const unsigned long long hit = __ballot(lm == km);
    const unsigned mrow = (unsigned)(hit >> (16 * rg)) & 0xffffu;
    const bool owner = li == __builtin_ctz(mrow);
    // the owner's lowest slot holding the key
    int jsel = V - 1;
#pragma unroll
    for (int j = V - 2; j >= 0; --j)
      if (key[j] == km) jsel = j;
#pragma unroll
    for (int j = 0; j < V; ++j)
      if (owner && j == jsel) key[j] = INT_MIN;
    if (owner) {
      pid[k] = e0 + jsel;
      pp[k] = expf(key_value(km) - m) * inv_s;
    }
  }
  // the picks' probabilities summed in pick order (every lane of the row alike)
  __syncthreads();
  float psum_sel = 0.0f;
  for (int k = 0; k < K; ++k) psum_sel += pp[k];
  if (live) {
    for (int k = li; k < K; k += 16) {
      const int e = pid[k];
      const float p = pp[k];
      const float w = norm_topk ? p / psum_sel : p;
      const int64_t o = (int64_t)row * K + k;
      top_idx[o] = e;
      top_w_f32[o] = w;
      store_scalar<TW>(top_w + o, w);
      atomicAdd(&s_cnt[e], 1);
    }
  }
  // ---- fixed-order block reduction of the statistics (deterministic)
#pragma unroll
  for (int j = 0; j < V; ++j)
    if (e0 + j < E) s_psum[rb * E + e0 + j] = live ? ex[j] * inv_s : 0.0f;
  if (li == 0) s_lse2[rb] = live ? lse * lse : 0.0f;
  __syncthreads();
  for (int e = tid; e < E; e += blockDim.x) {
    float t = s_psum[e];
    for (int r = 1; r < R; ++r) t += s_psum[r * E + e];
    blk_psum[(int64_t)blockIdx.x * E + e] = t;
    blk_counts[(int64_t)blockIdx.x * E + e] = s_cnt[e];
  }
  if (tid == 0) {
    float t = s_lse2[0];
    for (int r = 1; r < R; ++r) t += s_lse2[r];
    blk_lse2[blockIdx.x] = t;
  }
}

// One wave per expert (and one more for the lse^2 total): lane l sums the
// partials b = l, l + 64, ... in order, then a fixed butterfly combines lanes,
// so the result is the same on every run.
__global__ __launch_bounds__(256) void router_stats_reduce_kernel(const float* blk_psum, const float* blk_lse2,
                                                                  const int* blk_counts, int nblk, int E,
                                                                  float* prob_sum, float* lse_sq_sum,
                                                                  int32_t* counts) {
  const int lane = threadIdx.x & 63;
  const int e = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (e > E) return;
  if (e == E) {
    float l = 0.0f;
    for (int b = lane; b < nblk; b += 64) l += blk_lse2[b];
    l = wave_sum(l);
    if (lane == 0 && lse_sq_sum) *lse_sq_sum = l;
    return;
  }
  float ps = 0.0f;
  int c = 0;
  for (int b = lane; b < nblk; b += 64) {
    ps += blk_psum[(int64_t)b * E + e];
    c += blk_counts[(int64_t)b * E + e];
  }
  ps = wave_sum(ps);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) c += __shfl_xor(c, o, kWave);
  if (lane == 0) {
    if (prob_sum) prob_sum[e] = ps;
    if (counts) counts[e] = c;
  }
}

// d(loss)/d(logits) for one row per wave. See the closed forms in kernels.h users.
template <int EPL, typename TG>
__global__ __launch_bounds__(256) void router_dlogits_kernel(const float* __restrict__ logits,
                                                             const int64_t* __restrict__ top_idx,
                                                             const float* __restrict__ top_w_f32,
                                                             const TG* __restrict__ grad_w,
                                                             const float* __restrict__ grad_logits, int T, int E,
                                                             int K, int norm_topk, float* __restrict__ dl,
                                                             bf16_t* __restrict__ dl3, f16_t* __restrict__ dl2,
                                                             int ldl) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= T) return;
  // lane k < K holds slot k's expert, weight and upstream gradient (one load
  // each, all lanes at once); the slot loops below read them with readlane
  const bool slot = lane < K;
  const int64_t so = (int64_t)row * K + lane;
  const int e_l = slot ? (int)top_idx[so] : 0;
  const float w_l = slot ? top_w_f32[so] : 0.0f;
  const float g_l = (slot && grad_w != nullptr) ? load_scalar<TG>(grad_w + so) : 0.0f;
  auto rd = [](float v, int k) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), k)); };
  // inner = sum_k w_k G_k, in slot order
  float inner = 0.0f;
  if (grad_w != nullptr)
    for (int k = 0; k < K; ++k) inner += rd(w_l, k) * rd(g_l, k);
  float d[EPL];
  if (norm_topk) {
#pragma unroll
    for (int j = 0; j < EPL; ++j) d[j] = 0.0f;
    if (grad_w != nullptr) {
      const float val_l = w_l * (g_l - inner);
      for (int k = 0; k < K; ++k) {
        const int e = __builtin_amdgcn_readlane(e_l, k);
        const float val = rd(val_l, k);
        if ((e & 63) == lane) {
#pragma unroll
          for (int j = 0; j < EPL; ++j)
            if ((e >> 6) == j) d[j] = val;
        }
      }
    }
  } else {
    const float* lrow = logits + (int64_t)row * E;
    float v[EPL];
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const int e = lane + 64 * j;
      v[j] = e < E ? lrow[e] : -INFINITY;
      m = fmaxf(m, v[j]);
    }
    m = wave_max(m);
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      v[j] = (lane + 64 * j < E) ? expf(v[j] - m) : 0.0f;
      s += v[j];
    }
    s = wave_sum(s);
    const float inv_s = 1.0f / s;
#pragma unroll
    for (int j = 0; j < EPL; ++j) d[j] = -v[j] * inv_s * inner;
    if (grad_w != nullptr) {
      for (int k = 0; k < K; ++k) {
        const int e = __builtin_amdgcn_readlane(e_l, k);
        const float g = rd(g_l, k);
        if ((e & 63) == lane) {
#pragma unroll
          for (int j = 0; j < EPL; ++j)
            if ((e >> 6) == j) d[j] += v[j] * inv_s * g;
        }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = lane + 64 * j;
    float val = 0.0f;
    if (e < E) {
      val = d[j];
      if (grad_logits != nullptr) val += grad_logits[(int64_t)row * E + e];
    }
    if (e < ldl) {
      if (dl3 == nullptr) {
        dl[(int64_t)row * ldl + e] = val;
      } else {
        // val = hi + lo to 2^-16 relative; hi appears twice so that
        // [hi | hi | lo] . [W_hi; W_mid; W_hi] = dl . W to that precision.
        const bf16_t hi = f32_to_bf16(val);
        const bf16_t lo = f32_to_bf16(val - bf16_to_f32(hi));
        bf16_t* o = dl3 + (int64_t)row * 3 * ldl;
        o[e] = hi;
        o[ldl + e] = hi;
        o[2 * ldl + e] = lo;
      }
      if (dl2 != nullptr) {
        // fp16 planes for the fp16 weight gradient: val = hi + lo to 2^-22
        // relative for |val| >= 2^-3 (lo normal) and to 2^-25 absolute below;
        // fp16's range, as the fp16 dl of an fp16 linear layer has (an
        // overflow gives hi = inf and lo = 0, not inf - inf)
        const f16_t hi = (f16_t)val;
        const float hf = (float)hi;
        f16_t* o = dl2 + (int64_t)row * 2 * ldl;
        o[e] = hi;
        o[ldl + e] = (f16_t)(__builtin_isinf(hf) ? 0.0f : val - hf);
      }
    }
  }
  for (int e = 64 * EPL + lane; e < ldl; e += 64) {
    if (dl3 == nullptr) {
      dl[(int64_t)row * ldl + e] = 0.0f;
    } else {
      bf16_t* o = dl3 + (int64_t)row * 3 * ldl;
      o[e] = o[ldl + e] = o[2 * ldl + e] = 0;
    }
    if (dl2 != nullptr) {
      f16_t* o = dl2 + (int64_t)row * 2 * ldl;
      o[e] = o[ldl + e] = (f16_t)0.0f;
    }
  }
}

// w3t = [W_hi; W_mid; W_hi] (3*ldl, H), W_mid = bf16(W - W_hi), rows E..ldl-1
// of each plane zero: the input gradient's GEMM operand against dl's planes
// [dl_hi | dl_hi | dl_lo] (planes 1..3 of split_bf16x3's four-plane form).
template <typename TW>
__global__ void split_router_weight_bwd_kernel(const TW* __restrict__ w, int E, int H, int ldl,
                                               bf16_t* __restrict__ w3t) {
  const int64_t n = (int64_t)ldl * H;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int e = (int)(i / H);
    const float v = e < E ? load_scalar<TW>(w + i) : 0.0f;
    const bf16_t hi = f32_to_bf16(v);
    w3t[i] = hi;
    w3t[n + i] = f32_to_bf16(v - bf16_to_f32(hi));
    w3t[2 * n + i] = hi;
  }
}

template <typename TO>
__global__ void reduce_partials_kernel(const float* __restrict__ partial, int splits, int64_t n, TO* __restrict__ out) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    float acc = 0.0f;
    for (int g = 0; g < splits; ++g) acc += partial[(int64_t)g * n + i];
    store_scalar<TO>(out + i, acc);
  }
}

// The same sums, four consecutive values per thread (n a multiple of 4): 16-byte
// loads, four planes' loads issued before their adds; each value still sums
// the planes in order, so the result is the scalar kernel's bit for bit.
template <typename TO>
__global__ void reduce_partials4_kernel(const float* __restrict__ partial, int splits, int64_t n,
                                        TO* __restrict__ out) {
  const int64_t n4 = n / 4;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (int64_t)gridDim.x * blockDim.x) {
    const f32x4* src = reinterpret_cast<const f32x4*>(partial) + i;
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    int g = 0;
    for (; g + 4 <= splits; g += 4) {
      f32x4 v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = src[(int64_t)(g + j) * n4];
#pragma unroll
      for (int j = 0; j < 4; ++j) acc += v[j];
    }
    for (; g < splits; ++g) acc += src[(int64_t)g * n4];
#pragma unroll
    for (int j = 0; j < 4; ++j) store_scalar<TO>(out + 4 * i + j, acc[j]);
  }
}

// ---- permutation: stable counting sort of the P = T*K pairs by expert id

__device__ __forceinline__ int clamp_expert(int64_t e, int E) {
  return e < 0 ? 0 : (e >= E ? E - 1 : (int)e);
}

__global__ __launch_bounds__(256) void permute_hist_kernel(const int64_t* __restrict__ idx, int P, int E, int chunk,
                                                           int32_t* __restrict__ chunk_hist) {
  extern __shared__ int s_hist[];
  for (int e = threadIdx.x; e < E; e += blockDim.x) s_hist[e] = 0;
  __syncthreads();
  const int q0 = blockIdx.x * chunk;
  const int q1 = min(P, q0 + chunk);
  for (int q = q0 + threadIdx.x; q < q1; q += blockDim.x) atomicAdd(&s_hist[clamp_expert(idx[q], E)], 1);
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += blockDim.x) chunk_hist[(int64_t)blockIdx.x * E + e] = s_hist[e];
}

// One block of 1024 threads: per-expert scan over chunks, then an exclusive
// scan over experts. chunk_hist becomes the global base of (chunk, expert).
// TPE threads share an expert; thread s of expert e takes a contiguous run of
// chunks, so each pass is TPE independent streams of coalesced loads rather
// than one dependent chain over all chunks.
__global__ __launch_bounds__(1024) void permute_scan_kernel(int32_t* __restrict__ chunk_hist, int nchunks, int E,
                                                            int32_t* __restrict__ counts, int32_t* __restrict__ offs) {
  __shared__ int s_part[1024];
  __shared__ int s_tot[1024];
  __shared__ int s_wsum[16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int tpe = 1;
  while (tpe * 2 * E <= 1024) tpe *= 2;  // threads per expert (E <= 1024)
  const int e = tid / tpe, sub = tid % tpe;
  const int cps = (nchunks + tpe - 1) / tpe;
  const int c0 = min(nchunks, sub * cps), c1 = min(nchunks, c0 + cps);
  // chunks go through registers 32 at a time, so their loads are issued
  // together instead of one dependent load per chunk
  constexpr int RUN = 32;
  int part = 0;
  if (e < E) {
    for (int cb = c0; cb < c1; cb += RUN) {
      int v[RUN];
#pragma unroll
      for (int i = 0; i < RUN; ++i) v[i] = cb + i < c1 ? chunk_hist[(int64_t)(cb + i) * E + e] : 0;
#pragma unroll
      for (int i = 0; i < RUN; ++i) part += v[i];
    }
  }
  s_part[tid] = part;
  __syncthreads();
  // per-expert total and this thread's prefix within its expert
  int pre = 0, total = 0;
  if (e < E) {
    for (int j = 0; j < tpe; ++j) {
      const int v = s_part[e * tpe + j];
      if (j < sub) pre += v;
      total += v;
    }
  }
  // exclusive scan of the expert totals (thread t < E reads expert t's total)
  if (e < E && sub == 0) s_tot[e] = total;
  __syncthreads();
  const int tv = tid < E ? s_tot[tid] : 0;
  const int inc = wave_incl_scan(tv, lane);
  if (lane == 63) s_wsum[wave] = inc;
  __syncthreads();
  int wbase = 0;
  for (int w = 0; w < wave; ++w) wbase += s_wsum[w];
  if (tid < E) {
    const int excl_t = wbase + inc - tv;
    counts[tid] = tv;
    offs[tid] = excl_t + tv;
    s_part[tid] = excl_t;  // s_part is free again: expert t's exclusive base
  }
  __syncthreads();
  if (e < E) {
    int base = s_part[e] + pre;
    for (int cb = c0; cb < c1; cb += RUN) {
      int v[RUN];
#pragma unroll
      for (int i = 0; i < RUN; ++i) v[i] = cb + i < c1 ? chunk_hist[(int64_t)(cb + i) * E + e] : 0;
#pragma unroll
      for (int i = 0; i < RUN; ++i) {
        if (cb + i < c1) chunk_hist[(int64_t)(cb + i) * E + e] = base;
        base += v[i];
      }
    }
  }
}

// The expert GEMMs' row tables of sorted row p (pair q): sorted_token[p] =
// q / K and sorted_w[p] = float(w[q]) (w fp32, bf16 or fp16 by w_code 0, 1, 2;
// sorted_w may be NULL).
// With sorted_token NULL the permutation writes no tables.
struct RowTables {
  int32_t* sorted_token = nullptr;
  float* sorted_w = nullptr;
  const void* w = nullptr;
  int w_code = 0;
  int K = 1;
};

// The routing weight of pair q for the row tables (0 when none are written).
__device__ __forceinline__ float row_weight(const RowTables& rt, int q) {
  if (rt.sorted_w == nullptr) return 0.0f;
  return rt.w_code == 1   ? bf16_to_f32(static_cast<const bf16_t*>(rt.w)[q])
         : rt.w_code == 2 ? (float)static_cast<const f16_t*>(rt.w)[q]
                          : static_cast<const float*>(rt.w)[q];
}

__device__ __forceinline__ void write_row_tables(const RowTables& rt, int pos, int q, float wq) {
  if (rt.sorted_token != nullptr) {
    rt.sorted_token[pos] = q / rt.K;
    if (rt.sorted_w != nullptr) rt.sorted_w[pos] = wq;
  }
}

// Stable scatter of pairs q0 .. q1-1 by one block of NT threads: s_base[e]
// holds the position of expert e's first pair of the range, s_wcnt ([NT/64][E])
// is zero. Within a round of NT pairs, a pair's rank among the lower lanes of
// its wave with the same expert comes from ballots over the expert's bits, and
// the lower waves' counts of that expert are added from LDS. The ids (and
// routing weights) of the next round are loaded while this one is ranked.
template <int NT>
__device__ __forceinline__ void permute_scatter_range(const int64_t* __restrict__ idx, int q0, int q1, int E,
                                                      int nbits, int* s_base, int* s_wcnt,
                                                      int32_t* __restrict__ sorted_pair,
                                                      int32_t* __restrict__ inv_pos, const RowTables& rt) {
  constexpr int NW = NT / 64;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int e_nx = 0;
  float w_nx = 0.0f;
  if (q0 + tid < q1) {
    e_nx = clamp_expert(idx[q0 + tid], E);
    w_nx = row_weight(rt, q0 + tid);
  }
  for (int qb = q0; qb < q1; qb += NT) {
    const int q = qb + tid;
    const bool valid = q < q1;
    const int e = e_nx;
    const float wq = w_nx;
    if (q + NT < q1) {
      e_nx = clamp_expert(idx[q + NT], E);
      w_nx = row_weight(rt, q + NT);
    }
    uint64_t mask = __ballot(valid);
    for (int b = 0; b < nbits; ++b) {
      const bool bit = (e >> b) & 1;
      const uint64_t bal = __ballot(valid && bit);
      mask &= bit ? bal : ~bal;
    }
    const int rank = __popcll(mask & lt_mask);
    if (valid && rank == 0) s_wcnt[wave * E + e] = __popcll(mask);
    __syncthreads();
    if (valid) {
      int pos = s_base[e] + rank;
      for (int w = 0; w < wave; ++w) pos += s_wcnt[w * E + e];
      sorted_pair[pos] = q;
      inv_pos[q] = pos;
      write_row_tables(rt, pos, q, wq);
    }
    __syncthreads();
    for (int x = tid; x < E; x += NT) {
      int add = 0;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        add += s_wcnt[w * E + x];
        s_wcnt[w * E + x] = 0;
      }
      s_base[x] += add;
    }
    __syncthreads();
  }
}

template <int NT>
__global__ __launch_bounds__(NT) void permute_scatter_kernel(const int64_t* __restrict__ idx, int P, int E, int nbits,
                                                             int chunk, const int32_t* __restrict__ chunk_base,
                                                             int32_t* __restrict__ sorted_pair,
                                                             int32_t* __restrict__ inv_pos, RowTables rt) {
  constexpr int NW = NT / 64;
  extern __shared__ int sm[];
  int* s_base = sm;       // [E]
  int* s_wcnt = sm + E;   // [NW][E]
  for (int e = threadIdx.x; e < E; e += NT) {
    s_base[e] = chunk_base[(int64_t)blockIdx.x * E + e];
    for (int w = 0; w < NW; ++w) s_wcnt[w * E + e] = 0;
  }
  __syncthreads();
  const int q0 = blockIdx.x * chunk;
  permute_scatter_range<NT>(idx, q0, min(P, q0 + chunk), E, nbits, s_base, s_wcnt, sorted_pair, inv_pos, rt);
}

// The scatter for at most kFusedScanChunks chunks, with the scan folded in:
// every block reads the whole chunk histogram (nchunks x E counts, at most
// kFusedScanEntries: 32 KiB), sums each expert's column (its total, and the
// part before this block's chunk), and scans the totals over the experts, so
// the bases need no kernel of their own; block 0 also writes counts and offs.
// The sums run in chunk order and the scan in expert order, so every block
// derives the same bases as the separate scan would. Larger histograms (many
// experts and chunks: every block would re-read up to 256 KiB) take the
// separate scan kernel.
constexpr int kFusedScanChunks = 64;
constexpr int kFusedScanEntries = 8192;
template <int NT>
__global__ __launch_bounds__(NT) void permute_scatter_scan_kernel(const int64_t* __restrict__ idx, int P, int E,
                                                                  int nbits, int chunk, int nchunks,
                                                                  const int32_t* __restrict__ chunk_hist,
                                                                  int32_t* __restrict__ counts,
                                                                  int32_t* __restrict__ offs,
                                                                  int32_t* __restrict__ sorted_pair,
                                                                  int32_t* __restrict__ inv_pos, RowTables rt) {
  constexpr int NW = NT / 64;
  constexpr int PER = (1024 + NT - 1) / NT;  // experts per thread at E = 1024
  extern __shared__ int sm[];
  int* s_base = sm;       // [E]
  int* s_wcnt = sm + E;   // [NW][E]
  __shared__ int s_wsum[NW];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = blockIdx.x;
  // thread t takes experts t*per .. t*per+per-1 (per <= PER): their totals
  // over all chunks and their sums over the chunks before c
  const int per = (E + NT - 1) / NT;
  int tot[PER], pre[PER], sum = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = tid * per + j;
    tot[j] = pre[j] = 0;
    if (j < per && e < E) {
      int v[kFusedScanChunks];
#pragma unroll
      for (int i = 0; i < kFusedScanChunks; ++i) v[i] = i < nchunks ? chunk_hist[(int64_t)i * E + e] : 0;
#pragma unroll
      for (int i = 0; i < kFusedScanChunks; ++i) {
        if (i < c) pre[j] += v[i];
        tot[j] += v[i];
      }
    }
    sum += tot[j];
  }
  const int inc = wave_incl_scan(sum, lane);
  if (lane == 63) s_wsum[wave] = inc;
  __syncthreads();
  int excl = inc - sum;
  for (int w = 0; w < wave; ++w) excl += s_wsum[w];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = tid * per + j;
    if (j < per && e < E) {
      if (c == 0) {
        counts[e] = tot[j];
        offs[e] = excl + tot[j];
      }
      s_base[e] = excl + pre[j];
      excl += tot[j];
    }
  }
  for (int e = tid; e < NW * E; e += NT) s_wcnt[e] = 0;
  __syncthreads();
  const int q0 = c * chunk;
  permute_scatter_range<NT>(idx, q0, min(P, q0 + chunk), E, nbits, s_base, s_wcnt, sorted_pair, inv_pos, rt);
}

// The whole permutation of at most one chunk of pairs (decode) in one block:
// histogram, exclusive scan over the experts, stable scatter. Same result as
// the three-kernel path, in one launch instead of three.
template <int NT>
__global__ __launch_bounds__(NT) void permute_small_kernel(const int64_t* __restrict__ idx, int P, int E, int nbits,
                                                           int32_t* __restrict__ counts, int32_t* __restrict__ offs,
                                                           int32_t* __restrict__ sorted_pair,
                                                           int32_t* __restrict__ inv_pos, RowTables rt) {
  constexpr int NW = NT / 64;
  constexpr int PER = (1024 + NT - 1) / NT;
  extern __shared__ int sm[];
  int* s_base = sm;       // [E]: counts, then exclusive bases
  int* s_wcnt = sm + E;   // [NW][E]
  __shared__ int s_wsum[NW];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int e = tid; e < E; e += NT) {
    s_base[e] = 0;
    for (int w = 0; w < NW; ++w) s_wcnt[w * E + e] = 0;
  }
  __syncthreads();
  for (int q = tid; q < P; q += NT) atomicAdd(&s_base[clamp_expert(idx[q], E)], 1);
  __syncthreads();
  // thread t scans experts t*per .. t*per+per-1 (per <= PER)
  const int per = (E + NT - 1) / NT;
  int c[PER], sum = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = tid * per + j;
    c[j] = (j < per && e < E) ? s_base[e] : 0;
    sum += c[j];
  }
  const int inc = wave_incl_scan(sum, lane);
  if (lane == 63) s_wsum[wave] = inc;
  __syncthreads();
  int excl = inc - sum;
  for (int w = 0; w < wave; ++w) excl += s_wsum[w];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = tid * per + j;
    if (j < per && e < E) {
      counts[e] = c[j];
      offs[e] = excl + c[j];
      s_base[e] = excl;
      excl += c[j];
    }
  }
  __syncthreads();
  permute_scatter_range<NT>(idx, 0, P, E, nbits, s_base, s_wcnt, sorted_pair, inv_pos, rt);
}

// ---- row movers: one wave per token, 16-byte lanes. KC > 0 is the top-k
// as a compile-time constant: the K row addresses are read once and the K row
// loads of a chunk are all issued before the arithmetic, so each wave keeps K
// loads in flight. Sums run over k in ascending order in fp32 (deterministic).

template <typename T> struct RowVec { static constexpr int N = 16 / sizeof(T); };

// Scatter form of the dispatch gather: token t's row is read once and written
// to its K positions x_perm[inv_pos[t*K + k]].
template <typename T, int KC>
__global__ __launch_bounds__(256) void dispatch_kernel(const T* __restrict__ x, const int32_t* __restrict__ inv_pos,
                                                       int T_, int K, int H, T* __restrict__ x_perm) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T_) return;
  const u32x4* src = reinterpret_cast<const u32x4*>(x + (int64_t)t * H);
  const int nvec = H / RowVec<T>::N;
  if constexpr (KC > 0) {
    u32x4* dst[KC];
#pragma unroll
    for (int k = 0; k < KC; ++k)
      dst[k] = reinterpret_cast<u32x4*>(x_perm + (int64_t)inv_pos[(int64_t)t * KC + k] * H);
    for (int c = lane; c < nvec; c += 64) {
      const u32x4 v = src[c];
#pragma unroll
      for (int k = 0; k < KC; ++k) dst[k][c] = v;
    }
  } else {
    for (int c = lane; c < nvec; c += 64) {
      const u32x4 v = src[c];
      for (int k = 0; k < K; ++k)
        reinterpret_cast<u32x4*>(x_perm + (int64_t)inv_pos[(int64_t)t * K + k] * H)[c] = v;
    }
  }
}

// out[t] = (add[t] +) sum_k w[t,k] * y[inv_pos[t*K + k]].
// WEIGHTED = false: unit weights (w unused, may be null). HAS_ADD = false: no
// addend (add unused, may be null). The addend (TA) and the output (TO) may
// have another dtype than the rows (e.g. an fp32 residual stream). The
// gathered rows are read once, with non-temporal loads (at config 2 the
// combine 55.6 -> 49.2 us, the dispatch backward 66 -> 60 us).
template <typename T, typename TW, int KC, bool WEIGHTED, bool HAS_ADD, typename TA = T, typename TO = T>
__device__ __forceinline__ void gather_sum_row(const T* __restrict__ y, const TW* __restrict__ w,
                                               const int32_t* __restrict__ inv_pos, const TA* __restrict__ add, int t,
                                               int K, int H, TO* __restrict__ out, int lane) {
  if constexpr (KC > 0) {
    int64_t row[KC];
    float wk[KC];
#pragma unroll
    for (int k = 0; k < KC; ++k) {
      const int64_t q = (int64_t)t * KC + k;
      row[k] = (int64_t)inv_pos[q] * H;
      if constexpr (WEIGHTED) wk[k] = load_scalar<TW>(w + q);
      else wk[k] = 1.0f;
    }
    for (int c = lane * 8; c < H; c += 64 * 8) {
      float v[KC][8];
#pragma unroll
      for (int k = 0; k < KC; ++k) Vec8<T>::load_nt(y + row[k] + c, v[k]);
      float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      if constexpr (HAS_ADD) Vec8<TA>::load(add + (int64_t)t * H + c, acc);
#pragma unroll
      for (int k = 0; k < KC; ++k)
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] += WEIGHTED ? wk[k] * v[k][i] : v[k][i];
      Vec8<TO>::store(out + (int64_t)t * H + c, acc);
    }
  } else {
    for (int c = lane * 8; c < H; c += 64 * 8) {
      float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      if constexpr (HAS_ADD) Vec8<TA>::load(add + (int64_t)t * H + c, acc);
      for (int k = 0; k < K; ++k) {
        const int64_t q = (int64_t)t * K + k;
        float v[8];
        Vec8<T>::load_nt(y + (int64_t)inv_pos[q] * H + c, v);
        if constexpr (WEIGHTED) {
          const float wk = load_scalar<TW>(w + q);
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[i] += wk * v[i];
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[i] += v[i];
        }
      }
      Vec8<TO>::store(out + (int64_t)t * H + c, acc);
    }
  }
}

template <typename T, typename TW, int KC, bool WEIGHTED = true>
__global__ __launch_bounds__(256) void combine_kernel(const T* __restrict__ y, const TW* __restrict__ w,
                                                      const int32_t* __restrict__ inv_pos, int T_, int K, int H,
                                                      T* __restrict__ out) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T_) return;
  gather_sum_row<T, TW, KC, WEIGHTED, false>(y, w, inv_pos, static_cast<const T*>(nullptr), t, K, H, out,
                                             threadIdx.x & 63);
}

// out[t] = res[t] + sum_k w[t,k] * y[inv_pos[t*K + k]]: the combine with the
// block's residual add (qwen3_moe.py:281) fused; res and out share dtype TR.
template <typename T, typename TW, typename TR, int KC, bool WEIGHTED = true>
__global__ __launch_bounds__(256) void combine_residual_kernel(const T* __restrict__ y, const TW* __restrict__ w,
                                                               const int32_t* __restrict__ inv_pos,
                                                               const TR* __restrict__ res, int T_, int K, int H,
                                                               TR* __restrict__ out) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T_) return;
  gather_sum_row<T, TW, KC, WEIGHTED, true, TR, TR>(y, w, inv_pos, res, t, K, H, out, threadIdx.x & 63);
}

// grad_y[inv_pos[t*K+k]] = w[t,k] * dout[t]; dw[t,k] = <dout[t], y[inv_pos[t*K+k]]>.
// dout[t] (dtype TD, e.g. the fp32 gradient of a residual stream) is read
// once per chunk for all k.
template <typename T, typename TW, int KC, typename TD = T>
__global__ __launch_bounds__(256) void combine_bwd_kernel(const TD* __restrict__ dout, const T* __restrict__ y,
                                                          const TW* __restrict__ w,
                                                          const int32_t* __restrict__ inv_pos, int T_, int K, int H,
                                                          T* __restrict__ dy, TW* __restrict__ dw) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T_) return;
  const TD* drow = dout + (int64_t)t * H;
  if constexpr (KC > 0) {
    int64_t row[KC];
    float wk[KC], dot[KC];
#pragma unroll
    for (int k = 0; k < KC; ++k) {
      const int64_t q = (int64_t)t * KC + k;
      row[k] = (int64_t)inv_pos[q] * H;
      wk[k] = load_scalar<TW>(w + q);
      dot[k] = 0.0f;
    }
    for (int c = lane * 8; c < H; c += 64 * 8) {
      float g[8], v[KC][8];
      Vec8<TD>::load(drow + c, g);
#pragma unroll
      for (int k = 0; k < KC; ++k) Vec8<T>::load_nt(y + row[k] + c, v[k]);
#pragma unroll
      for (int k = 0; k < KC; ++k) {
        float o[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          dot[k] += g[i] * v[k][i];
          o[i] = wk[k] * g[i];
        }
        Vec8<T>::store(dy + row[k] + c, o);
      }
    }
#pragma unroll
    for (int k = 0; k < KC; ++k) {
      const float d = wave_sum(dot[k]);
      if (lane == 0) store_scalar<TW>(dw + (int64_t)t * KC + k, d);
    }
  } else {
    for (int k = 0; k < K; ++k) {
      const int64_t q = (int64_t)t * K + k;
      const float wk = load_scalar<TW>(w + q);
      const int64_t pos = inv_pos[q];
      float dot = 0.0f;
      for (int c = lane * 8; c < H; c += 64 * 8) {
        float g[8], v[8], o[8];
        Vec8<TD>::load(drow + c, g);
        Vec8<T>::load_nt(y + pos * H + c, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          dot += g[i] * v[i];
          o[i] = wk * g[i];
        }
        Vec8<T>::store(dy + pos * H + c, o);
      }
      dot = wave_sum(dot);
      if (lane == 0) store_scalar<TW>(dw + q, dot);
    }
  }
}

// dx[t] = (add[t] +) sum_k dx_perm[inv_pos[t*K + k]]; HAS_ADD only with a non-null add
template <typename T, int KC, bool HAS_ADD>
__global__ __launch_bounds__(256) void dispatch_bwd_kernel(const T* __restrict__ dx_perm,
                                                           const int32_t* __restrict__ inv_pos,
                                                           const T* __restrict__ add, int T_, int K, int H,
                                                           T* __restrict__ dx) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T_) return;
  gather_sum_row<T, float, KC, false, HAS_ADD>(dx_perm, nullptr, inv_pos, add, t, K, H, dx, threadIdx.x & 63);
}

unsigned blocks_for(int64_t rows, int per_block) { return (unsigned)((rows + per_block - 1) / per_block); }

}  // namespace

hipError_t split_bf16x3(const float* w, int64_t n, int planes, bf16_t* out, hipStream_t s) {
  if (n == 0) return hipSuccess;
  if (planes != 3 && planes != 4) return hipErrorInvalidValue;
  const unsigned grid = (unsigned)std::min<int64_t>((n + 255) / 256, 2048);
  hipLaunchKernelGGL(split_bf16x3_kernel, dim3(grid), dim3(256), 0, s, w, n, planes, out);
  return hipGetLastError();
}

template <typename TW>
hipError_t router_topk(const float* parts, int nsplit, int64_t split_stride, int64_t ldp, float* logits,
                       const float* logit_bias, int T, int E, int K, int norm_topk, TW* top_w, int64_t* top_idx,
                       float* top_w_f32, float* blk_psum, float* blk_lse2, int* blk_counts, int rows_per_block,
                       hipStream_t s) {
  if (T == 0) return hipSuccess;
  if (nsplit < 1 || nsplit > kMaxSplits) return hipErrorInvalidValue;
  if (rows_per_block < 1 || rows_per_block > 16) return hipErrorInvalidValue;
  const unsigned grid = blocks_for(T, rows_per_block);
  if (E <= 256 && rows_per_block % 4 == 0) {
    // four rows per wave: the same blocks of rows, a quarter of the waves
    const unsigned threads16 = 16u * (unsigned)rows_per_block;
    const size_t shmem16 =
        (size_t)((rows_per_block + 1) * E + rows_per_block + 2 * rows_per_block * K) * sizeof(float);
    const bool vec = E % 4 == 0 && ldp % 4 == 0 && split_stride % 4 == 0 &&
                     (reinterpret_cast<uintptr_t>(parts) & 15) == 0 && (reinterpret_cast<uintptr_t>(logits) & 15) == 0;
#define PMOE_TOPK16(V, VEC)                                                                                        \
  hipLaunchKernelGGL((router_topk16_kernel<V, VEC, TW>), dim3(grid), dim3(threads16), shmem16, s, parts, nsplit,   \
                     split_stride, ldp, logits, logit_bias, T, E, K, norm_topk, top_w, top_idx, top_w_f32, blk_psum, \
                     blk_lse2, blk_counts)
    if (E <= 16) PMOE_TOPK16(1, false);
    else if (E <= 32) PMOE_TOPK16(2, false);
    else if (E <= 64) { if (vec) PMOE_TOPK16(4, true); else PMOE_TOPK16(4, false); }
    else if (E <= 128) { if (vec) PMOE_TOPK16(8, true); else PMOE_TOPK16(8, false); }
    else { if (vec) PMOE_TOPK16(16, true); else PMOE_TOPK16(16, false); }
#undef PMOE_TOPK16
    return hipGetLastError();
  }
  const unsigned threads = 64u * (unsigned)rows_per_block;
  const size_t shmem = (size_t)((rows_per_block + 1) * E + rows_per_block) * sizeof(float);
#define PMOE_TOPK_CASE(EPL)                                                                                        \
  hipLaunchKernelGGL((router_topk_kernel<EPL, TW>), dim3(grid), dim3(threads), shmem, s, parts, nsplit,            \
                     split_stride, ldp, logits, logit_bias, T, E, K, norm_topk, top_w, top_idx, top_w_f32, blk_psum, \
                     blk_lse2, blk_counts)
  if (E <= 64) PMOE_TOPK_CASE(1);
  else if (E <= 128) PMOE_TOPK_CASE(2);
  else if (E <= 256) PMOE_TOPK_CASE(4);
  else if (E <= 512) PMOE_TOPK_CASE(8);
  else if (E <= 1024) PMOE_TOPK_CASE(16);
  else return hipErrorInvalidValue;
#undef PMOE_TOPK_CASE
  return hipGetLastError();
}

hipError_t router_stats_reduce(const float* blk_psum, const float* blk_lse2, const int* blk_counts, int nblk, int E,
                               float* prob_sum, float* lse_sq_sum, int32_t* counts, hipStream_t s) {
  hipLaunchKernelGGL(router_stats_reduce_kernel, dim3((unsigned)((E + 1 + 3) / 4)), dim3(256), 0, s, blk_psum, blk_lse2,
                     blk_counts, nblk, E, prob_sum, lse_sq_sum, counts);
  return hipGetLastError();
}

template <typename TW>
hipError_t split_router_weight_bwd(const TW* w, int E, int H, int ldl, bf16_t* w3t, hipStream_t s) {
  const int64_t n = (int64_t)ldl * H;
  const unsigned grid = (unsigned)std::min<int64_t>((n + 255) / 256, 2048);
  hipLaunchKernelGGL((split_router_weight_bwd_kernel<TW>), dim3(grid), dim3(256), 0, s, w, E, H, ldl, w3t);
  return hipGetLastError();
}
template hipError_t split_router_weight_bwd<float>(const float*, int, int, int, bf16_t*, hipStream_t);
template hipError_t split_router_weight_bwd<bf16_t>(const bf16_t*, int, int, int, bf16_t*, hipStream_t);
template hipError_t split_router_weight_bwd<f16_t>(const f16_t*, int, int, int, bf16_t*, hipStream_t);

template <typename TG>
hipError_t router_dlogits(const float* logits, const int64_t* top_idx, const float* top_w_f32, const TG* grad_w,
                          const float* grad_logits, int T, int E, int K, int norm_topk, float* dl, bf16_t* dl3,
                          f16_t* dl2, int ldl, hipStream_t s) {
  if (T == 0) return hipSuccess;
  const unsigned grid = blocks_for(T, 4);
#define PMOE_DL_CASE(EPL)                                                                                        \
  hipLaunchKernelGGL((router_dlogits_kernel<EPL, TG>), dim3(grid), dim3(256), 0, s, logits, top_idx, top_w_f32, \
                     grad_w, grad_logits, T, E, K, norm_topk, dl, dl3, dl2, ldl)
  if (E <= 64) PMOE_DL_CASE(1);
  else if (E <= 128) PMOE_DL_CASE(2);
  else if (E <= 256) PMOE_DL_CASE(4);
  else if (E <= 512) PMOE_DL_CASE(8);
  else if (E <= 1024) PMOE_DL_CASE(16);
  else return hipErrorInvalidValue;
#undef PMOE_DL_CASE
  return hipGetLastError();
}

template <typename TO>
hipError_t reduce_partials(const float* partial, int splits, int64_t n, TO* out, hipStream_t s) {
  if (n == 0) return hipSuccess;
  if (n % 4 == 0 && (reinterpret_cast<uintptr_t>(partial) & 15) == 0) {
    const unsigned grid4 = (unsigned)std::min<int64_t>((n / 4 + 255) / 256, 4096);
    hipLaunchKernelGGL((reduce_partials4_kernel<TO>), dim3(grid4), dim3(256), 0, s, partial, splits, n, out);
    return hipGetLastError();
  }
  const unsigned grid = (unsigned)std::min<int64_t>((n + 255) / 256, 4096);
  hipLaunchKernelGGL((reduce_partials_kernel<TO>), dim3(grid), dim3(256), 0, s, partial, splits, n, out);
  return hipGetLastError();
}

hipError_t permute_pairs(const int64_t* top_idx, int T, int K, int E, int32_t* counts, int32_t* offs,
                         int32_t* sorted_pair, int32_t* inv_pos, int32_t* chunk_hist, int chunk, hipStream_t s,
                         int32_t* sorted_token, float* sorted_w, const void* w, int w_code) {
  const int P = T * K;
  const int nchunks = (P + chunk - 1) / chunk;
  if (E > 1024 || E < 1) return hipErrorInvalidValue;
  int nbits = 0;
  while ((1 << nbits) < E) ++nbits;
  RowTables rt;
  rt.sorted_token = sorted_token;
  rt.sorted_w = sorted_w;
  rt.w = w;
  rt.w_code = w_code;
  rt.K = K;
  // The scatter ranks a round of one pair per thread at a time: blocks of 1024
  // threads (a 2048-pair chunk in 2 rounds) while their LDS counts, one row of E
  // per wave, stay small; 256 threads for E > 256.
  auto launch = [&](auto ntc) {
    constexpr int NT = decltype(ntc)::value;
    const size_t shm = (size_t)(1 + NT / 64) * E * sizeof(int);
    if (nchunks <= 1) {
      hipLaunchKernelGGL((permute_small_kernel<NT>), dim3(1), dim3(NT), shm, s, top_idx, P, E, nbits, counts, offs,
                         sorted_pair, inv_pos, rt);
      return hipGetLastError();
    }
    hipLaunchKernelGGL(permute_hist_kernel, dim3(nchunks), dim3(256), E * sizeof(int), s, top_idx, P, E, chunk,
                       chunk_hist);
    if (nchunks <= kFusedScanChunks && nchunks * E <= kFusedScanEntries) {
      hipLaunchKernelGGL((permute_scatter_scan_kernel<NT>), dim3(nchunks), dim3(NT), shm, s, top_idx, P, E, nbits,
                         chunk, nchunks, chunk_hist, counts, offs, sorted_pair, inv_pos, rt);
      return hipGetLastError();
    }
    hipLaunchKernelGGL(permute_scan_kernel, dim3(1), dim3(1024), 0, s, chunk_hist, nchunks, E, counts, offs);
    hipLaunchKernelGGL((permute_scatter_kernel<NT>), dim3(nchunks), dim3(NT), shm, s, top_idx, P, E, nbits, chunk,
                       chunk_hist, sorted_pair, inv_pos, rt);
    return hipGetLastError();
  };
  if (E <= 256) return launch(std::integral_constant<int, 1024>());
  return launch(std::integral_constant<int, 256>());
}

// Ids outside [0, E): one block of 1024 threads strides over all n ids and
// writes the count (no atomics, no prior clearing of `count`).
__global__ __launch_bounds__(1024) void count_invalid_ids_kernel(const int64_t* __restrict__ idx, int64_t n, int64_t E,
                                                                 int32_t* __restrict__ count) {
  __shared__ int s_w[16];
  int c = 0;
  for (int64_t i = threadIdx.x; i < n; i += 1024) {
    const int64_t e = idx[i];
    c += (e < 0 || e >= E) ? 1 : 0;
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  c = wave_incl_scan(c, lane);
  if (lane == 63) s_w[wave] = c;
  __syncthreads();
  if (threadIdx.x == 0) {
    int t = 0;
    for (int w = 0; w < 16; ++w) t += s_w[w];
    count[0] = t;
  }
}

hipError_t count_invalid_ids(const int64_t* idx, int64_t n, int64_t E, int32_t* count, hipStream_t s) {
  hipLaunchKernelGGL(count_invalid_ids_kernel, dim3(1), dim3(1024), 0, s, idx, n, E, count);
  return hipGetLastError();
}

// Per sorted row p (pair q = sorted_pair[p]): its token q / K and its routing
// weight w[q] as fp32 (w may be null: no weights).
template <typename TW>
__global__ __launch_bounds__(256) void sort_rows_kernel(const int32_t* __restrict__ sorted_pair,
                                                        const TW* __restrict__ w, int P, int K,
                                                        int32_t* __restrict__ sorted_token, float* __restrict__ sorted_w) {
  for (int p = blockIdx.x * 256 + threadIdx.x; p < P; p += gridDim.x * 256) {
    const int q = sorted_pair[p];
    sorted_token[p] = q / K;
    if (sorted_w != nullptr) sorted_w[p] = load_scalar<TW>(w + q);
  }
}

template <typename TW>
hipError_t sort_rows(const int32_t* sorted_pair, const TW* w, int P, int K, int32_t* sorted_token, float* sorted_w,
                     hipStream_t s) {
  if (P == 0) return hipSuccess;
  const int blocks = std::min((P + 255) / 256, 4096);
  hipLaunchKernelGGL((sort_rows_kernel<TW>), dim3(blocks), dim3(256), 0, s, sorted_pair, w, P, K, sorted_token,
                     sorted_w);
  return hipGetLastError();
}
template hipError_t sort_rows<float>(const int32_t*, const float*, int, int, int32_t*, float*, hipStream_t);
template hipError_t sort_rows<bf16_t>(const int32_t*, const bf16_t*, int, int, int32_t*, float*, hipStream_t);
template hipError_t sort_rows<f16_t>(const int32_t*, const f16_t*, int, int, int32_t*, float*, hipStream_t);

// The routing weights' gradient from the per-row partials of the down
// backward: grad_w[q] = sum_j part[inv_pos[q] * ld + j] (j ascending, fp32).
template <typename TG>
__global__ __launch_bounds__(256) void pair_weight_grad_kernel(const float* __restrict__ part, int ld, int nparts,
                                                               const int32_t* __restrict__ inv_pos, int P,
                                                               TG* __restrict__ grad_w) {
  for (int q = blockIdx.x * 256 + threadIdx.x; q < P; q += gridDim.x * 256) {
    const float* r = part + (int64_t)inv_pos[q] * ld;
    float acc = 0.0f;
    for (int j = 0; j < nparts; ++j) acc += r[j];
    store_scalar<TG>(grad_w + q, acc);
  }
}

template <typename TG>
hipError_t pair_weight_grad(const float* part, int ld, int nparts, const int32_t* inv_pos, int P, TG* grad_w,
                            hipStream_t s) {
  if (P == 0) return hipSuccess;
  const int blocks = std::min((P + 255) / 256, 4096);
  hipLaunchKernelGGL((pair_weight_grad_kernel<TG>), dim3(blocks), dim3(256), 0, s, part, ld, nparts, inv_pos, P,
                     grad_w);
  return hipGetLastError();
}
template hipError_t pair_weight_grad<float>(const float*, int, int, const int32_t*, int, float*, hipStream_t);
template hipError_t pair_weight_grad<bf16_t>(const float*, int, int, const int32_t*, int, bf16_t*, hipStream_t);
template hipError_t pair_weight_grad<f16_t>(const float*, int, int, const int32_t*, int, f16_t*, hipStream_t);

// Calls F with the compile-time top-k (the common values) or 0 (runtime K).
template <class F>
hipError_t with_kc(int K, F&& f) {
  switch (K) {
    case 1: return f(std::integral_constant<int, 1>());
    case 2: return f(std::integral_constant<int, 2>());
    case 4: return f(std::integral_constant<int, 4>());
    case 6: return f(std::integral_constant<int, 6>());
    case 8: return f(std::integral_constant<int, 8>());
    default: return f(std::integral_constant<int, 0>());
  }
}

template <typename T>
hipError_t dispatch_rows(const T* x, const int32_t* inv_pos, int T_, int K, int H, T* x_perm, hipStream_t s) {
  if (T_ == 0) return hipSuccess;
  return with_kc(K, [&](auto kc) {
    hipLaunchKernelGGL((dispatch_kernel<T, decltype(kc)::value>), dim3(blocks_for(T_, 4)), dim3(256), 0, s, x, inv_pos,
                       T_, K, H, x_perm);
    return hipGetLastError();
  });
}

template <typename T, typename TW>
hipError_t combine_rows(const T* y, const TW* w, const int32_t* inv_pos, int T_, int K, int H, T* out,
                        hipStream_t s) {
  if (T_ == 0) return hipSuccess;
  return with_kc(K, [&](auto kc) {
    if (w != nullptr)
      hipLaunchKernelGGL((combine_kernel<T, TW, decltype(kc)::value>), dim3(blocks_for(T_, 4)), dim3(256), 0, s, y, w,
                         inv_pos, T_, K, H, out);
    else  // unit weights: the rows already carry their routing weight
      hipLaunchKernelGGL((combine_kernel<T, TW, decltype(kc)::value, false>), dim3(blocks_for(T_, 4)), dim3(256), 0,
                         s, y, w, inv_pos, T_, K, H, out);
    return hipGetLastError();
  });
}

template <typename T, typename TW>
hipError_t combine_rows_bwd(const T* dout, const T* y, const TW* w, const int32_t* inv_pos, int T_, int K, int H,
                            T* dy, TW* dw, hipStream_t s) {
  if (T_ == 0) return hipSuccess;
  return with_kc(K, [&](auto kc) {
    hipLaunchKernelGGL((combine_bwd_kernel<T, TW, decltype(kc)::value>), dim3(blocks_for(T_, 4)), dim3(256), 0, s,
                       dout, y, w, inv_pos, T_, K, H, dy, dw);
    return hipGetLastError();
  });
}

// Top-k values with a compile-time specialisation in the residual variants.
template <class F>
hipError_t with_kc8(int K, F&& f) {
  if (K == 8) return f(std::integral_constant<int, 8>());
  return f(std::integral_constant<int, 0>());
}

template <typename T, typename TW, typename TR>
hipError_t combine_rows_residual(const T* y, const TW* w, const int32_t* inv_pos, const TR* res, int T_, int K, int H,
                                 TR* out, hipStream_t s) {
  if (T_ == 0) return hipSuccess;
  return with_kc8(K, [&](auto kc) {
    if (w != nullptr)
      hipLaunchKernelGGL((combine_residual_kernel<T, TW, TR, decltype(kc)::value>), dim3(blocks_for(T_, 4)),
                         dim3(256), 0, s, y, w, inv_pos, res, T_, K, H, out);
    else
      hipLaunchKernelGGL((combine_residual_kernel<T, TW, TR, decltype(kc)::value, false>), dim3(blocks_for(T_, 4)),
                         dim3(256), 0, s, y, w, inv_pos, res, T_, K, H, out);
    return hipGetLastError();
  });
}

template <typename T, typename TW, typename TD>
hipError_t combine_rows_residual_bwd(const TD* dout, const T* y, const TW* w, const int32_t* inv_pos, int T_, int K,
                                     int H, T* dy, TW* dw, hipStream_t s) {
  if (T_ == 0) return hipSuccess;
  return with_kc8(K, [&](auto kc) {
    hipLaunchKernelGGL((combine_bwd_kernel<T, TW, decltype(kc)::value, TD>), dim3(blocks_for(T_, 4)), dim3(256), 0, s,
                       dout, y, w, inv_pos, T_, K, H, dy, dw);
    return hipGetLastError();
  });
}

template <typename T>
hipError_t dispatch_rows_bwd(const T* dx_perm, const int32_t* inv_pos, const T* add, int T_, int K, int H, T* dx,
                             hipStream_t s) {
  if (T_ == 0) return hipSuccess;
  return with_kc(K, [&](auto kc) {
    if (add != nullptr)
      hipLaunchKernelGGL((dispatch_bwd_kernel<T, decltype(kc)::value, true>), dim3(blocks_for(T_, 4)), dim3(256), 0,
                         s, dx_perm, inv_pos, add, T_, K, H, dx);
    else
      hipLaunchKernelGGL((dispatch_bwd_kernel<T, decltype(kc)::value, false>), dim3(blocks_for(T_, 4)), dim3(256), 0,
                         s, dx_perm, inv_pos, add, T_, K, H, dx);
    return hipGetLastError();
  });
}

template hipError_t router_topk<bf16_t>(const float*, int, int64_t, int64_t, float*, const float*, int, int, int, int,
                                        bf16_t*, int64_t*, float*, float*, float*, int*, int, hipStream_t);
template hipError_t router_topk<float>(const float*, int, int64_t, int64_t, float*, const float*, int, int, int, int,
                                       float*, int64_t*, float*, float*, float*, int*, int, hipStream_t);
template hipError_t router_topk<f16_t>(const float*, int, int64_t, int64_t, float*, const float*, int, int, int, int,
                                       f16_t*, int64_t*, float*, float*, float*, int*, int, hipStream_t);
template hipError_t router_dlogits<bf16_t>(const float*, const int64_t*, const float*, const bf16_t*, const float*,
                                           int, int, int, int, float*, bf16_t*, f16_t*, int, hipStream_t);
template hipError_t router_dlogits<f16_t>(const float*, const int64_t*, const float*, const f16_t*, const float*,
                                          int, int, int, int, float*, bf16_t*, f16_t*, int, hipStream_t);
template hipError_t router_dlogits<float>(const float*, const int64_t*, const float*, const float*, const float*, int,
                                          int, int, int, float*, bf16_t*, f16_t*, int, hipStream_t);
template hipError_t reduce_partials<float>(const float*, int, int64_t, float*, hipStream_t);
template hipError_t reduce_partials<bf16_t>(const float*, int, int64_t, bf16_t*, hipStream_t);
template hipError_t reduce_partials<f16_t>(const float*, int, int64_t, f16_t*, hipStream_t);

#define PMOE_INST_COMBINE(T, TW)                                                                                \
  template hipError_t combine_rows<T, TW>(const T*, const TW*, const int32_t*, int, int, int, T*, hipStream_t);     \
  template hipError_t combine_rows_bwd<T, TW>(const T*, const T*, const TW*, const int32_t*, int, int, int, T*, TW*, \
                                              hipStream_t);
#define PMOE_INST_ROWS(T)                                                                                      \
  template hipError_t dispatch_rows<T>(const T*, const int32_t*, int, int, int, T*, hipStream_t);              \
  template hipError_t dispatch_rows_bwd<T>(const T*, const int32_t*, const T*, int, int, int, T*, hipStream_t); \
  PMOE_INST_COMBINE(T, bf16_t) PMOE_INST_COMBINE(T, f16_t) PMOE_INST_COMBINE(T, float)

PMOE_INST_ROWS(bf16_t)
PMOE_INST_ROWS(f16_t)
PMOE_INST_ROWS(float)

#define PMOE_INST_RES(T, TW, TR)                                                                                  \
  template hipError_t combine_rows_residual<T, TW, TR>(const T*, const TW*, const int32_t*, const TR*, int, int,   \
                                                       int, TR*, hipStream_t);                                      \
  template hipError_t combine_rows_residual_bwd<T, TW, TR>(const TR*, const T*, const TW*, const int32_t*, int,    \
                                                           int, int, T*, TW*, hipStream_t);
#define PMOE_INST_RES2(T, TW) PMOE_INST_RES(T, TW, bf16_t) PMOE_INST_RES(T, TW, float)
PMOE_INST_RES2(bf16_t, bf16_t)
PMOE_INST_RES2(bf16_t, float)
PMOE_INST_RES2(float, bf16_t)
PMOE_INST_RES2(float, float)

}  // namespace pmoe
