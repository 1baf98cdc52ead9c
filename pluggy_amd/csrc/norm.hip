// The MoE block's neighbours fused into its row kernels: the RMSNorm in front
// of the router (Qwen3MoeTransformerBlock.norm2, qwen3_moe.py:260 and :281,
// torch.nn.RMSNorm) and, in the backward, the RMSNorm gradient and the
// residual gradient folded into the K-row sum of the dispatch backward.
//
// One wave per row, 8 consecutive elements per lane per 512-column chunk,
// fp32 arithmetic; row sums are butterfly reductions, so every lane holds the
// same bits and the results are deterministic.
#include "kernels.h"

namespace pmoe {
namespace {

// out[t] = (x[t] * r_t) * w, r_t = 1 / sqrt(sum_j x[t,j]^2 / H + eps); rstd[t] = r_t.
template <typename TX, typename TO>
__global__ __launch_bounds__(256) void rmsnorm_fwd_kernel(const TX* __restrict__ x, const float* __restrict__ w,
                                                          float eps, int T_, int H, TO* __restrict__ out,
                                                          float* __restrict__ rstd) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T_) return;
  const TX* row = x + (int64_t)t * H;
  float ss = 0.0f;
  for (int c = lane * 8; c < H; c += 512) {
    float v[8];
    Vec8<TX>::load(row + c, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += v[i] * v[i];
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / (float)H + eps);
  if (lane == 0) rstd[t] = r;
  for (int c = lane * 8; c < H; c += 512) {
    float v[8], g[8];
    Vec8<TX>::load(row + c, v);
    Vec8<float>::load(w + c, g);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (v[i] * r) * g[i];
    Vec8<TO>::store(out + (int64_t)t * H + c, v);
  }
}

// Per row t (one wave), with n = (x * r) * w the RMSNorm output:
//   g[t]  = add[t] + sum_k gxp[inv_pos[t*K + k]]              (dL/dn, k ascending)
//   gx[t] = res[t] + r * w * g - (r^3 / H) * <g * w, x[t]> * x[t]
//   gw_partial[block] = sum over the block's rows of g * x[t] * r
// gxp, add and res may each be null (a missing term). NCH chunks of 512
// columns per row are held in registers (H <= 512 * NCH).
template <typename T, typename TX, int KC, int NCH>
__global__ __launch_bounds__(256) void dispatch_rmsnorm_bwd_kernel(
    const T* __restrict__ gxp, const int32_t* __restrict__ inv_pos, const T* __restrict__ add,
    const TX* __restrict__ x, const float* __restrict__ w, const float* __restrict__ rstd, const TX* __restrict__ res,
    int T_, int K, int H, TX* __restrict__ gx, float* __restrict__ gw_partial) {
  __shared__ float s_gw[3][512 * NCH];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nwaves = gridDim.x * 4;
  float gw[NCH][8];
#pragma unroll
  for (int i = 0; i < NCH; ++i)
#pragma unroll
    for (int e = 0; e < 8; ++e) gw[i][e] = 0.0f;

  for (int t = blockIdx.x * 4 + wave; t < T_; t += nwaves) {
    float g[NCH][8];
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = lane * 8 + 512 * i;
#pragma unroll
      for (int e = 0; e < 8; ++e) g[i][e] = 0.0f;
      if (c < H && add != nullptr) Vec8<T>::load(add + (int64_t)t * H + c, g[i]);
    }
    if (gxp != nullptr) {
      if constexpr (KC > 0) {
        int64_t row[KC];
#pragma unroll
        for (int k = 0; k < KC; ++k) row[k] = (int64_t)inv_pos[(int64_t)t * KC + k] * H;
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
          const int c = lane * 8 + 512 * i;
          if (c < H) {
            float v[KC][8];
#pragma unroll
            for (int k = 0; k < KC; ++k) Vec8<T>::load_nt(gxp + row[k] + c, v[k]);  // read once
#pragma unroll
            for (int k = 0; k < KC; ++k)
#pragma unroll
              for (int e = 0; e < 8; ++e) g[i][e] += v[k][e];
          }
        }
      } else {
        for (int k = 0; k < K; ++k) {
          const int64_t rk = (int64_t)inv_pos[(int64_t)t * K + k] * H;
#pragma unroll
          for (int i = 0; i < NCH; ++i) {
            const int c = lane * 8 + 512 * i;
            if (c < H) {
              float v[8];
              Vec8<T>::load_nt(gxp + rk + c, v);
#pragma unroll
              for (int e = 0; e < 8; ++e) g[i][e] += v[e];
            }
          }
        }
      }
    }
    const TX* xr = x + (int64_t)t * H;
    float dot = 0.0f;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = lane * 8 + 512 * i;
      if (c < H) {
        float xv[8], wv[8];
        Vec8<TX>::load(xr + c, xv);
        Vec8<float>::load(w + c, wv);
#pragma unroll
        for (int e = 0; e < 8; ++e) dot += g[i][e] * wv[e] * xv[e];
      }
    }
    dot = wave_sum(dot);
    const float r = rstd[t];
    const float coef = r * r * r * dot / (float)H;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = lane * 8 + 512 * i;
      if (c < H) {
        float xv[8], wv[8], o[8];
        Vec8<TX>::load(xr + c, xv);
        Vec8<float>::load(w + c, wv);
        if (res != nullptr) Vec8<TX>::load(res + (int64_t)t * H + c, o);
        else
#pragma unroll
          for (int e = 0; e < 8; ++e) o[e] = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          o[e] += r * wv[e] * g[i][e] - coef * xv[e];
          gw[i][e] += g[i][e] * (xv[e] * r);
        }
        Vec8<TX>::store(gx + (int64_t)t * H + c, o);
      }
    }
  }
  if (gw_partial == nullptr) return;  // uniform over the grid
  // the block's four waves -> one partial row, summed in wave order
  if (wave > 0) {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = lane * 8 + 512 * i;
      if (c < H)
#pragma unroll
        for (int e = 0; e < 8; ++e) s_gw[wave - 1][c + e] = gw[i][e];
    }
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = lane * 8 + 512 * i;
      if (c < H) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          gw[i][e] = ((gw[i][e] + s_gw[0][c + e]) + s_gw[1][c + e]) + s_gw[2][c + e];
        Vec8<float>::store(gw_partial + (int64_t)blockIdx.x * H + c, gw[i]);
      }
    }
  }
}

// The same row backward for rows too wide to hold in registers (H > 512 *
// 8): each row is walked twice in 512-column chunks, first for <g * w, x>,
// then for gx, re-reading its K expert rows (twice the gxp traffic of the
// register kernel). The norm-weight partial of each of the block's two waves
// accumulates in its own LDS row (dynamic shared memory, 2 * H floats); the
// two rows are summed in wave order at the end, as in the register kernel.
template <typename T, typename TX>
__global__ __launch_bounds__(128) void dispatch_rmsnorm_bwd_wide_kernel(
    const T* __restrict__ gxp, const int32_t* __restrict__ inv_pos, const T* __restrict__ add,
    const TX* __restrict__ x, const float* __restrict__ w, const float* __restrict__ rstd, const TX* __restrict__ res,
    int T_, int K, int H, TX* __restrict__ gx, float* __restrict__ gw_partial) {
  extern __shared__ float s_gw_wide[];  // [2][H]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nwaves = gridDim.x * 2;
  float* my_gw = s_gw_wide + (size_t)wave * H;
  for (int c = lane; c < H; c += 64) my_gw[c] = 0.0f;
  // g (dL/dn) of 8 columns from c of row t: add + the K expert rows in order
  auto row_grad = [&](int t, int c, float* g) {
#pragma unroll
    for (int e = 0; e < 8; ++e) g[e] = 0.0f;
    if (add != nullptr) Vec8<T>::load(add + (int64_t)t * H + c, g);
    if (gxp != nullptr) {
      for (int k = 0; k < K; ++k) {
        float v[8];
        Vec8<T>::load(gxp + (int64_t)inv_pos[(int64_t)t * K + k] * H + c, v);
#pragma unroll
        for (int e = 0; e < 8; ++e) g[e] += v[e];
      }
    }
  };
  for (int t = blockIdx.x * 2 + wave; t < T_; t += nwaves) {
    const TX* xr = x + (int64_t)t * H;
    float dot = 0.0f;
    for (int c = lane * 8; c < H; c += 512) {
      float g[8], xv[8], wv[8];
      row_grad(t, c, g);
      Vec8<TX>::load(xr + c, xv);
      Vec8<float>::load(w + c, wv);
#pragma unroll
      for (int e = 0; e < 8; ++e) dot += g[e] * wv[e] * xv[e];
    }
    dot = wave_sum(dot);
    const float r = rstd[t];
    const float coef = r * r * r * dot / (float)H;
    for (int c = lane * 8; c < H; c += 512) {
      float g[8], xv[8], wv[8], o[8];
      row_grad(t, c, g);
      Vec8<TX>::load(xr + c, xv);
      Vec8<float>::load(w + c, wv);
      if (res != nullptr) Vec8<TX>::load(res + (int64_t)t * H + c, o);
      else
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        o[e] += r * wv[e] * g[e] - coef * xv[e];
        my_gw[c + e] += g[e] * (xv[e] * r);  // this lane's own columns: no other lane writes them
      }
      Vec8<TX>::store(gx + (int64_t)t * H + c, o);
    }
  }
  if (gw_partial == nullptr) return;  // uniform over the grid
  __syncthreads();
  for (int c = threadIdx.x; c < H; c += 128)
    gw_partial[(int64_t)blockIdx.x * H + c] = s_gw_wide[c] + s_gw_wide[(size_t)H + c];
}

// tmp[g, j] = sum_{r in group g} partial[r, j], groups of kRowGroup rows in
// order: the first of two passes that reduce a tall (rows x n) partial matrix
// with the whole grid busy (one thread per column and group).
__global__ __launch_bounds__(256) void sum_row_groups_kernel(const float* __restrict__ partial, int rows, int n,
                                                             float* __restrict__ tmp) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= n) return;
  const int r0 = blockIdx.y * kRowGroup, r1 = min(r0 + kRowGroup, rows);
  float acc = 0.0f;
#pragma unroll 8
  for (int r = r0; r < r1; ++r) acc += partial[(int64_t)r * n + j];
  tmp[(int64_t)blockIdx.y * n + j] = acc;
}

}  // namespace

int rmsnorm_bwd_groups(int T_) { return (rmsnorm_bwd_blocks(T_) + kRowGroup - 1) / kRowGroup; }

hipError_t sum_row_groups(const float* partial, int rows, int n, float* tmp, hipStream_t s) {
  if (rows == 0 || n == 0) return hipSuccess;
  hipLaunchKernelGGL(sum_row_groups_kernel, dim3((n + 255) / 256, (rows + kRowGroup - 1) / kRowGroup), dim3(256), 0,
                     s, partial, rows, n, tmp);
  return hipGetLastError();
}

template <typename TX, typename TO>
hipError_t rmsnorm_fwd(const TX* x, const float* w, float eps, int T_, int H, TO* out, float* rstd, hipStream_t s) {
  if (T_ == 0) return hipSuccess;
  hipLaunchKernelGGL((rmsnorm_fwd_kernel<TX, TO>), dim3((T_ + 3) / 4), dim3(256), 0, s, x, w, eps, T_, H, out, rstd);
  return hipGetLastError();
}

int rmsnorm_bwd_blocks(int T_) { return std::max(1, std::min((T_ + 7) / 8, kRmsnormBwdMaxBlocks)); }

template <typename T, typename TX>
hipError_t dispatch_rmsnorm_bwd(const T* gxp, const int32_t* inv_pos, const T* add, const TX* x, const float* w,
                                const float* rstd, const TX* res, int T_, int K, int H, TX* gx, float* gw_partial,
                                hipStream_t s) {
  if (T_ == 0) return hipSuccess;
  const int nb = rmsnorm_bwd_blocks(T_);
  auto go = [&](auto kc, auto nch) {
    hipLaunchKernelGGL((dispatch_rmsnorm_bwd_kernel<T, TX, decltype(kc)::value, decltype(nch)::value>), dim3(nb),
                       dim3(256), 0, s, gxp, inv_pos, add, x, w, rstd, res, T_, K, H, gx, gw_partial);
    return hipGetLastError();
  };
  auto by_k = [&](auto nch) {
    return K == 8 ? go(std::integral_constant<int, 8>(), nch) : go(std::integral_constant<int, 0>(), nch);
  };
  if (H <= 1024) return by_k(std::integral_constant<int, 2>());
  if (H <= 2048) return by_k(std::integral_constant<int, 4>());
  if (H <= kRmsnormRegH) return by_k(std::integral_constant<int, 8>());
  if (H > kRmsnormMaxH) return hipErrorInvalidValue;
  const size_t lds = (size_t)2 * H * sizeof(float);
  auto wide = dispatch_rmsnorm_bwd_wide_kernel<T, TX>;
  const hipError_t ea = hipFuncSetAttribute((const void*)wide, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (ea != hipSuccess) return ea;
  hipLaunchKernelGGL(wide, dim3(nb), dim3(128), lds, s, gxp, inv_pos, add, x, w, rstd, res, T_, K, H, gx, gw_partial);
  return hipGetLastError();
}

#define PMOE_INST_NORM(TX, TO) \
  template hipError_t rmsnorm_fwd<TX, TO>(const TX*, const float*, float, int, int, TO*, float*, hipStream_t);
PMOE_INST_NORM(float, float)
PMOE_INST_NORM(float, bf16_t)
PMOE_INST_NORM(bf16_t, float)
PMOE_INST_NORM(bf16_t, bf16_t)

#define PMOE_INST_NORM_BWD(T, TX)                                                                                   \
  template hipError_t dispatch_rmsnorm_bwd<T, TX>(const T*, const int32_t*, const T*, const TX*, const float*,      \
                                                  const float*, const TX*, int, int, int, TX*, float*, hipStream_t);
PMOE_INST_NORM_BWD(bf16_t, float)
PMOE_INST_NORM_BWD(bf16_t, bf16_t)
PMOE_INST_NORM_BWD(float, float)
PMOE_INST_NORM_BWD(float, bf16_t)

}  // namespace pmoe
