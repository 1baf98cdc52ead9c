// Launchers of the grouped expert GEMMs and the router GEMMs.
#include "gemm.h"
#include "kernels.h"

namespace pmoe {

namespace {

// Tile shapes. bf16: 128x128 block, four 64x64 wave tiles of 2x2 MFMA 32x32x16.
// fp32: 64x128 block, four 32x64 wave tiles of MFMA 32x32x2.
typedef TileCfg<bf16_t, 128, 128, 64, 64> CfgBf16;
typedef TileCfg<float, 64, 128, 32, 64> CfgF32;

template <typename T> struct CfgFor;
template <> struct CfgFor<bf16_t> { typedef CfgBf16 type; };
template <> struct CfgFor<float> { typedef CfgF32 type; };

template <class Cfg, typename TA, typename TB, typename Tout, bool A_KC, bool B_KC, int GM, int EPI>
hipError_t launch(const GemmParams& p, hipStream_t s) {
  const int ntn = (EPI == EPI_SWIGLU) ? (p.inter + Cfg::BN / 2 - 1) / (Cfg::BN / 2) : (p.N + Cfg::BN - 1) / Cfg::BN;
  int64_t slots;
  if (GM == GM_ROWS) slots = (p.M + Cfg::BM - 1) / Cfg::BM + p.groups;
  else if (GM == GM_RED) slots = (int64_t)p.groups * ((p.M + Cfg::BM - 1) / Cfg::BM);
  else slots = (p.M + Cfg::BM - 1) / Cfg::BM;
  const int64_t grid = slots * ntn;
  if (grid <= 0) return hipSuccess;
  if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL((grouped_gemm_kernel<Cfg, TA, TB, Tout, A_KC, B_KC, GM, EPI>), dim3((unsigned)grid),
                     dim3(Cfg::NT), 0, s, p);
  return hipGetLastError();
}

GemmParams zero_params() {
  GemmParams p;
  p.A = nullptr; p.lda = 0;
  p.B = nullptr; p.ldb = 0; p.strideB = 0;
  p.C = nullptr; p.ldc = 0; p.strideC = 0;
  p.C2 = nullptr; p.ldc2 = 0;
  p.aux = nullptr; p.ldaux = 0;
  p.offs = nullptr; p.groups = 1;
  p.M = p.N = p.K = 0; p.split_chunk = 0; p.inter = 0;
  return p;
}

}  // namespace

template <typename T>
hipError_t gate_up_swiglu_fwd(const T* x_perm, const T* w_gu, const int32_t* offs, int P, int E, int H, int I,
                              T* gu_out, T* mid, hipStream_t s) {
  GemmParams p = zero_params();
  p.A = x_perm; p.lda = H;
  p.B = w_gu; p.ldb = H; p.strideB = (int64_t)2 * I * H;
  p.C = gu_out; p.ldc = 2 * I;
  p.C2 = mid; p.ldc2 = I;
  p.offs = offs; p.groups = E;
  p.M = P; p.N = 2 * I; p.K = H; p.inter = I;
  return launch<typename CfgFor<T>::type, T, T, T, true, true, GM_ROWS, EPI_SWIGLU>(p, s);
}

template <typename T>
hipError_t down_fwd(const T* mid, const T* w_dn, const int32_t* offs, int P, int E, int H, int I, T* y,
                    hipStream_t s) {
  GemmParams p = zero_params();
  p.A = mid; p.lda = I;
  p.B = w_dn; p.ldb = I; p.strideB = (int64_t)H * I;
  p.C = y; p.ldc = H;
  p.offs = offs; p.groups = E;
  p.M = P; p.N = H; p.K = I;
  return launch<typename CfgFor<T>::type, T, T, T, true, true, GM_ROWS, EPI_STORE>(p, s);
}

template <typename T>
hipError_t down_dgrad_swiglu_bwd(const T* dy, const T* w_dn, const T* gu_out, const int32_t* offs, int P, int E,
                                 int H, int I, T* dgu, hipStream_t s) {
  GemmParams p = zero_params();
  p.A = dy; p.lda = H;
  p.B = w_dn; p.ldb = I; p.strideB = (int64_t)H * I;  // B[k=h][n=i] = W_dn[e][h][i]
  p.C = dgu; p.ldc = 2 * I;
  p.aux = gu_out; p.ldaux = 2 * I;
  p.offs = offs; p.groups = E;
  p.M = P; p.N = I; p.K = H; p.inter = I;
  return launch<typename CfgFor<T>::type, T, T, T, true, false, GM_ROWS, EPI_SWIGLU_BWD>(p, s);
}

template <typename T>
hipError_t down_wgrad(const T* dy, const T* mid, const int32_t* offs, int P, int E, int H, int I, T* dw_dn,
                      hipStream_t s) {
  GemmParams p = zero_params();
  p.A = dy; p.lda = H;   // A[m=h][k=p] = dy[p][h]
  p.B = mid; p.ldb = I;  // B[k=p][n=i] = mid[p][i]
  p.C = dw_dn; p.ldc = I; p.strideC = (int64_t)H * I;
  p.offs = offs; p.groups = E;
  p.M = H; p.N = I; p.K = P;
  return launch<typename CfgFor<T>::type, T, T, T, false, false, GM_RED, EPI_STORE>(p, s);
}

template <typename T>
hipError_t gate_up_dgrad(const T* dgu, const T* w_gu, const int32_t* offs, int P, int E, int H, int I, T* dx_perm,
                         hipStream_t s) {
  GemmParams p = zero_params();
  p.A = dgu; p.lda = 2 * I;
  p.B = w_gu; p.ldb = H; p.strideB = (int64_t)2 * I * H;  // B[k=j][n=h] = W_gu[e][j][h]
  p.C = dx_perm; p.ldc = H;
  p.offs = offs; p.groups = E;
  p.M = P; p.N = H; p.K = 2 * I;
  return launch<typename CfgFor<T>::type, T, T, T, true, false, GM_ROWS, EPI_STORE>(p, s);
}

template <typename T>
hipError_t gate_up_wgrad(const T* dgu, const T* x_perm, const int32_t* offs, int P, int E, int H, int I, T* dw_gu,
                         hipStream_t s) {
  GemmParams p = zero_params();
  p.A = dgu; p.lda = 2 * I;  // A[m=j][k=p] = dgu[p][j]
  p.B = x_perm; p.ldb = H;   // B[k=p][n=h] = x_perm[p][h]
  p.C = dw_gu; p.ldc = H; p.strideC = (int64_t)2 * I * H;
  p.offs = offs; p.groups = E;
  p.M = 2 * I; p.N = H; p.K = P;
  return launch<typename CfgFor<T>::type, T, T, T, false, false, GM_RED, EPI_STORE>(p, s);
}

template <typename TX, typename TW>
hipError_t router_logits_gemm(const TX* x, const TW* w, int T, int H, int E, float* logits, hipStream_t s) {
  GemmParams p = zero_params();
  p.A = x; p.lda = H;
  p.B = w; p.ldb = H;
  p.C = logits; p.ldc = E;
  p.M = T; p.N = E; p.K = H;
  return launch<CfgF32, TX, TW, float, true, true, GM_NONE, EPI_STORE>(p, s);
}

template <typename TX, typename TW>
hipError_t router_dx_gemm(const float* dl, int ldl, const TW* w, int T, int H, int E, TX* dx, hipStream_t s) {
  GemmParams p = zero_params();
  p.A = dl; p.lda = ldl;
  p.B = w; p.ldb = H;  // B[k=e][n=h] = W[e][h]
  p.C = dx; p.ldc = H;
  p.M = T; p.N = H; p.K = E;
  return launch<CfgF32, float, TW, TX, true, false, GM_NONE, EPI_STORE>(p, s);
}

template <typename TX>
hipError_t router_dw_gemm(const float* dl, int ldl, const TX* x, int T, int H, int E, int split_chunk,
                          float* partial, hipStream_t s) {
  GemmParams p = zero_params();
  p.A = dl; p.lda = ldl;  // A[m=e][k=t] = dl[t][e]
  p.B = x; p.ldb = H;     // B[k=t][n=h] = x[t][h]
  p.C = partial; p.ldc = H; p.strideC = (int64_t)E * H;
  p.offs = nullptr; p.split_chunk = split_chunk; p.groups = (T + split_chunk - 1) / split_chunk;
  p.M = E; p.N = H; p.K = T;
  return launch<CfgF32, float, TX, float, false, false, GM_RED, EPI_STORE>(p, s);
}

#define PMOE_INST_EXPERT(T)                                                                                      \
  template hipError_t gate_up_swiglu_fwd<T>(const T*, const T*, const int32_t*, int, int, int, int, T*, T*,      \
                                            hipStream_t);                                                       \
  template hipError_t down_fwd<T>(const T*, const T*, const int32_t*, int, int, int, int, T*, hipStream_t);     \
  template hipError_t down_dgrad_swiglu_bwd<T>(const T*, const T*, const T*, const int32_t*, int, int, int, int, \
                                               T*, hipStream_t);                                                \
  template hipError_t down_wgrad<T>(const T*, const T*, const int32_t*, int, int, int, int, T*, hipStream_t);   \
  template hipError_t gate_up_dgrad<T>(const T*, const T*, const int32_t*, int, int, int, int, T*, hipStream_t); \
  template hipError_t gate_up_wgrad<T>(const T*, const T*, const int32_t*, int, int, int, int, T*, hipStream_t);

PMOE_INST_EXPERT(bf16_t)
PMOE_INST_EXPERT(float)

#define PMOE_INST_ROUTER(TX, TW)                                                                              \
  template hipError_t router_logits_gemm<TX, TW>(const TX*, const TW*, int, int, int, float*, hipStream_t);  \
  template hipError_t router_dx_gemm<TX, TW>(const float*, int, const TW*, int, int, int, TX*, hipStream_t);

PMOE_INST_ROUTER(bf16_t, float)
PMOE_INST_ROUTER(bf16_t, bf16_t)
PMOE_INST_ROUTER(float, float)
PMOE_INST_ROUTER(float, bf16_t)

template hipError_t router_dw_gemm<bf16_t>(const float*, int, const bf16_t*, int, int, int, int, float*,
                                           hipStream_t);
template hipError_t router_dw_gemm<float>(const float*, int, const float*, int, int, int, int, float*,
                                          hipStream_t);

}  // namespace pmoe
