// Launchers of the grouped expert GEMMs and the router GEMMs.
#include <mutex>

#include "gemm_persist.h"
#include "kernels.h"

namespace pmoe {

namespace {

// Tile shapes of the register-staged engine: fp32 (MFMA 32x32x2) uses 64x128
// blocks of four 32x64 wave tiles.
typedef TileCfg<bf16_t, 128, 128, 64, 64> CfgBf16;
typedef TileCfg<float, 64, 128, 32, 64> CfgF32;

template <typename T> struct CfgFor;
template <> struct CfgFor<bf16_t> { typedef CfgBf16 type; };
template <> struct CfgFor<float> { typedef CfgF32 type; };

// bf16 expert GEMMs run on the persistent DMA engine: 256x256 blocks of eight
// 128x64 wave tiles (two waves per SIMD, one block per CU) with a four-stage
// ring of 32-deep k tiles (128 KiB of LDS) and 16-row epilogue slabs (8-row
// for fp32 staging). Chosen by measurement at the Qwen3-30B-A3B shape over
// 128x128 .. 256x256 tilings, 2..5 stages and 32/64-deep k tiles: larger
// tiles fetch fewer bytes per MFMA through each CU's vector-memory path, which
// bounds the smaller ones. A fourth stage does not speed up the k-loop, but
// the next tile's first three stages are then in flight before a tile's
// epilogue stores, which drain while they are used. Against three stages
// (with 128 x 512 tiles covering short last m-tiles in the forward GEMMs,
// whose 40 KiB slots fit only three), same bits, alternating runs on one box:
// the config-2 step -0.4 to -0.8 % on two boxes (down dgrad -2 %, the other
// GEMMs within +-1 %), config 3 -0.8 %, config 4 +0.5 % (its many short last
// m-tiles: gate_up fwd +3 %, down fwd -5 %); fp32 weight gradients the same.
typedef DmaCfg<256, 256, 128, 64, 4, 32, 1> DmaExpert;
// Row-grouped GEMMs whose 256-row tiles would leave whole rounds of the
// persistent walk idle: 128 x 256 blocks of eight 64 x 64 wave tiles (same
// ring and k order, so the same bits). A 128-row tile moves 3/4 of a 256-row
// tile's bytes per stage and, the k-loop being bound by those bytes, takes
// ≈0.75 of its time (measured 0.70-0.77 on one GPU's EP=8 share of config 2),
// so it pays only where it keeps the number of rounds: see use_rows128.
typedef DmaCfg<128, 256, 64, 64, 4, 32, 1> DmaExpert128;
// The router's input gradient: one tile per CU, so no epilogue to hide; the
// three-stage ring as measured.
typedef DmaCfg<256, 256, 128, 64, 3, 32, 1> DmaRouterDx;
// Forward GEMMs of few-token (decode) batches, where each expert holds a few
// rows and the GEMM is a stream of expert weights: 32-row x 128-column blocks
// of four 32x32 wave tiles, 128-deep k stages (256-byte weight-row pieces, which
// stream from HBM ≈15 % faster than the 64-byte pieces of 32-deep stages), a
// three-stage ring (120 KiB). Used when the experts average at most 32 rows.
// Each weight block is read by one tile only, so the weights stream in with
// non-temporal loads.
typedef DmaCfg<32, 128, 32, 32, 3, 128, 1, bf16_t, true> DmaDecode;
constexpr int kDecodeRowsPerExpert = 32;

// The same tile shapes for each 16-bit operand format (fp16 runs the same
// kernels on v_mfma_f32_32x32x16_f16, with fp16 conversions in the epilogues).
template <typename T16> struct PersistCfgs {
  typedef DmaCfg<256, 256, 128, 64, 4, 32, 1, T16> Main;
  typedef DmaCfg<128, 256, 64, 64, 4, 32, 1, T16> Rows128;
  typedef DmaCfg<32, 128, 32, 32, 3, 128, 1, T16, true> Decode;
};
static_assert(std::is_same<PersistCfgs<bf16_t>::Main, DmaExpert>::value &&
                  std::is_same<PersistCfgs<bf16_t>::Rows128, DmaExpert128>::value &&
                  std::is_same<PersistCfgs<bf16_t>::Decode, DmaDecode>::value,
              "one set of tile shapes");

// Compute units of the current device (the persistent kernels launch one
// block per CU), queried once per device and cached.
constexpr int kMaxDevices = 64;
std::once_flag g_cus_once[kMaxDevices];
int g_cus[kMaxDevices];

int num_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  std::call_once(g_cus_once[dev], [dev] {
    int n = 0;
    g_cus[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0
                     ? n : 256;
  });
  return g_cus[dev];
}

// Whether a row-grouped GEMM runs on 128-row tiles: when its estimated rounds
// of tiles per CU, weighted 0.75 for 128-row tiles, come out lower. The host
// has the pair count, not the experts' row counts (those are on the device),
// so each expert is taken to hold P / E rows and its last m-tile half full.
// Only where experts average at least 128 rows (fewer leave a tile's A bytes
// the same in both shapes). The comparison favours GEMMs with few column
// tiles: at one GPU's EP=8 share of config 2 (16 experts, ≈520 rows) down
// dgrad (3 column tiles) fits one round either way and takes 0.75 of the
// time, while gate_up fwd (6) would need two rounds instead of one; configs
// 2-4 keep 256-row tiles throughout.
bool use_rows128(int kind, int P, int E, int H, int I, int cus) {
  if (kind == EG_DOWN_WGRAD || kind == EG_GATE_UP_WGRAD || E <= 0 || P < 128 * E) return false;
  const int ntn = kind == EG_GATE_UP_FWD ? (I + 127) / 128 : (kind == EG_DOWN_DGRAD ? (I + 255) / 256 : (H + 255) / 256);
  const double a = (double)P / E;
  auto rounds = [&](int bm) {
    const double tiles = E * (a / bm + 0.5) * ntn;
    return std::ceil(tiles / cus);
  };
  return 0.75 * rounds(128) < rounds(256);
}

}  // namespace

int expert_gemm_tile_rows(int kind, int P, int E, int H, int I, bool half, int cus) {
  if (!half) return CfgF32::BM;
  if (cus <= 0) cus = num_cus();
  if ((kind == EG_GATE_UP_FWD || kind == EG_DOWN_FWD) && (int64_t)P <= (int64_t)kDecodeRowsPerExpert * E)
    return DmaDecode::BM;
  if (use_rows128(kind, P, E, H, I, cus)) return DmaExpert128::BM;
  return DmaExpert::BM;
}

template <typename T, typename Tw>
hipError_t expert_gemm_run(int kind, const T* A, const T* B, const T* aux, T* C, T* C2, Tw* Cw, const int32_t* offs,
                           int P, int E, int H, int I, const ExpertGather& xg, hipStream_t s) {
  const bool wgrad = kind == EG_DOWN_WGRAD || kind == EG_GATE_UP_WGRAD;
  if constexpr (sizeof(T) == 2) {
    typedef PersistCfgs<T> Cfgs;
    const int rows = expert_gemm_tile_rows(kind, P, E, H, I, true, num_cus());
    if (rows == Cfgs::Decode::BM)
      return expert_gemm_persist_fwd<typename Cfgs::Decode>(kind, A, B, C, C2, offs, P, E, H, I, xg, num_cus(), s);
    if (rows == Cfgs::Rows128::BM)
      return expert_gemm_persist_rows<typename Cfgs::Rows128>(kind, A, B, aux, C, C2, offs, P, E, H, I, xg, num_cus(),
                                                               s);
    return expert_gemm_persist<typename Cfgs::Main, Tw>(kind, A, B, aux, C, C2, Cw, offs, P, E, H, I, xg, num_cus(), s);
  } else {
    static_assert(std::is_same<T, Tw>::value, "fp32 operands give fp32 weight gradients");
    return expert_gemm<typename CfgFor<T>::type, T>(kind, A, B, aux, wgrad ? Cw : C, C2, offs, P, E, H, I, xg, s);
  }
}

template hipError_t expert_gemm_run<bf16_t, bf16_t>(int, const bf16_t*, const bf16_t*, const bf16_t*, bf16_t*, bf16_t*,
                                                    bf16_t*, const int32_t*, int, int, int, int, const ExpertGather&,
                                                    hipStream_t);
template hipError_t expert_gemm_run<bf16_t, float>(int, const bf16_t*, const bf16_t*, const bf16_t*, bf16_t*, bf16_t*,
                                                   float*, const int32_t*, int, int, int, int, const ExpertGather&,
                                                   hipStream_t);
template hipError_t expert_gemm_run<f16_t, f16_t>(int, const f16_t*, const f16_t*, const f16_t*, f16_t*, f16_t*,
                                                  f16_t*, const int32_t*, int, int, int, int, const ExpertGather&,
                                                  hipStream_t);
template hipError_t expert_gemm_run<f16_t, float>(int, const f16_t*, const f16_t*, const f16_t*, f16_t*, f16_t*,
                                                  float*, const int32_t*, int, int, int, int, const ExpertGather&,
                                                  hipStream_t);
template hipError_t expert_gemm_run<float, float>(int, const float*, const float*, const float*, float*, float*,
                                                  float*, const int32_t*, int, int, int, int, const ExpertGather&,
                                                  hipStream_t);

template <typename TX, typename TW>
hipError_t router_logits_gemm(const TX* x, const TW* w, int T, int H, int E, float* logits, hipStream_t s) {
  GemmParams p = zero_params();
  p.A = x; p.lda = H;
  p.B = w; p.ldb = H;
  p.C = logits; p.ldc = E;
  p.M = T; p.N = E; p.K = H;
  return launch_gemm<CfgF32, TX, TW, float, true, true, GM_NONE, EPI_STORE>(p, s);
}

// Router GEMM tile configurations. The logits GEMM from the three bf16 pieces
// of an fp32 weight: 128 x 128 output blocks whose eight 64 x 96 wave tiles
// hold the three pieces of the same 32 columns (the x stage is loaded once for
// all three, and the epilogue sums them). From a bf16 weight (one piece):
// 64 x 64 blocks of four 32 x 32 wave tiles. The weight gradient (a long
// reduction over tokens, split into chunks): 128 x 128 blocks with a 4-deep
// ring. (The input gradient runs on the persistent expert engine.)
typedef DmaCfg<128, 384, 64, 96, 2, 64> DmaRouterLogits3;
typedef DmaCfg<64, 64, 32, 32, 2> DmaRouterLogits;
typedef DmaCfg<128, 128, 64, 64, 4> DmaRouterDw;
// The same one-piece logits and weight-gradient tiles on fp16 operands.
typedef DmaCfg<64, 64, 32, 32, 2, 64, 1, f16_t> DmaRouterLogitsF16;
typedef DmaCfg<128, 128, 64, 64, 4, 64, 1, f16_t> DmaRouterDwF16;

// Router logits x . W^T in fp32 from bf16 x and npieces bf16 pieces of W
// stacked along rows (w3 = [lo; hi; mid], each (E, H), as split_bf16x3 writes
// them; npieces is 1 or 3). Each piece is accumulated over the block's k range
// on its own; the epilogue adds them as (hi + mid) + lo. With splits > 1 the
// reduction over H is split into that many chunks (a multiple of the k tile),
// each writing its own (T, E) plane at parts + s * T * E, which the caller
// sums in order; few tokens give too few blocks to fill the GPU otherwise.
hipError_t router_logits_bf16_pieces(const bf16_t* x, const bf16_t* w3, int npieces, int T, int H, int E,
                                     int splits, float* parts, hipStream_t s) {
  GemmParams p = zero_params();
  p.A = x; p.lda = H;
  p.B = w3; p.ldb = H;
  p.C = parts; p.ldc = E;
  p.M = T; p.N = E; p.K = H;
  p.a_bytes = (uint64_t)T * H * 2; p.b_bytes = (uint64_t)npieces * E * H * 2;
  p.groups = splits;
  p.strideC = (int64_t)T * E;
  if (npieces == 3) {
    constexpr int BK = DmaRouterLogits3::BK;
    p.split_chunk = splits > 1 ? ((H + splits - 1) / splits + BK - 1) / BK * BK : 0;
    return launch_gemm_dma<DmaRouterLogits3, true, true, GM_BATCH, EPI_SUM3, float>(p, s);
  }
  if (npieces != 1) return hipErrorInvalidValue;
  constexpr int BK = DmaRouterLogits::BK;
  p.split_chunk = splits > 1 ? ((H + splits - 1) / splits + BK - 1) / BK * BK : 0;
  return launch_gemm_dma<DmaRouterLogits, true, true, GM_BATCH, EPI_STORE, float>(p, s);
}

// Router logits x . W^T in fp32 from fp16 x and an fp16 W. A product of two
// fp16 values (11-bit significands) is exact in fp32, so one piece on the fp16
// MFMAs gives fp32-accumulated logits of exact products, as the bf16 pieces do.
// The split-K planes are as in router_logits_bf16_pieces with one piece.
hipError_t router_logits_f16(const f16_t* x, const f16_t* w, int T, int H, int E, int splits, float* parts,
                             hipStream_t s) {
  GemmParams p = zero_params();
  p.A = x; p.lda = H;
  p.B = w; p.ldb = H;
  p.C = parts; p.ldc = E;
  p.M = T; p.N = E; p.K = H;
  p.a_bytes = (uint64_t)T * H * 2; p.b_bytes = (uint64_t)E * H * 2;
  p.groups = splits;
  p.strideC = (int64_t)T * E;
  constexpr int BK = DmaRouterLogitsF16::BK;
  p.split_chunk = splits > 1 ? ((H + splits - 1) / splits + BK - 1) / BK * BK : 0;
  return launch_gemm_dma<DmaRouterLogitsF16, true, true, GM_BATCH, EPI_STORE, float>(p, s);
}

// Router backward from bf16 planes (see api.hip): dl3 = [dl_hi | dl_hi | dl_lo]
// (T, 3*ldl), w3t = [W_hi; W_mid; W_hi] (3*ldl, H). dx = dl3 . w3t has the
// expert input-gradient GEMM's form (k-contiguous A, [k][n] B), so it runs on
// the persistent engine as one group of T rows with reduction 3*ldl: its 256 x
// 256 tiles move half the operand bytes of 128 x 128 ones (measured at config
// 2: 24 -> 21.5 us; with one tile per CU the loads, MFMAs and the 33.5 MB of
// stores follow each other rather than overlap). dx is written in TO: bf16,
// or fp16 for an fp16 router (whose weight's bf16 pieces are exact).
template <typename TO>
hipError_t router_dx_bf16(const bf16_t* dl3, int ldl, const bf16_t* w3t, int T, int H, TO* dx, hipStream_t s) {
  static_assert(sizeof(TO) == 2, "16-bit input gradient");
  if ((3 * ldl) % 2) return hipErrorInvalidValue;
  const GemmParams p = expert_params<bf16_t>(EG_GATE_UP_DGRAD, dl3, w3t, nullptr, reinterpret_cast<bf16_t*>(dx),
                                             nullptr, nullptr, T, 1, H, 3 * ldl / 2);
  return launch_gemm_persist<DmaRouterDx, true, false, GM_ROWS, EPI_STORE, TO>(p, num_cus(), s);
}
template hipError_t router_dx_bf16<bf16_t>(const bf16_t*, int, const bf16_t*, int, int, bf16_t*, hipStream_t);
template hipError_t router_dx_bf16<f16_t>(const bf16_t*, int, const bf16_t*, int, int, f16_t*, hipStream_t);

// partial[plane * splits + c] = dl_plane[chunk c]^T . x[chunk c] for the hi and
// lo planes of dl3 (columns 0 and 2*ldl of its rows) -> (2 * splits, E, H) fp32.
hipError_t router_dw_bf16(const bf16_t* dl3, int ldl, const bf16_t* x, int T, int H, int E, int split_chunk,
                          float* partial, hipStream_t s) {
  GemmParams p = zero_params();
  p.A = dl3; p.lda = 3 * ldl;  // A[m=e][k=t] = dl_plane[t][e]
  p.B = x; p.ldb = H;          // B[k=t][n=h]
  p.C = partial; p.ldc = H; p.strideC = (int64_t)E * H;
  const int splits = (T + split_chunk - 1) / split_chunk;
  p.planes = 2; p.strideA = 2 * ldl; p.groups = 2 * splits; p.split_chunk = split_chunk;
  p.M = E; p.N = H; p.K = T;
  p.a_bytes = (uint64_t)T * 3 * ldl * 2; p.b_bytes = (uint64_t)T * H * 2;
  return launch_gemm_dma<DmaRouterDw, false, false, GM_RED, EPI_STORE, float>(p, s);
}

// The fp16 router's weight gradient: dl2 = [dl_hi | dl_lo] (T, 2*ldl) fp16
// planes of the fp32 dl and fp16 x, on the fp16 MFMAs (every product exact).
// partial[plane * splits + c] = dl_plane[chunk c]^T . x[chunk c] -> (2 * splits, E, H) fp32.
hipError_t router_dw_f16(const f16_t* dl2, int ldl, const f16_t* x, int T, int H, int E, int split_chunk,
                         float* partial, hipStream_t s) {
  GemmParams p = zero_params();
  p.A = dl2; p.lda = 2 * ldl;  // A[m=e][k=t] = dl_plane[t][e]
  p.B = x; p.ldb = H;          // B[k=t][n=h]
  p.C = partial; p.ldc = H; p.strideC = (int64_t)E * H;
  const int splits = (T + split_chunk - 1) / split_chunk;
  p.planes = 2; p.strideA = ldl; p.groups = 2 * splits; p.split_chunk = split_chunk;
  p.M = E; p.N = H; p.K = T;
  p.a_bytes = (uint64_t)T * 2 * ldl * 2; p.b_bytes = (uint64_t)T * H * 2;
  return launch_gemm_dma<DmaRouterDwF16, false, false, GM_RED, EPI_STORE, float>(p, s);
}

template <typename TX, typename TW>
hipError_t router_dx_gemm(const float* dl, int ldl, const TW* w, int T, int H, int E, TX* dx, hipStream_t s) {
  GemmParams p = zero_params();
  p.A = dl; p.lda = ldl;
  p.B = w; p.ldb = H;  // B[k=e][n=h] = W[e][h]
  p.C = dx; p.ldc = H;
  p.M = T; p.N = H; p.K = E;
  return launch_gemm<CfgF32, float, TW, TX, true, false, GM_NONE, EPI_STORE>(p, s);
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
  return launch_gemm<CfgF32, float, TX, float, false, false, GM_RED, EPI_STORE>(p, s);
}

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
