// Grouped GEMM engine for the MoE expert FFN on CDNA4 MFMA.
//
// C[m, n] = sum_k A[m, k] * B[k, n] over a set of groups:
//   GM_ROWS : groups partition the rows m (expert-contiguous token rows); each
//             group has its own B (an expert's weight). Forward and dgrad.
//   GM_RED  : groups partition the reduction index k; each group writes its own
//             C (an expert's weight gradient). Wgrad, and split-K.
//   GM_NONE : one plain GEMM.
// Operands are row-major in HBM. "KCONTIG" means the operand's k index is the
// contiguous one (A stored [m][k], B stored [n][k]); otherwise the operand is
// stored [k][m] / [k][n] and is transposed in registers while it is staged into
// LDS. LDS tiles are always [row][k] so every MFMA fragment is one vector read.
//
// Compute types: bf16 (v_mfma_f32_32x32x16_bf16) and fp32
// (v_mfma_f32_32x32x2_f32); both accumulate in fp32.
#pragma once

#include <type_traits>

#include "common.h"

namespace pmoe {

// GM_BATCH: per-group B and C (strideB, strideC) over a shared A; with
// split_chunk > 0 group g instead reduces k in [g * split_chunk, ...), a
// split-K whose partial products land in separate C planes.
enum GroupMode { GM_NONE = 0, GM_ROWS = 1, GM_RED = 2, GM_BATCH = 3 };
enum EpiKind { EPI_STORE = 0, EPI_SWIGLU = 1, EPI_SWIGLU_BWD = 2, EPI_SUM3 = 3 };

template <typename Tc> struct Mfma;

template <> struct Mfma<bf16_t> {
  static constexpr int KPACK = 8;  // consecutive k per lane in one fragment
  static constexpr int MK = 16;    // k extent of one MFMA
  static constexpr int BK = 64;    // k extent of one LDS stage (128 B per row)
  static constexpr int PADK = 8;   // row padding (16 B) against bank conflicts
  typedef bf16x8 frag_t;
  __device__ static __forceinline__ frag_t load(const bf16_t* p) {
    return *reinterpret_cast<const bf16x8*>(p);
  }
  __device__ static __forceinline__ f32x16 mma(frag_t a, frag_t b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

template <> struct Mfma<float> {
  static constexpr int KPACK = 1;
  static constexpr int MK = 2;
  static constexpr int BK = 32;
  static constexpr int PADK = 4;
  typedef float frag_t;
  __device__ static __forceinline__ frag_t load(const float* p) { return *p; }
  __device__ static __forceinline__ f32x16 mma(frag_t a, frag_t b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
};

template <typename Tc_, int BM_, int BN_, int WM_, int WN_>
struct TileCfg {
  typedef Tc_ Tc;
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_;
  static constexpr int WAVES_M = BM / WM, WAVES_N = BN / WN;
  static constexpr int NT = kWave * WAVES_M * WAVES_N;
  static constexpr int MI = WM / 32, NI = WN / 32;
  static constexpr int BK = Mfma<Tc>::BK;
  static constexpr int LDK = BK + Mfma<Tc>::PADK;
  static constexpr int STAGE_ELEMS = (BM + BN) * LDK;
  static constexpr int EPI_LD = WN + 4;  // fp32 staging row stride (floats)
  static constexpr int EPI_BYTES = WAVES_M * WAVES_N * 32 * EPI_LD * 4;
  static constexpr int MAIN_BYTES = 2 * STAGE_ELEMS * (int)sizeof(Tc);
  static constexpr int SMEM_BYTES = MAIN_BYTES > EPI_BYTES ? MAIN_BYTES : EPI_BYTES;
  static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile is a multiple of the 32x32 MFMA");
  static_assert(BM % WM == 0 && BN % WN == 0, "block tile is a multiple of the wave tile");
};

// ------------------------------------------------------------- staging ----

// Element conversion of one 16-byte global chunk into LDS elements.
template <typename Tg, typename Tc> struct ChunkCvt;
template <> struct ChunkCvt<bf16_t, bf16_t> {
  __device__ static __forceinline__ void put(bf16_t* dst, u32x4 v) { *reinterpret_cast<u32x4*>(dst) = v; }
};
template <> struct ChunkCvt<float, float> {
  __device__ static __forceinline__ void put(float* dst, u32x4 v) { *reinterpret_cast<u32x4*>(dst) = v; }
};
template <> struct ChunkCvt<bf16_t, float> {  // 8 bf16 -> 8 fp32 (exact)
  __device__ static __forceinline__ void put(float* dst, u32x4 v) {
    u32x4 lo, hi;
    lo[0] = v[0] << 16; lo[1] = v[0] & 0xffff0000u; lo[2] = v[1] << 16; lo[3] = v[1] & 0xffff0000u;
    hi[0] = v[2] << 16; hi[1] = v[2] & 0xffff0000u; hi[2] = v[3] << 16; hi[3] = v[3] & 0xffff0000u;
    reinterpret_cast<u32x4*>(dst)[0] = lo;
    reinterpret_cast<u32x4*>(dst)[1] = hi;
  }
};

// Operand whose k index is contiguous in HBM: rows of R x BK, 16-byte chunks.
template <typename Tg, typename Tc, int R, int BK, int LDK, int NT>
struct KContigStager {
  static constexpr int VEC = 16 / (int)sizeof(Tg);
  static constexpr int CPR = BK / VEC;  // chunks per row
  static constexpr int CHUNKS = R * CPR;
  static constexpr int PER_T = (CHUNKS + NT - 1) / NT;
  const Tg* rowp[PER_T];  // row base pointer, or nullptr when the row is out of range
  u32x4 reg[PER_T];

  // rowptr(r) -> pointer to element (r, 0) of the tile's row r, or nullptr.
  template <class RowFn>
  __device__ __forceinline__ void init(RowFn rowptr, int tid) {
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      int c = tid + i * NT;
      rowp[i] = (c < CHUNKS) ? rowptr(c / CPR) : nullptr;
    }
  }
  __device__ __forceinline__ void load(int k0, int k_hi, int tid) {
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      int c = tid + i * NT;
      int k = k0 + (c % CPR) * VEC;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (rowp[i] != nullptr && k < k_hi) v = *reinterpret_cast<const u32x4*>(rowp[i] + k);
      reg[i] = v;
    }
  }
  __device__ __forceinline__ void store(Tc* lds, int tid) const {
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      int c = tid + i * NT;
      if (CHUNKS % NT == 0 || c < CHUNKS)
        ChunkCvt<Tg, Tc>::put(lds + (c / CPR) * LDK + (c % CPR) * VEC, reg[i]);
    }
  }
};

// Transpose of one VEC x VEC register block: in[j] holds k = j, r = 0..VEC-1;
// writes LDS row r with k = 0..VEC-1.
template <typename Tg, typename Tc> struct BlockT;
template <> struct BlockT<bf16_t, bf16_t> {
  __device__ static __forceinline__ void put(bf16_t* dst, int ldk, const u32x4* in) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      u32x4 o;
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        uint32_t a = in[2 * p][c >> 1], b = in[2 * p + 1][c >> 1];
        o[p] = (c & 1) ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
      }
      *reinterpret_cast<u32x4*>(dst + c * ldk) = o;
    }
  }
};
template <> struct BlockT<bf16_t, float> {
  __device__ static __forceinline__ void put(float* dst, int ldk, const u32x4* in) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      u32x4 lo, hi;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t a = in[j][c >> 1], b = in[4 + j][c >> 1];
        lo[j] = (c & 1) ? (a & 0xffff0000u) : (a << 16);
        hi[j] = (c & 1) ? (b & 0xffff0000u) : (b << 16);
      }
      reinterpret_cast<u32x4*>(dst + c * ldk)[0] = lo;
      reinterpret_cast<u32x4*>(dst + c * ldk)[1] = hi;
    }
  }
};
template <> struct BlockT<float, float> {
  __device__ static __forceinline__ void put(float* dst, int ldk, const u32x4* in) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      u32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = in[j][c];
      *reinterpret_cast<u32x4*>(dst + c * ldk) = o;
    }
  }
};

// First n (< 16 / sizeof(T)) elements of a 16-byte chunk, the rest zero.
template <typename T>
__device__ __forceinline__ u32x4 load_partial16(const T* p, int n) {
  union { u32x4 v; T e[16 / sizeof(T)]; } u;
  u.v = u32x4{0u, 0u, 0u, 0u};
  for (int i = 0; i < n; ++i) u.e[i] = p[i];
  return u.v;
}

// Operand stored [k][r] (r contiguous): VEC k-rows x VEC r-columns per unit.
// Consecutive threads take consecutive k-blocks of the same r-block so that
// each global load instruction reads 128-byte row segments.
template <typename Tg, typename Tc, int R, int BK, int LDK, int NT>
struct TransStager {
  static constexpr int VEC = 16 / (int)sizeof(Tg);
  static constexpr int UK = BK / VEC;
  static constexpr int UR = R / VEC;
  static constexpr int UNITS = UK * UR;
  static constexpr int PER_T = (UNITS + NT - 1) / NT;
  static_assert(BK % VEC == 0 && R % VEC == 0, "tile not a multiple of the transpose block");
  const Tg* base;
  int64_t ld;
  int r0, r_hi;
  const int32_t* kidx;  // k-row k is row kidx[k] of base (nullptr: row k)
  u32x4 reg[PER_T][VEC];

  __device__ __forceinline__ void init(const Tg* base_, int64_t ld_, int r0_, int r_hi_,
                                       const int32_t* kidx_ = nullptr) {
    base = base_; ld = ld_; r0 = r0_; r_hi = r_hi_; kidx = kidx_;
  }
  __device__ __forceinline__ void load(int k0, int k_hi, int tid) {
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      int u = tid + i * NT;
      int kb = u % UK, rb = u / UK;
      int r = r0 + rb * VEC;
      bool ok_r = (UNITS % NT == 0 || u < UNITS) && r < r_hi;
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        int k = k0 + kb * VEC + j;
        u32x4 v = {0u, 0u, 0u, 0u};
        if (ok_r && k < k_hi) {
          const Tg* src = base + (int64_t)(kidx != nullptr ? kidx[k] : k) * ld + r;
          if (r + VEC <= r_hi) v = *reinterpret_cast<const u32x4*>(src);
          else v = load_partial16(src, r_hi - r);
        }
        reg[i][j] = v;
      }
    }
  }
  __device__ __forceinline__ void store(Tc* lds, int tid) const {
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      int u = tid + i * NT;
      if (UNITS % NT == 0 || u < UNITS) {
        int kb = u % UK, rb = u / UK;
        BlockT<Tg, Tc>::put(lds + (rb * VEC) * LDK + kb * VEC, LDK, reg[i]);
      }
    }
  }
};

// --------------------------------------------------------------- params ----

struct GemmParams {
  const void* A; int64_t lda;
  const void* B; int64_t ldb; int64_t strideB;  // per-group B stride (GM_ROWS)
  void* C; int64_t ldc; int64_t strideC;        // per-group C stride (GM_RED)
  void* C2; int64_t ldc2;                       // SwiGLU: the activation output
  const void* aux; int64_t ldaux;               // SwiGLU backward: the pre-activation
  const int32_t* offs;  // inclusive end offset per group (nullptr: uniform split_chunk)
  int groups;
  int M, N, K;          // see GroupMode; GM_RED: M x N per group, K = total reduction
  int split_chunk;
  int inter;            // SwiGLU: I (columns of gate; up starts at I)
  uint64_t a_bytes;     // extent of A's storage (from A), and of one group's B (from B + g*strideB)
  uint64_t b_bytes;
  int planes;           // GM_RED uniform split: groups = planes * splits, plane g / splits reads A + plane * strideA
  int64_t strideA;
  // Row gathers of a token-major operand (the expert-sorted rows are never
  // materialised): with a_index, row p of A (GM_ROWS) or k-row p of A (GM_RED)
  // is row a_index[p] of A's storage, which holds a_rows rows; b_index / b_rows
  // likewise for the k-rows of B (GM_RED). a_index / b_index hold P entries.
  const int32_t* a_index; int64_t a_rows;
  const int32_t* b_index; int64_t b_rows;
  int64_t n_index;      // entries of a_index / b_index (P)
  // Epilogue extras. row_w[p]: the routing weight of output row p; EPI_SWIGLU
  // writes mid = row_w * silu(g) * u, EPI_SWIGLU_BWD takes the accumulators as
  // the gradient of that scaled activation. part: with EPI_SWIGLU_BWD and
  // row_w, part[p * part_ld + c / 64] = sum over the 64 columns c.. of the
  // accumulators times silu(g) * u (the routing weight's gradient, by block).
  const float* row_w;
  float* part; int part_ld;
};

struct TileInfo {
  int m0, m_end;   // output rows [m0, m_end) valid
  int n0;          // output column base (SwiGLU: gate column base)
  int k_lo, k_hi;  // reduction range
  int group;
};

// GM_ROWS: map a linear m-tile slot to (group, first row). Returns false when
// the slot is past the last tile. s_scan must hold >= groups+1 ints.
template <int BM>
__device__ bool rows_tile_lookup(const int32_t* offs, int groups, int slot, int* s_scan,
                                 int* s_found, int& group, int& row0, int& row_end) {
  const int tid = threadIdx.x, lane = tid & 63;
  if (tid < 64) {
    int carry = 0;
    for (int base = 0; base < groups; base += 64) {
      int g = base + lane;
      int tiles = 0;
      if (g < groups) {
        int lo = g == 0 ? 0 : offs[g - 1];
        tiles = (offs[g] - lo + BM - 1) / BM;
      }
      int inc = wave_incl_scan(tiles, lane) + carry;
      if (g < groups) s_scan[g + 1] = inc;
      carry = __shfl(inc, 63, kWave);
    }
    if (lane == 0) { s_scan[0] = 0; *s_found = -1; }
  }
  __syncthreads();
  const int total = s_scan[groups];
  if (slot >= total) return false;
  for (int g = tid; g < groups; g += blockDim.x)
    if (s_scan[g] <= slot && slot < s_scan[g + 1]) *s_found = g;
  __syncthreads();
  group = *s_found;
  int lo = group == 0 ? 0 : offs[group - 1];
  row0 = lo + (slot - s_scan[group]) * BM;
  row_end = offs[group];
  return true;
}

// ------------------------------------------------------------- epilogue ----

template <typename Tout>
__device__ __forceinline__ float round_to(float v) {
  if constexpr (sizeof(Tout) == 2) return bf16_to_f32(f32_to_bf16(v));
  else return v;
}

// Epilogue shared by the GEMM engines: each wave stages its accumulators one
// 32-row slab at a time through LDS (fp32), then writes rows with 16-byte
// vector stores, applying the fused SwiGLU forward / backward when asked.
template <class Cfg, typename Tout, int GM, int EPI>
__device__ __forceinline__ void store_tile(const f32x16 (&acc)[Cfg::MI][Cfg::NI], float* smem_f, const TileInfo& ti,
                                          const GemmParams& p, int wave, int wm, int wn, int lane) {
  constexpr int MI = Cfg::MI, NI = Cfg::NI;
  float* stage = smem_f + wave * 32 * Cfg::EPI_LD;
  Tout* C = reinterpret_cast<Tout*>(p.C);
  if constexpr (GM == GM_RED || GM == GM_BATCH) C += (int64_t)ti.group * p.strideC;
  constexpr int WN = Cfg::WN;

#pragma unroll
  for (int i = 0; i < MI; ++i) {
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          stage[(8 * q + 4 * (lane >> 5) + r) * Cfg::EPI_LD + j * 32 + (lane & 31)] = acc[i][j][4 * q + r];
    __syncthreads();
    const int row_base = ti.m0 + wm * Cfg::WM + i * 32;
    if constexpr (EPI == EPI_SWIGLU) {
      constexpr int H2 = WN / 2, CPR = H2 / 8;
      Tout* MID = reinterpret_cast<Tout*>(p.C2);
      const int col_base = ti.n0 + wn * H2;
      for (int e = lane; e < 32 * CPR; e += 64) {
        const int r = e / CPR, c = (e % CPR) * 8;
        const int row = row_base + r, col = col_base + c;
        if (row < ti.m_end && col < p.inter) {
          float g[8], u[8], m[8];
          const float ws = p.row_w != nullptr ? p.row_w[row] : 1.0f;
#pragma unroll
          for (int t = 0; t < 8; ++t) {
            g[t] = round_to<Tout>(stage[r * Cfg::EPI_LD + c + t]);
            u[t] = round_to<Tout>(stage[r * Cfg::EPI_LD + H2 + c + t]);
            m[t] = g[t] * sigmoidf_(g[t]) * u[t] * ws;
          }
          Vec8<Tout>::store(C + (int64_t)row * p.ldc + col, g);
          Vec8<Tout>::store(C + (int64_t)row * p.ldc + p.inter + col, u);
          Vec8<Tout>::store(MID + (int64_t)row * p.ldc2 + col, m);
        }
      }
    } else {
      constexpr int CPR = WN / 8;
      static_assert(EPI != EPI_SWIGLU_BWD || WN == 64, "routing-weight partials are per 64-column block");
      const int col_base = ti.n0 + wn * WN;
      for (int e = lane; e < 32 * CPR; e += 64) {
        const int r = e / CPR, c = (e % CPR) * 8;
        const int row = row_base + r, col = col_base + c;
        float pd = 0.0f;  // this lane's share of <acc, silu(g) u> (EPI_SWIGLU_BWD with row_w)
        if (row < ti.m_end && col < p.N) {
          float v[8];
#pragma unroll
          for (int t = 0; t < 8; ++t) v[t] = stage[r * Cfg::EPI_LD + c + t];
          if constexpr (EPI == EPI_SWIGLU_BWD) {
            // v = d(mid), or with row_w d(w * mid); aux row holds [gate | up] pre-activations.
            const Tout* GU = reinterpret_cast<const Tout*>(p.aux) + (int64_t)row * p.ldaux;
            float g[8], u[8], dg[8], du[8];
            Vec8<Tout>::load(GU + col, g);
            Vec8<Tout>::load(GU + p.inter + col, u);
            const float ws = p.row_w != nullptr ? p.row_w[row] : 1.0f;
#pragma unroll
            for (int t = 0; t < 8; ++t) {
              const float s = sigmoidf_(g[t]);
              const float silu = g[t] * s;
              const float dsilu = s * (1.0f + g[t] * (1.0f - s));
              pd += v[t] * (silu * u[t]);
              const float dm = v[t] * ws;
              dg[t] = dm * u[t] * dsilu;
              du[t] = dm * silu;
            }
            Vec8<Tout>::store(C + (int64_t)row * p.ldc + col, dg);
            Vec8<Tout>::store(C + (int64_t)row * p.ldc + p.inter + col, du);
          } else if (col + 8 <= p.N) {
            Vec8<Tout>::store(C + (int64_t)row * p.ldc + col, v);
          } else {
            for (int t = 0; col + t < p.N; ++t) store_scalar<Tout>(C + (int64_t)row * p.ldc + col + t, v[t]);
          }
        }
        if constexpr (EPI == EPI_SWIGLU_BWD) {
          if (p.part != nullptr) {  // the CPR = 8 lanes of a row are consecutive: sum them in a fixed order
            pd += __shfl_xor(pd, 1);
            pd += __shfl_xor(pd, 2);
            pd += __shfl_xor(pd, 4);
            if ((e % CPR) == 0 && row < ti.m_end && col_base < p.N)
              p.part[(int64_t)row * p.part_ld + col_base / 64] = pd;
          }
        }
      }
    }
    __syncthreads();
  }
}

// ----------------------------------------------------------------- kernel ----

template <class Cfg, typename TA, typename TB, typename Tout, bool A_KC, bool B_KC, int GM, int EPI>
__global__ __launch_bounds__(Cfg::NT) void grouped_gemm_kernel(GemmParams p) {
  typedef typename Cfg::Tc Tc;
  typedef Mfma<Tc> MF;
  constexpr int BM = Cfg::BM, BN = Cfg::BN, BK = Cfg::BK, LDK = Cfg::LDK, NT = Cfg::NT;
  constexpr int MI = Cfg::MI, NI = Cfg::NI;
  static_assert(!(GM == GM_RED && (A_KC || B_KC)), "GM_RED expects [k][m] and [k][n] operands");
  static_assert(EPI != EPI_SWIGLU || (B_KC && GM == GM_ROWS), "SwiGLU epilogue is the gate_up forward");
  static_assert(EPI != EPI_SWIGLU || (Cfg::NI % 2 == 0), "SwiGLU pairs gate and up halves of a wave tile");

  __shared__ __attribute__((aligned(16))) char smem[Cfg::SMEM_BYTES];
  __shared__ int s_scan[1025];
  __shared__ int s_found;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / Cfg::WAVES_N, wn = wave % Cfg::WAVES_N;

  // ---- tile mapping
  const int ntiles_n = (EPI == EPI_SWIGLU) ? (p.inter + BN / 2 - 1) / (BN / 2) : (p.N + BN - 1) / BN;
  const int bid = blockIdx.x;
  const int tn = bid % ntiles_n;
  const int slot = bid / ntiles_n;
  TileInfo ti;
  const TA* A = reinterpret_cast<const TA*>(p.A);
  const TB* B = reinterpret_cast<const TB*>(p.B);
  if constexpr (GM == GM_ROWS) {
    int g, r0, re;
    if (!rows_tile_lookup<BM>(p.offs, p.groups, slot, s_scan, &s_found, g, r0, re)) return;
    ti.group = g; ti.m0 = r0; ti.m_end = re; ti.k_lo = 0; ti.k_hi = p.K;
    B += (int64_t)g * p.strideB;
  } else if constexpr (GM == GM_RED) {
    const int mt = (p.M + BM - 1) / BM;
    const int g = slot / mt;
    if (g >= p.groups) return;
    ti.group = g; ti.m0 = (slot % mt) * BM; ti.m_end = p.M;
    if (p.offs != nullptr) {
      ti.k_lo = g == 0 ? 0 : p.offs[g - 1];
      ti.k_hi = p.offs[g];
    } else {
      ti.k_lo = g * p.split_chunk;
      ti.k_hi = min(p.K, ti.k_lo + p.split_chunk);
    }
  } else {
    ti.group = 0; ti.m0 = slot * BM; ti.m_end = p.M; ti.k_lo = 0; ti.k_hi = p.K;
    if (ti.m0 >= p.M) return;
  }
  ti.n0 = (EPI == EPI_SWIGLU) ? tn * (BN / 2) : tn * BN;

  // LDS stage s holds the A tile at [s*STAGE_ELEMS] and the B tile right after it.
  // Addresses are always formed from the __shared__ base so they stay in the
  // LDS address space (ds_read/ds_write, not flat accesses).
  Tc* const lds = reinterpret_cast<Tc*>(smem);

  // ---- operand stagers
  typedef typename std::conditional<A_KC, KContigStager<TA, Tc, BM, BK, LDK, NT>,
                                    TransStager<TA, Tc, BM, BK, LDK, NT>>::type StA;
  typedef typename std::conditional<B_KC, KContigStager<TB, Tc, BN, BK, LDK, NT>,
                                    TransStager<TB, Tc, BN, BK, LDK, NT>>::type StB;
  StA sa;
  StB sb;
  if constexpr (A_KC) {
    const int m0 = ti.m0, me = ti.m_end;
    const int64_t lda = p.lda;
    const int32_t* ai = p.a_index;
    sa.init([&](int r) -> const TA* {
      return (m0 + r < me) ? A + (int64_t)(ai != nullptr ? ai[m0 + r] : m0 + r) * lda : nullptr;
    }, tid);
  } else {
    sa.init(A, p.lda, ti.m0, ti.m_end, p.a_index);
  }
  if constexpr (B_KC) {
    const int n0 = ti.n0, N = p.N, I = p.inter;
    const int64_t ldb = p.ldb;
    if constexpr (EPI == EPI_SWIGLU) {
      // Block column c -> B row: each wave's WN columns are WN/2 gate rows then
      // the WN/2 matching up rows (offset I), so one lane holds both halves.
      sb.init([&](int c) -> const TB* {
        int w = c / Cfg::WN, cc = c % Cfg::WN, h = Cfg::WN / 2;
        int gcol = n0 + w * h + (cc % h);
        if (gcol >= I) return nullptr;
        int row = (cc < h) ? gcol : I + gcol;
        return B + (int64_t)row * ldb;
      }, tid);
    } else {
      sb.init([&](int c) -> const TB* { return (n0 + c < N) ? B + (int64_t)(n0 + c) * ldb : nullptr; }, tid);
    }
  } else {
    sb.init(B, p.ldb, ti.n0, p.N, p.b_index);
  }

  f32x16 acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int klen = ti.k_hi - ti.k_lo;
  const int nk = klen > 0 ? (klen + BK - 1) / BK : 0;

  if (nk > 0) {
    sa.load(ti.k_lo, ti.k_hi, tid);
    sb.load(ti.k_lo, ti.k_hi, tid);
    sa.store(lds, tid);
    sb.store(lds + BM * LDK, tid);
  }
  __syncthreads();

  const int frag_row = lane & 31;
  const int frag_k = (lane >> 5) * MF::KPACK;
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) {
      sa.load(ti.k_lo + (kt + 1) * BK, ti.k_hi, tid);
      sb.load(ti.k_lo + (kt + 1) * BK, ti.k_hi, tid);
    }
    const Tc* a_base = lds + cur * Cfg::STAGE_ELEMS + (wm * Cfg::WM + frag_row) * LDK + frag_k;
    const Tc* b_base = lds + cur * Cfg::STAGE_ELEMS + BM * LDK + (wn * Cfg::WN + frag_row) * LDK + frag_k;
#pragma unroll
    for (int ks = 0; ks < BK / MF::MK; ++ks) {
      typename MF::frag_t af[MI], bf[NI];
#pragma unroll
      for (int i = 0; i < MI; ++i) af[i] = MF::load(a_base + i * 32 * LDK + ks * MF::MK);
#pragma unroll
      for (int j = 0; j < NI; ++j) bf[j] = MF::load(b_base + j * 32 * LDK + ks * MF::MK);
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) acc[i][j] = MF::mma(af[i], bf[j], acc[i][j]);
    }
    if (kt + 1 < nk) {
      sa.store(lds + (cur ^ 1) * Cfg::STAGE_ELEMS, tid);
      sb.store(lds + (cur ^ 1) * Cfg::STAGE_ELEMS + BM * LDK, tid);
    }
    __syncthreads();
  }

  // ---- epilogue: stage each 32-row slab of the wave tile through LDS as fp32
  store_tile<Cfg, Tout, GM, EPI>(acc, reinterpret_cast<float*>(smem), ti, p, wave, wm, wn, lane);
}

// ------------------------------------------------------------- launchers ----

inline GemmParams zero_params() {
  GemmParams p;
  p.A = nullptr; p.lda = 0;
  p.B = nullptr; p.ldb = 0; p.strideB = 0;
  p.C = nullptr; p.ldc = 0; p.strideC = 0;
  p.C2 = nullptr; p.ldc2 = 0;
  p.aux = nullptr; p.ldaux = 0;
  p.offs = nullptr; p.groups = 1;
  p.M = p.N = p.K = 0; p.split_chunk = 0; p.inter = 0;
  p.a_bytes = p.b_bytes = 0;
  p.planes = 1; p.strideA = 0;
  p.a_index = nullptr; p.a_rows = 0;
  p.b_index = nullptr; p.b_rows = 0;
  p.n_index = 0;
  p.row_w = nullptr;
  p.part = nullptr; p.part_ld = 0;
  return p;
}

template <class Cfg, typename TA, typename TB, typename Tout, bool A_KC, bool B_KC, int GM, int EPI>
hipError_t launch_gemm(const GemmParams& p, hipStream_t s) {
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

// Problem description of one expert GEMM. A, B: operands as listed above;
// aux: gu for EG_DOWN_DGRAD; C2: mid for EG_GATE_UP_FWD.
template <typename T>
GemmParams expert_params(int kind, const T* A, const T* B, const T* aux, T* C, T* C2, const int32_t* offs, int P,
                         int E, int H, int I, const ExpertGather& xg = ExpertGather()) {
  GemmParams p = zero_params();
  const uint64_t es = sizeof(T);
  p.offs = offs;
  p.groups = E;
  p.A = A;
  p.B = B;
  p.C = C;
  switch (kind) {
    case EG_GATE_UP_FWD:
      p.lda = H; p.ldb = H; p.strideB = (int64_t)2 * I * H;
      p.ldc = 2 * I; p.C2 = C2; p.ldc2 = I;
      p.M = P; p.N = 2 * I; p.K = H; p.inter = I;
      p.a_bytes = (uint64_t)P * H * es; p.b_bytes = (uint64_t)2 * I * H * es;
      break;
    case EG_DOWN_FWD:
      p.lda = I; p.ldb = I; p.strideB = (int64_t)H * I;
      p.ldc = H;
      p.M = P; p.N = H; p.K = I;
      p.a_bytes = (uint64_t)P * I * es; p.b_bytes = (uint64_t)H * I * es;
      break;
    case EG_DOWN_DGRAD:  // B[k=h][n=i] = W_dn[e][h][i]
      p.lda = H; p.ldb = I; p.strideB = (int64_t)H * I;
      p.ldc = 2 * I; p.aux = aux; p.ldaux = 2 * I;
      p.M = P; p.N = I; p.K = H; p.inter = I;
      p.a_bytes = (uint64_t)P * H * es; p.b_bytes = (uint64_t)H * I * es;
      break;
    case EG_DOWN_WGRAD:  // A[m=h][k=p] = dy[p][h], B[k=p][n=i] = mid[p][i]
      p.lda = H; p.ldb = I;
      p.ldc = I; p.strideC = (int64_t)H * I;
      p.M = H; p.N = I; p.K = P;
      p.a_bytes = (uint64_t)P * H * es; p.b_bytes = (uint64_t)P * I * es;
      break;
    case EG_GATE_UP_DGRAD:  // B[k=j][n=h] = W_gu[e][j][h]
      p.lda = 2 * I; p.ldb = H; p.strideB = (int64_t)2 * I * H;
      p.ldc = H;
      p.M = P; p.N = H; p.K = 2 * I;
      p.a_bytes = (uint64_t)P * 2 * I * es; p.b_bytes = (uint64_t)2 * I * H * es;
      break;
    case EG_GATE_UP_WGRAD:  // A[m=j][k=p] = dgu[p][j], B[k=p][n=h] = x_perm[p][h]
      p.lda = 2 * I; p.ldb = H;
      p.ldc = H; p.strideC = (int64_t)2 * I * H;
      p.M = 2 * I; p.N = H; p.K = P;
      p.a_bytes = (uint64_t)P * 2 * I * es; p.b_bytes = (uint64_t)P * H * es;
      break;
  }
  if (xg.index != nullptr) {
    p.n_index = P;
    if (kind == EG_GATE_UP_WGRAD) {
      p.b_index = xg.index; p.b_rows = xg.rows; p.b_bytes = (uint64_t)xg.rows * p.ldb * es;
    } else if (kind == EG_GATE_UP_FWD || kind == EG_DOWN_DGRAD || kind == EG_DOWN_WGRAD) {
      p.a_index = xg.index; p.a_rows = xg.rows; p.a_bytes = (uint64_t)xg.rows * p.lda * es;
    }
  }
  if (kind == EG_GATE_UP_FWD || kind == EG_DOWN_DGRAD) p.row_w = xg.row_w;
  if (kind == EG_DOWN_DGRAD) { p.part = xg.part; p.part_ld = xg.part_ld; }
  return p;
}

template <class Cfg, typename T>
hipError_t expert_gemm(int kind, const T* A, const T* B, const T* aux, T* C, T* C2, const int32_t* offs, int P,
                       int E, int H, int I, const ExpertGather& xg, hipStream_t s) {
  const GemmParams p = expert_params<T>(kind, A, B, aux, C, C2, offs, P, E, H, I, xg);
  switch (kind) {
    case EG_GATE_UP_FWD: return launch_gemm<Cfg, T, T, T, true, true, GM_ROWS, EPI_SWIGLU>(p, s);
    case EG_DOWN_FWD: return launch_gemm<Cfg, T, T, T, true, true, GM_ROWS, EPI_STORE>(p, s);
    case EG_DOWN_DGRAD: return launch_gemm<Cfg, T, T, T, true, false, GM_ROWS, EPI_SWIGLU_BWD>(p, s);
    case EG_DOWN_WGRAD: return launch_gemm<Cfg, T, T, T, false, false, GM_RED, EPI_STORE>(p, s);
    case EG_GATE_UP_DGRAD: return launch_gemm<Cfg, T, T, T, true, false, GM_ROWS, EPI_STORE>(p, s);
    case EG_GATE_UP_WGRAD: return launch_gemm<Cfg, T, T, T, false, false, GM_RED, EPI_STORE>(p, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace pmoe
