// bf16 grouped GEMM engine for gfx950 with asynchronous global->LDS DMA.
//
// Same problem set as gemm.h (GM_ROWS / GM_RED / GM_NONE, KCONTIG or [k][r]
// operands, fused epilogues) with a different data path:
//  * tiles move HBM -> LDS with buffer_load_dwordx4 ... lds (no staging
//    registers); lanes whose chunk is out of range get a buffer offset past
//    the resource bound, which the hardware turns into zeros;
//  * an NS-stage LDS ring keeps NS-1 k-tiles in flight;
//  * LDS tiles are unpadded and XOR-swizzled at 16-byte granularity:
//      k-contiguous tile [r][64]:  chunk' = chunk ^ ((r >> 1) & 7)
//      [k][r] tile, R columns:     chunk' = chunk ^ (2 * (k & 7))
//    so fragment reads of 16 consecutive lanes hit distinct banks;
//  * fragments of k-contiguous tiles are one ds_read_b128; fragments of [k][r]
//    tiles are two ds_read_b64_tr_b16, which transpose 4x4 blocks of 16-bit
//    elements across each group of 16 lanes (lane q of a group supplies the
//    address of row k0 + q/4, columns r0 + 4(q%4) .. +3, and receives the
//    four k-values of column r0 + q).
#pragma once

#include "gemm.h"

namespace pmoe {

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));

#define PMOE_LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))

constexpr uint32_t kBufOOB = 0xFFFFFFF0u;  // buffer offset past every resource bound

template <int BM_, int BN_, int WM_, int WN_, int NS_>
struct DmaCfg {
  typedef bf16_t Tc;
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, NS = NS_;
  static constexpr int WAVES_M = BM / WM, WAVES_N = BN / WN;
  static constexpr int NW = WAVES_M * WAVES_N;
  static constexpr int NT = kWave * NW;
  static constexpr int MI = WM / 32, NI = WN / 32;
  static constexpr int BK = 64;
  static constexpr int A_BYTES = BM * BK * 2, B_BYTES = BN * BK * 2;
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static constexpr int A_INSTR = BM / 8 / NW, B_INSTR = BN / 8 / NW;  // 1 KB DMA instructions per wave
  static constexpr int D = A_INSTR + B_INSTR;
  static constexpr int EPI_LD = WN + 4;
  static constexpr int EPI_BYTES = NW * 32 * EPI_LD * 4;
  static constexpr int MAIN_BYTES = NS * STAGE_BYTES;
  static constexpr int SMEM_BYTES = MAIN_BYTES > EPI_BYTES ? MAIN_BYTES : EPI_BYTES;
  static_assert(WM % 32 == 0 && WN % 32 == 0 && BM % WM == 0 && BN % WN == 0, "tile shape");
  static_assert(A_INSTR * NW * 8 == BM && B_INSTR * NW * 8 == BN, "DMA instructions must divide among waves");
  static_assert(NS >= 2, "at least double buffering");
};

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef i32x4 BufRsrc;  // buffer resource descriptor (V#), kept in SGPRs

// Raw buffer over [base, base + bytes): stride 0, bound = bytes, dword 3 as
// for untyped raw buffers on gfx9. Offsets at or past the bound read as zero.
__device__ __forceinline__ BufRsrc make_rsrc(const void* base, uint64_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  BufRsrc r;
  r[0] = (int)(uint32_t)a;
  r[1] = (int)((uint32_t)(a >> 32) & 0xffffu);
  r[2] = (int)(bytes > (uint64_t)kBufOOB ? kBufOOB : (uint32_t)bytes);
  r[3] = 0x00020000;
  return r;
}

__device__ __forceinline__ uint32_t lds_addr(const char* p) {
  return (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const char*)p);
}

// One wave-wide 16-byte-per-lane DMA: lane l's chunk goes to lds_dst + 16*l.
// Issued from inline asm so that the compiler adds no waits of its own; every
// consumer waits explicitly with wait_vmcnt<> and a barrier.
// m0 (the LDS destination) is saved and restored inside the statement, so the
// compiler's view of m0 is untouched.
__device__ __forceinline__ void dma16(const BufRsrc& rs, char* lds_dst, uint32_t voff) {
  int saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %2, %3, 0 offen lds\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(__builtin_amdgcn_readfirstlane(lds_addr(lds_dst))), "v"(voff), "s"(rs)
      : "memory");
}

// Block barrier for the DMA pipeline: waits for this wave's LDS reads only
// (lgkmcnt(0)), never for outstanding DMA; fences compiler reordering.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// s_waitcnt vmcnt(n) with the other counters left unconstrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ int swz_t(int k) { return 2 * (k & 7); }

// k-contiguous operand, R rows x 64 k per stage.
template <int R, int NW>
struct KcDma {
  static constexpr int INSTR = R / 8 / NW;
  uint32_t rowoff[INSTR];  // bytes of (row, this lane's chunk) at k = 0, or kBufOOB
  int kc[INSTR];           // this lane's k offset within the stage (8 * logical chunk)

  // row_of(r) -> global storage row of tile row r, or -1 when out of range
  template <class RowFn>
  __device__ __forceinline__ void init(RowFn row_of, int64_t ld, int wave, int lane) {
#pragma unroll
    for (int i = 0; i < INSTR; ++i) {
      const int r = 8 * (wave + i * NW) + (lane >> 3);
      const int c = (lane & 7) ^ ((r >> 1) & 7);
      const int g = row_of(r);
      kc[i] = 8 * c;
      rowoff[i] = g < 0 ? kBufOOB : (uint32_t)(((int64_t)g * ld + 8 * c) * 2);
    }
  }
  __device__ __forceinline__ void issue(const BufRsrc& rs, char* tile, int k0, int k_hi, int wave) const {
#pragma unroll
    for (int i = 0; i < INSTR; ++i) {
      const uint32_t v = (rowoff[i] != kBufOOB && k0 + kc[i] < k_hi) ? rowoff[i] + (uint32_t)(k0 * 2) : kBufOOB;
      dma16(rs, tile + (wave + i * NW) * 1024, v);
    }
  }
};

__device__ __forceinline__ bf16x8 kc_frag(const char* tile, int r, int c) {
  return *reinterpret_cast<const bf16x8*>(tile + r * 128 + ((c ^ ((r >> 1) & 7)) << 4));
}

// [k][r] operand: 64 k-rows x R columns per stage.
template <int R, int NW>
struct TDma {
  static_assert(R >= 128, "[k][r] swizzle needs 16 chunks per row");
  static constexpr int CPR = R / 8;       // 16-byte chunks per k-row
  static constexpr int KPI = 64 / CPR;    // k-rows per 1 KB instruction
  static constexpr int INSTR = R / 8 / NW;
  int kk[INSTR];
  uint32_t coloff[INSTR];  // bytes of this lane's column chunk, or kBufOOB

  __device__ __forceinline__ void init(int r0, int r_limit, int wave, int lane) {
#pragma unroll
    for (int i = 0; i < INSTR; ++i) {
      const int k = (wave + i * NW) * KPI + lane / CPR;
      const int c = (lane % CPR) ^ swz_t(k);
      const int col = r0 + 8 * c;
      kk[i] = k;
      coloff[i] = col < r_limit ? (uint32_t)(col * 2) : kBufOOB;
    }
  }
  __device__ __forceinline__ void issue(const BufRsrc& rs, char* tile, int k0, int k_hi, int64_t ld,
                                        int wave) const {
#pragma unroll
    for (int i = 0; i < INSTR; ++i) {
      const int kg = k0 + kk[i];
      const uint32_t v = (coloff[i] != kBufOOB && kg < k_hi) ? (uint32_t)((int64_t)kg * ld * 2) + coloff[i] : kBufOOB;
      dma16(rs, tile + (wave + i * NW) * 1024, v);
    }
  }
};

template <int R>
__device__ __forceinline__ uint32_t t_addr(int k, int r) {
  return (uint32_t)(k * R * 2 + (((r >> 3) ^ swz_t(k)) << 4) + (r & 7) * 2);
}

// MFMA 32x32x16 operand fragment from a [k][r] tile: rows r_base .. r_base+31,
// k = kbase .. kbase+15 (lane l holds r_base + l%32, k = kbase + 8*(l/32) .. +7).
template <int R>
__device__ __forceinline__ bf16x8 t_frag(const char* tile, int r_base, int kbase, int lane) {
  const int g = lane >> 4, q = lane & 15;
  const int r = r_base + 16 * (g & 1) + 4 * (q & 3);
  const int k = kbase + 8 * (g >> 1) + (q >> 2);
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(tile + t_addr<R>(k, r)));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(tile + t_addr<R>(k + 4, r)));
  const i16x8 v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8, v);
}

// Blocks are dispatched to the 8 XCDs round-robin; give each XCD a contiguous
// range of logical tiles so that tiles sharing operands share an L2.
__device__ __forceinline__ int xcd_remap(int b, int grid) {
  const int per = grid / 8, rem = grid % 8;
  const int xcd = b % 8, idx = b / 8;
  return (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + idx;
}

template <class Cfg, typename Tout, bool A_KC, bool B_KC, int GM, int EPI>
__global__ __launch_bounds__(Cfg::NT) void grouped_gemm_dma_kernel(GemmParams p) {
  constexpr int BM = Cfg::BM, BN = Cfg::BN, NW = Cfg::NW, NS = Cfg::NS;
  constexpr int MI = Cfg::MI, NI = Cfg::NI;
  static_assert(!(GM == GM_RED && (A_KC || B_KC)), "GM_RED expects [k][m] and [k][n] operands");
  static_assert(EPI != EPI_SWIGLU || (B_KC && GM == GM_ROWS && NI % 2 == 0), "SwiGLU epilogue layout");

  __shared__ __attribute__((aligned(1024))) char smem[Cfg::SMEM_BYTES];
  __shared__ int s_scan[1025];
  __shared__ int s_found;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / Cfg::WAVES_N, wn = wave % Cfg::WAVES_N;

  // ---- tile mapping (logical tile id, n fastest)
  const int ntiles_n = (EPI == EPI_SWIGLU) ? (p.inter + BN / 2 - 1) / (BN / 2) : (p.N + BN - 1) / BN;
  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int tn = bid % ntiles_n;
  const int slot = bid / ntiles_n;
  TileInfo ti;
  const bf16_t* A = reinterpret_cast<const bf16_t*>(p.A);
  const bf16_t* B = reinterpret_cast<const bf16_t*>(p.B);
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
      const int splits = p.groups / p.planes;
      A += (int64_t)(g / splits) * p.strideA;
      ti.k_lo = (g % splits) * p.split_chunk;
      ti.k_hi = min(p.K, ti.k_lo + p.split_chunk);
    }
  } else if constexpr (GM == GM_BATCH) {
    const int mt = (p.M + BM - 1) / BM;
    const int g = slot / mt;
    if (g >= p.groups) return;
    ti.group = g; ti.m0 = (slot % mt) * BM; ti.m_end = p.M; ti.k_lo = 0; ti.k_hi = p.K;
    B += (int64_t)g * p.strideB;
  } else {
    ti.group = 0; ti.m0 = slot * BM; ti.m_end = p.M; ti.k_lo = 0; ti.k_hi = p.K;
    if (ti.m0 >= p.M) return;
  }
  ti.n0 = (EPI == EPI_SWIGLU) ? tn * (BN / 2) : tn * BN;

  // ---- operand DMA descriptors, based at the tile's first row (k-contiguous
  // A) or first k (the [k][r] operands of GM_RED) so every offset stays small.
  const bf16_t* a_base = A;
  uint64_t a_bytes = p.a_bytes;
  const bf16_t* b_base = B;
  uint64_t b_bytes = p.b_bytes;
  if constexpr (A_KC) {
    a_base = A + (int64_t)ti.m0 * p.lda;
    a_bytes = (uint64_t)(ti.m_end - ti.m0) * p.lda * 2;
  } else if constexpr (GM == GM_RED) {
    a_base = A + (int64_t)ti.k_lo * p.lda;
    a_bytes = (uint64_t)(ti.k_hi - ti.k_lo) * p.lda * 2;
  }
  if constexpr (GM == GM_RED) {
    b_base = B + (int64_t)ti.k_lo * p.ldb;
    b_bytes = (uint64_t)(ti.k_hi - ti.k_lo) * p.ldb * 2;
  }
  const BufRsrc rsA = make_rsrc(a_base, a_bytes);
  const BufRsrc rsB = make_rsrc(b_base, b_bytes);
  const int k_org = (GM == GM_RED) ? ti.k_lo : 0;  // k of the descriptors' origin
  typedef typename std::conditional<A_KC, KcDma<BM, NW>, TDma<BM, NW>>::type LdA;
  typedef typename std::conditional<B_KC, KcDma<BN, NW>, TDma<BN, NW>>::type LdB;
  LdA la;
  LdB lb;
  if constexpr (A_KC) {
    const int rows = ti.m_end - ti.m0;
    la.init([&](int r) { return r < rows ? r : -1; }, p.lda, wave, lane);
  } else {
    la.init(ti.m0, ti.m_end, wave, lane);
  }
  if constexpr (B_KC) {
    const int n0 = ti.n0, N = p.N, I = p.inter;
    if constexpr (EPI == EPI_SWIGLU) {
      lb.init([&](int c) {
        const int w = c / Cfg::WN, cc = c % Cfg::WN, h = Cfg::WN / 2;
        const int gcol = n0 + w * h + (cc % h);
        if (gcol >= I) return -1;
        return cc < h ? gcol : I + gcol;
      }, p.ldb, wave, lane);
    } else {
      lb.init([&](int c) { return n0 + c < N ? n0 + c : -1; }, p.ldb, wave, lane);
    }
  } else {
    lb.init(ti.n0, p.N, wave, lane);
  }

  f32x16 acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int klen = ti.k_hi - ti.k_lo;
  const int nk = klen > 0 ? (klen + Cfg::BK - 1) / Cfg::BK : 0;

  auto issue = [&](int kt) {
    char* st = smem + (kt % NS) * Cfg::STAGE_BYTES;
    const int k0 = ti.k_lo + kt * Cfg::BK - k_org;  // relative to the descriptors' origin
    const int kh = ti.k_hi - k_org;
    if constexpr (A_KC) la.issue(rsA, st, k0, kh, wave);
    else la.issue(rsA, st, k0, kh, p.lda, wave);
    if constexpr (B_KC) lb.issue(rsB, st + Cfg::A_BYTES, k0, kh, wave);
    else lb.issue(rsB, st + Cfg::A_BYTES, k0, kh, p.ldb, wave);
  };

#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < nk) issue(s);

  const int a_row0 = wm * Cfg::WM, b_row0 = wn * Cfg::WN;
  // Fragments of k-substep ks (16 deep) of the stage at sa / sb.
  auto load_frags = [&](const char* sa, const char* sb, int ks, bf16x8 (&af)[MI], bf16x8 (&bfr)[NI]) {
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      if constexpr (A_KC) af[i] = kc_frag(sa, a_row0 + i * 32 + (lane & 31), ks * 2 + (lane >> 5));
      else af[i] = t_frag<BM>(sa, a_row0 + i * 32, ks * 16, lane);
    }
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      if constexpr (B_KC) bfr[j] = kc_frag(sb, b_row0 + j * 32 + (lane & 31), ks * 2 + (lane >> 5));
      else bfr[j] = t_frag<BN>(sb, b_row0 + j * 32, ks * 16, lane);
    }
  };
  constexpr int KS = Cfg::BK / 16;
  // LDS reads per substep (a [k][r] fragment takes two transposing reads)
  constexpr int NREAD = MI * (A_KC ? 1 : 2) + NI * (B_KC ? 1 : 2);
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + NS - 2 < nk) wait_vmcnt<(NS - 2) * Cfg::D>();
    else wait_vmcnt<0>();
    lds_barrier();
    const char* sa = smem + (kt % NS) * Cfg::STAGE_BYTES;
    const char* sb = sa + Cfg::A_BYTES;
    // Software pipeline over the substeps: the fragments of substep ks + 1 are
    // read while the MFMAs of substep ks run. The first reads go out ahead of
    // the next stage's DMA issue so their latency overlaps it.
    bf16x8 af[2][MI], bfr[2][NI];
    load_frags(sa, sb, 0, af[0], bfr[0]);
    if (kt + NS - 1 < nk) issue(kt + NS - 1);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int cur = ks & 1;
      if (ks + 1 < KS) load_frags(sa, sb, ks + 1, af[cur ^ 1], bfr[cur ^ 1]);
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[cur][i], bfr[cur][j], acc[i][j], 0, 0, 0);
      if (ks + 1 < KS) {
        // interleave: one LDS read, one MFMA, ...; remaining MFMAs after
#pragma unroll
        for (int q = 0; q < (NREAD < MI * NI ? NREAD : MI * NI); ++q) {
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        }
        if constexpr (NREAD < MI * NI) __builtin_amdgcn_sched_group_barrier(0x008, MI * NI - NREAD, 0);
        else if constexpr (NREAD > MI * NI) __builtin_amdgcn_sched_group_barrier(0x100, NREAD - MI * NI, 0);
      }
    }
  }
  wait_vmcnt<0>();
  lds_barrier();
  store_tile<Cfg, Tout, GM, EPI>(acc, reinterpret_cast<float*>(smem), ti, p, wave, wm, wn, lane);
}

template <class Cfg, bool A_KC, bool B_KC, int GM, int EPI, typename Tout = bf16_t>
hipError_t launch_gemm_dma(const GemmParams& p, hipStream_t s) {
  const int ntn = (EPI == EPI_SWIGLU) ? (p.inter + Cfg::BN / 2 - 1) / (Cfg::BN / 2) : (p.N + Cfg::BN - 1) / Cfg::BN;
  int64_t slots;
  if (GM == GM_ROWS) slots = (p.M + Cfg::BM - 1) / Cfg::BM + p.groups;
  else if (GM == GM_RED || GM == GM_BATCH) slots = (int64_t)p.groups * ((p.M + Cfg::BM - 1) / Cfg::BM);
  else slots = (p.M + Cfg::BM - 1) / Cfg::BM;
  const int64_t grid = slots * ntn;
  if (grid <= 0) return hipSuccess;
  if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL((grouped_gemm_dma_kernel<Cfg, Tout, A_KC, B_KC, GM, EPI>), dim3((unsigned)grid), dim3(Cfg::NT), 0,
                     s, p);
  return hipGetLastError();
}

// The six expert GEMMs (see ExpertGemm in gemm.h) on the DMA engine, bf16 only.
template <class Cfg>
hipError_t expert_gemm_dma(int kind, const bf16_t* A, const bf16_t* B, const bf16_t* aux, bf16_t* C, bf16_t* C2,
                           const int32_t* offs, int P, int E, int H, int I, hipStream_t s) {
  GemmParams p = expert_params(kind, A, B, aux, C, C2, offs, P, E, H, I);
  switch (kind) {
    case EG_GATE_UP_FWD: return launch_gemm_dma<Cfg, true, true, GM_ROWS, EPI_SWIGLU>(p, s);
    case EG_DOWN_FWD: return launch_gemm_dma<Cfg, true, true, GM_ROWS, EPI_STORE>(p, s);
    case EG_DOWN_DGRAD: return launch_gemm_dma<Cfg, true, false, GM_ROWS, EPI_SWIGLU_BWD>(p, s);
    case EG_DOWN_WGRAD: return launch_gemm_dma<Cfg, false, false, GM_RED, EPI_STORE>(p, s);
    case EG_GATE_UP_DGRAD: return launch_gemm_dma<Cfg, true, false, GM_ROWS, EPI_STORE>(p, s);
    case EG_GATE_UP_WGRAD: return launch_gemm_dma<Cfg, false, false, GM_RED, EPI_STORE>(p, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace pmoe
