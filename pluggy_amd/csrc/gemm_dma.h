// bf16 grouped GEMM engine for gfx950 with asynchronous global->LDS DMA.
//
// Same problem set as gemm.h (GM_ROWS / GM_RED / GM_NONE, KCONTIG or [k][r]
// operands, fused epilogues) with a different data path:
//  * tiles move HBM -> LDS with buffer_load_dwordx4 ... lds (no staging
//    registers); lanes whose chunk is out of range get a buffer offset past
//    the resource bound, which the hardware turns into zeros;
//  * an NS-stage LDS ring of BK-deep k-tiles: the prologue fills every slot,
//    and each slot is refilled as soon as the block has finished reading it,
//    so NS-1 stages are in flight while one is consumed;
//  * LDS tiles are unpadded and XOR-swizzled at 16-byte granularity:
//      k-contiguous tile [r][BK]:  chunk' = chunk ^ (r & 15)         (BK 128)
//                                  chunk' = chunk ^ ((r >> 1) & 7)  (BK 64)
//                                  chunk' = chunk ^ ((r >> 2) & 3)  (BK 32)
//      [k][r] tile, R columns:     chunk' = chunk ^ (4 * (k & 3))
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


// MINB: blocks per CU the register allocation must allow (launch bounds).
// Tc: the 16-bit operand format (bf16_t or f16_t; the persistent engine
// serves both, the kernel in this file bf16 only).
// STREAM_B: B (k-contiguous) is loaded non-temporally (see dma16).
template <int BM_, int BN_, int WM_, int WN_, int NS_, int BK_ = 64, int MINB_ = 1, typename Tc_ = bf16_t,
          bool STREAM_B_ = false>
struct DmaCfg {
  typedef Tc_ Tc;
  static constexpr bool STREAM_B = STREAM_B_;
  static_assert(std::is_same<Tc_, bf16_t>::value || std::is_same<Tc_, f16_t>::value, "16-bit operand format");
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, NS = NS_, BK = BK_, MINB = MINB_;
  static constexpr int WAVES_M = BM / WM, WAVES_N = BN / WN;
  static constexpr int NW = WAVES_M * WAVES_N;
  static constexpr int NT = kWave * NW;
  static constexpr int MI = WM / 32, NI = WN / 32;
  static constexpr int A_BYTES = BM * BK * 2, B_BYTES = BN * BK * 2;
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static constexpr int A_INSTR = A_BYTES / 1024 / NW, B_INSTR = B_BYTES / 1024 / NW;  // 1 KB DMAs per wave
  static constexpr int D = A_INSTR + B_INSTR;  // DMAs per wave per stage
  static constexpr int EPI_LD = WN + 4;
  static constexpr int EPI_BYTES = NW * 32 * EPI_LD * 4;
  static constexpr int MAIN_BYTES = NS * STAGE_BYTES;
  static constexpr int SMEM_BYTES = MAIN_BYTES > EPI_BYTES ? MAIN_BYTES : EPI_BYTES;
  static_assert(WM % 32 == 0 && WN % 32 == 0 && BM % WM == 0 && BN % WN == 0, "tile shape");
  static_assert(BK == 32 || BK == 64 || BK == 128, "k extent of a stage");
  static_assert(A_INSTR * NW * 1024 == A_BYTES && B_INSTR * NW * 1024 == B_BYTES,
                "DMA instructions must divide among waves");
  static_assert(NS >= 2 && (NS - 1) * D < 64, "ring depth");
};

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef i32x4 BufRsrc;  // buffer resource descriptor (V#), kept in SGPRs

// Offsets at or above kOOB lie past every descriptor bound (make_rsrc keeps
// bounds below 2^31) and read as zero; adding a k offset keeps them there.
constexpr uint32_t kOOB = 0x80000000u;

// Raw buffer over [base, base + bytes): stride 0, bound = bytes, dword 3 as
// for untyped raw buffers on gfx9. Offsets at or past the bound read as zero.
// Callers pass wave-uniform values; readfirstlane states that to the compiler,
// so the descriptor stays in SGPRs (the DMA's "s" operand) even when its
// inputs came through LDS.
__device__ __forceinline__ BufRsrc make_rsrc(const void* base, uint64_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  BufRsrc r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  r[1] = __builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xffffu));
  r[2] = __builtin_amdgcn_readfirstlane((int)(bytes >= (uint64_t)kOOB ? kOOB - 16 : (uint32_t)bytes));
  r[3] = 0x00020000;
  return r;
}

__device__ __forceinline__ uint32_t lds_addr(const char* p) {
  return (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const char*)p);
}

// One wave-wide 16-byte-per-lane DMA: lane l's chunk goes to LDS byte address
// lds + 16*l (lds is wave-uniform). Issued from inline asm so that the
// compiler adds no waits of its own; every consumer waits explicitly with
// wait_vmcnt<> and a barrier. m0 (the LDS destination) is an input operand
// of the statement, so the compiler sets it (often computing the address
// straight into m0) and knows what it holds. NTL: a non-temporal (streaming)
// load, for data each tile reads once and no other tile reuses (the weight
// stream of the decode tiles).
template <bool NTL = false>
__device__ __forceinline__ void dma16(const BufRsrc& rs, uint32_t lds, uint32_t voff) {
  if constexpr (NTL)
    asm volatile(
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %0, %1, 0 offen nt lds"
        :
        : "v"(voff), "s"(rs), "{m0}"(lds)
        : "memory");
  else
    asm volatile(
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %0, %1, 0 offen lds"
        :
        : "v"(voff), "s"(rs), "{m0}"(lds)
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

// Wait until at most n stages of D DMAs each are outstanding (n a runtime
// value in [0, NS-1]; the count must be an immediate, hence the switch).
template <int D, int NS>
__device__ __forceinline__ void wait_stages(int n) {
  if constexpr (NS >= 5) { if (n >= 4) { wait_vmcnt<4 * D>(); return; } }
  if constexpr (NS >= 4) { if (n >= 3) { wait_vmcnt<3 * D>(); return; } }
  if constexpr (NS >= 3) { if (n >= 2) { wait_vmcnt<2 * D>(); return; } }
  if (n >= 1) { wait_vmcnt<D>(); return; }
  wait_vmcnt<0>();
}

// [k][r] tiles: a ds_read_b64_tr_b16 half-wave reads 4 consecutive k-rows x 32
// columns (4 chunks per row); shifting the chunk by 4 per k (mod 4) puts those
// 16 chunks in 16 distinct 16-byte bank groups.
__device__ __forceinline__ int swz_t(int k) { return 4 * (k & 3); }

// k-contiguous tiles, rows of BK bf16 (CPR = BK/8 chunks): the chunk is XORed
// with a function of the row so that 16 consecutive rows at one logical chunk
// fall in 16 distinct 16-byte bank groups.
template <int BK>
__device__ __forceinline__ int swz_kc(int r) {
  if constexpr (BK == 128) return r & 15;
  else if constexpr (BK == 64) return (r >> 1) & 7;
  else return (r >> 2) & 3;
}

// k-contiguous operand, R rows x BK k per stage; instruction i of wave w fills
// rows [(w + i*NW) * RPI, +RPI) with RPI = 512 / BK.
template <int R, int NW, int BK>
struct KcDma {
  static constexpr int CPR = BK / 8, RPI = 512 / BK;
  static constexpr int INSTR = R / RPI / NW;
  uint32_t rowoff[INSTR];  // bytes of (row, this lane's chunk) at k = 0, or kOOB
  int kc[INSTR];           // this lane's k offset within the stage

  // row_of(r) -> storage row of tile row r relative to the descriptor base, or -1
  template <class RowFn>
  __device__ __forceinline__ void init(RowFn row_of, int64_t ld, int wave, int lane) {
#pragma unroll
    for (int i = 0; i < INSTR; ++i) {
      const int r = RPI * (wave + i * NW) + lane / CPR;
      const int c = (lane % CPR) ^ swz_kc<BK>(r);
      const int g = row_of(r);
      kc[i] = 8 * c;
      rowoff[i] = g < 0 ? kOOB : (uint32_t)(((int64_t)g * ld + 8 * c) * 2);
    }
  }
  // Row gather: tile row r (< rows) is storage row idx[m0 + r] of the
  // descriptor. The RPI rows of an instruction are consecutive, so their
  // indices come through the scalar cache (uniform addresses, clamped into the
  // table) and each lane picks its own; m0 must be wave-uniform.
  __device__ __forceinline__ void init_gather(const int32_t* idx, int64_t n_idx, int m0, int rows, int64_t ld,
                                              int wave, int lane) {
    typedef const __attribute__((address_space(4))) int32_t cint;
    cint* ci = (cint*)idx;  // wave-uniform reads through the scalar cache
    const int64_t last = n_idx - 1;
#pragma unroll
    for (int i = 0; i < INSTR; ++i) {
      const int rb = RPI * (wave + i * NW);
      const int sel = lane / CPR;
      int tok = 0;
#pragma unroll
      for (int j = 0; j < RPI; ++j) {
        const int v = ci[min<int64_t>((int64_t)m0 + rb + j, last)];
        tok = sel == j ? v : tok;
      }
      const int r = rb + sel;
      const int c = (lane % CPR) ^ swz_kc<BK>(r);
      kc[i] = 8 * c;
      rowoff[i] = r < rows ? (uint32_t)(((int64_t)tok * ld + 8 * c) * 2) : kOOB;
    }
  }
  // this = second ? y : x, element by element (stays in registers)
  __device__ __forceinline__ void select(bool second, const KcDma& y, const KcDma& x) {
#pragma unroll
    for (int i = 0; i < INSTR; ++i) {
      rowoff[i] = second ? y.rowoff[i] : x.rowoff[i];
      kc[i] = second ? y.kc[i] : x.kc[i];
    }
  }
  // k0: first k of the stage relative to the descriptor; tail: the stage
  // reaches past k_hi (only then are lanes checked one by one).
  // instruction I of the stage at LDS byte address tile
  template <int I, bool NTL = false>
  __device__ __forceinline__ void issue1(const BufRsrc& rs, uint32_t tile, int k0, int k_hi, bool tail,
                                         int wave) const {
    uint32_t v = rowoff[I] + (uint32_t)(k0 * 2);
    if (tail && k0 + kc[I] >= k_hi) v = kOOB;
    dma16<NTL>(rs, tile + (wave + I * NW) * 1024, v);
  }
};

template <int BK>
__device__ __forceinline__ bf16x8 kc_frag(const char* tile, int r, int c) {
  return *reinterpret_cast<const bf16x8*>(tile + r * (BK * 2) + ((c ^ swz_kc<BK>(r)) << 4));
}

// [k][r] operand: BK k-rows x R columns per stage; instruction i of wave w
// fills k-rows [(w + i*NW) * KPI, +KPI) with KPI = 512 / R. k-rows past the
// descriptor bound read as zero, so ragged reduction ranges need no checks.
template <int R, int NW, int BK>
struct TDma {
  static_assert(R >= 128, "[k][r] swizzle needs 16 chunks per row");
  static constexpr int CPR = R / 8;       // 16-byte chunks per k-row
  static constexpr int KPI = 512 / R;     // k-rows per 1 KB instruction
  static constexpr int INSTR = BK / KPI / NW;
  static_assert(INSTR * KPI * NW == BK, "[k][r] DMA instructions must divide among waves");
  int kk[INSTR];
  uint32_t coloff[INSTR];  // bytes of this lane's column chunk, or kOOB

  __device__ __forceinline__ void init(int r0, int r_limit, int wave, int lane) {
#pragma unroll
    for (int i = 0; i < INSTR; ++i) {
      const int k = (wave + i * NW) * KPI + lane / CPR;
      const int c = (lane % CPR) ^ swz_t(k);
      const int col = r0 + 8 * c;
      kk[i] = k;
      coloff[i] = col < r_limit ? (uint32_t)(col * 2) : kOOB;
    }
  }
  __device__ __forceinline__ void select(bool second, const TDma& y, const TDma& x) {
#pragma unroll
    for (int i = 0; i < INSTR; ++i) {
      kk[i] = second ? y.kk[i] : x.kk[i];
      coloff[i] = second ? y.coloff[i] : x.coloff[i];
    }
  }
  template <int I>
  __device__ __forceinline__ void issue1(const BufRsrc& rs, uint32_t tile, int k0, int64_t ld, int wave) const {
    dma16(rs, tile + (wave + I * NW) * 1024, (uint32_t)((int64_t)(k0 + kk[I]) * ld * 2) + coloff[I]);
  }
  // k-row gather: the k-row of instruction I is storage row tok0 for lanes
  // 0-31 and tok1 for lanes 32-63 (the caller's wave-uniform tokens of its two
  // k-rows); k-rows at or past k_hi read zero. ld2: bytes per storage row. The
  // offset is a 32-bit buffer offset, so the row's byte offset is formed in 32
  // bits (the same value the instruction takes from 64-bit arithmetic). Both
  // k-rows' offsets and range checks are wave-uniform scalar work; a lane then
  // picks its half's offset and adds its column with a saturating add, so an
  // out-of-range row or column (kOOB) stays past every bound.
  template <int I>
  __device__ __forceinline__ void issue1_rows(const BufRsrc& rs, uint32_t tile, int k0, int k_hi, int tok0,
                                              int tok1, uint32_t ld2, int wave, int lane) const {
    static_assert(KPI == 2 && CPR == 32, "one k-row per half-wave");
    const int kr = k0 + (wave + I * NW) * KPI;  // the half-waves' k-rows: kr, kr + 1
    const uint32_t r0 = kr < k_hi ? (uint32_t)tok0 * ld2 : kOOB;
    const uint32_t r1 = kr + 1 < k_hi ? (uint32_t)tok1 * ld2 : kOOB;
    const uint32_t v = __builtin_elementwise_add_sat(lane < 32 ? r0 : r1, coloff[I]);
    dma16(rs, tile + (wave + I * NW) * 1024, v);
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

// The same fragment from a lane offset computed once: the swizzle depends on
// k only through k & 3, which a k base of 16 ks and the +4 of the second read
// leave unchanged, so the fragment at k base 16 ks lies at the lane's offset
// for k base 0 (t_lane_off) plus 16 ks k-rows, a constant the reads take as
// their immediate offset.
template <int R>
__device__ __forceinline__ uint32_t t_lane_off(int r_base, int lane) {
  const int g = lane >> 4, q = lane & 15;
  return t_addr<R>(8 * (g >> 1) + (q >> 2), r_base + 16 * (g & 1) + 4 * (q & 3));
}
template <int R>
__device__ __forceinline__ bf16x8 t_frag_at(const char* tile, uint32_t lane_off, int ks) {
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  const char* p = tile + lane_off + ks * 16 * R * 2;
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)p);
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p + 4 * R * 2));
  const i16x8 v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8, v);
}

// 8 consecutive outputs from fp32: bf16 through the native converter, or fp32.
template <typename Tout> struct Out8;
template <> struct Out8<bf16_t> {
  __device__ static __forceinline__ u32x4 pack(const float* v) {
    u32x4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = cvt_pk_bf16(v[2 * i], v[2 * i + 1]);
    return w;
  }
  __device__ static __forceinline__ void store(bf16_t* p, const float* v) { *reinterpret_cast<u32x4*>(p) = pack(v); }
};
template <> struct Out8<f16_t> {
  __device__ static __forceinline__ u32x4 pack(const float* v) {
    u32x4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = cvt_pk_f16(v[2 * i], v[2 * i + 1]);
    return w;
  }
  __device__ static __forceinline__ void store(f16_t* p, const float* v) { *reinterpret_cast<u32x4*>(p) = pack(v); }
};
template <> struct Out8<float> {
  __device__ static __forceinline__ void store(float* p, const float* v) { Vec8<float>::store(p, v); }
};

// 8 packed 16-bit values (format T16) to fp32.
template <typename T16 = bf16_t>
__device__ __forceinline__ void unpack8(const u32x4& w, float* v) {
#pragma unroll
  for (int i = 0; i < 4; ++i) { v[2 * i] = Fmt16<T16>::lo(w[i]); v[2 * i + 1] = Fmt16<T16>::hi(w[i]); }
}

// One 32x32x16 MFMA on 16-bit fragments of format T16 (the fragments travel
// as bf16x8 bit patterns through LDS and registers).
template <typename T16>
__device__ __forceinline__ f32x16 mfma16(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  if constexpr (std::is_same<T16, f16_t>::value)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Epilogue of the DMA engine. Each wave moves its accumulators to HBM one
// 32-row slab at a time through its own LDS region (no block barriers): lanes
// write their MFMA columns as fp32, then read back 8 consecutive columns of a
// row with 16-byte LDS reads, convert with v_cvt_pk_bf16_f32 and store 16-byte
// vectors (or 16 bytes of fp32 per half row). The router's logits GEMM sums
// its three weight pieces here (EPI_SUM3).
template <class Cfg, typename Tout, int GM, int EPI>
__device__ __forceinline__ void store_tile_dma(const f32x16 (&acc)[Cfg::MI][Cfg::NI], float* smem_f,
                                               const TileInfo& ti, const GemmParams& p, int wave, int wm, int wn,
                                               int lane) {
  constexpr int MI = Cfg::MI, NI = Cfg::NI, LD = Cfg::EPI_LD;
  // EPI_SUM3: the wave's three 32-column blocks are the three weight pieces of
  // the same 32 output columns, [lo; hi; mid]; they are summed (hi + mid) + lo.
  constexpr int WN = EPI == EPI_SUM3 ? 32 : Cfg::WN;
  static_assert(LD % 4 == 0, "16-byte aligned staging rows");
  static_assert(EPI == EPI_STORE || EPI == EPI_SUM3, "the router GEMMs store plainly or sum weight pieces");
  static_assert(EPI != EPI_SUM3 || NI == 3, "EPI_SUM3 takes three pieces per wave");
  float* stage = smem_f + wave * 32 * LD;
  Tout* C = reinterpret_cast<Tout*>(p.C);
  if constexpr (GM == GM_RED || GM == GM_BATCH) C += (int64_t)ti.group * p.strideC;
  const int half = lane >> 5, col_l = lane & 31;
#pragma unroll
  for (int i = 0; i < MI; ++i) {
    if constexpr (EPI == EPI_SUM3) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          stage[(8 * q + 4 * half + r) * LD + col_l] =
              (acc[i][1][4 * q + r] + acc[i][2][4 * q + r]) + acc[i][0][4 * q + r];
    } else {
#pragma unroll
      for (int j = 0; j < NI; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int r = 0; r < 4; ++r) stage[(8 * q + 4 * half + r) * LD + j * 32 + col_l] = acc[i][j][4 * q + r];
    }
    __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0): slab written
    asm volatile("" ::: "memory");
    const int row_base = ti.m0 + wm * Cfg::WM + i * 32;
    constexpr int CPR = WN / 8;
    const int col_base = ti.n0 + wn * WN;
#pragma unroll
    for (int e = lane; e < 32 * CPR; e += 64) {
      const int r = e / CPR, c = (e % CPR) * 8;
      const int row = row_base + r, col = col_base + c;
      if (row < ti.m_end && col < p.N) {
        float v[8];
        Vec8<float>::load(stage + r * LD + c, v);
        if (col + 8 <= p.N) {
          Out8<Tout>::store(C + (int64_t)row * p.ldc + col, v);
        } else {
          for (int t = 0; col + t < p.N; ++t) store_scalar<Tout>(C + (int64_t)row * p.ldc + col + t, v[t]);
        }
      }
    }
  }
}

// Compile-time loop: f(integral_constant<int, B>), ..., f(integral_constant<int, E-1>).
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>());
    static_for<B + 1, E>(f);
  }
}

// Blocks are dispatched to the 8 XCDs round-robin; give each XCD a contiguous
// range of logical tiles so that tiles sharing operands share an L2.
__device__ __forceinline__ int xcd_remap(int b, int grid) {
  const int per = grid / 8, rem = grid % 8;
  const int xcd = b % 8, idx = b / 8;
  return (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + idx;
}

// GM_ROWS tile scan: s_scan[g] = first m-tile of group g (s_scan[groups] =
// total m-tiles), computed by wave 0 from the inclusive end offsets; every
// thread returns the total. s_scan holds >= groups+1 ints.
template <int BM>
__device__ __forceinline__ int rows_scan(const int32_t* offs, int groups, int* s_scan) {
  const int tid = threadIdx.x, lane = tid & 63;
  if (tid < 64) {
    int carry = 0;
    for (int base = 0; base < groups; base += 64) {
      const int g = base + lane;
      int tiles = 0;
      if (g < groups) {
        const int lo = g == 0 ? 0 : offs[g - 1];
        tiles = (offs[g] - lo + BM - 1) / BM;
      }
      const int inc = wave_incl_scan(tiles, lane) + carry;
      if (g < groups) s_scan[g + 1] = inc;
      carry = __shfl(inc, 63, kWave);
    }
    if (lane == 0) s_scan[0] = 0;
  }
  __syncthreads();
  return s_scan[groups];
}

// Group of m-tile `slot` (binary search over the scan; slot < total).
__device__ __forceinline__ int rows_group(const int* s_scan, int groups, int slot) {
  int lo = 0, hi = groups - 1;  // the group g with s_scan[g] <= slot < s_scan[g + 1]
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (s_scan[mid] <= slot) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// Logical tile of this block when `total` tiles are spread over the 8 XCDs
// (blocks reach XCD blockIdx % 8): XCD x takes a contiguous share of
// total/8 (+1) tiles, so neighbouring tiles share its L2 and every XCD gets
// the same amount of work. -1: no tile for this block.
__device__ __forceinline__ int xcd_tile(int b, int total) {
  const int x = b & 7, i = b >> 3;
  const int per = total >> 3, rem = total & 7;
  const int cnt = per + (x < rem ? 1 : 0);
  if (i >= cnt) return -1;
  return x * per + (x < rem ? x : rem) + i;
}

template <class Cfg, typename Tout, bool A_KC, bool B_KC, int GM, int EPI>
__global__ __launch_bounds__(Cfg::NT, Cfg::MINB) void grouped_gemm_dma_kernel(GemmParams p) {
  constexpr int BM = Cfg::BM, BN = Cfg::BN, BK = Cfg::BK, NW = Cfg::NW, NS = Cfg::NS, D = Cfg::D;
  constexpr int MI = Cfg::MI, NI = Cfg::NI;
  static_assert(!(GM == GM_RED && (A_KC || B_KC)), "GM_RED expects [k][m] and [k][n] operands");
  static_assert(EPI != EPI_SUM3 || (B_KC && Cfg::WN == 96), "EPI_SUM3: three 32-row pieces per wave");

  __shared__ __attribute__((aligned(1024))) char smem[Cfg::SMEM_BYTES];
  __shared__ int s_scan[1025];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / Cfg::WAVES_N, wn = wave % Cfg::WAVES_N;

  // ---- tile mapping (logical tile id, n fastest)
  // EPI_SUM3 tiles cover BN / 3 output columns (three weight pieces each)
  constexpr int TN = EPI == EPI_SUM3 ? BN / 3 : BN;
  const int ntiles_n = (p.N + TN - 1) / TN;
  TileInfo ti;
  const bf16_t* A = reinterpret_cast<const bf16_t*>(p.A);
  const bf16_t* B = reinterpret_cast<const bf16_t*>(p.B);
  int tn, slot;
  if constexpr (GM == GM_ROWS) {
    // the grid covers the worst case; only the real tiles are spread over XCDs
    const int mtiles = rows_scan<BM>(p.offs, p.groups, s_scan);
    const int bid = xcd_tile(blockIdx.x, mtiles * ntiles_n);
    if (bid < 0) return;
    tn = bid % ntiles_n;
    slot = bid / ntiles_n;
    const int g = rows_group(s_scan, p.groups, slot);
    const int lo = g == 0 ? 0 : p.offs[g - 1];
    ti.group = g; ti.m0 = lo + (slot - s_scan[g]) * BM; ti.m_end = p.offs[g]; ti.k_lo = 0; ti.k_hi = p.K;
    B += (int64_t)g * p.strideB;
  } else {
    const int bid = xcd_remap(blockIdx.x, gridDim.x);
    tn = bid % ntiles_n;
    slot = bid / ntiles_n;
  }
  if constexpr (GM == GM_ROWS) {
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
    if (p.split_chunk > 0) {  // split-K: group g reduces k in [g * chunk, (g + 1) * chunk)
      ti.k_lo = min(p.K, g * p.split_chunk);
      ti.k_hi = min(p.K, ti.k_lo + p.split_chunk);
    }
    B += (int64_t)g * p.strideB;
  } else {
    ti.group = 0; ti.m0 = slot * BM; ti.m_end = p.M; ti.k_lo = 0; ti.k_hi = p.K;
    if (ti.m0 >= p.M) return;
  }
  ti.n0 = tn * TN;

  // ---- operand DMA descriptors. k-contiguous A is based at the tile's first
  // row and bounded by the group's last row; the [k][r] operands of GM_RED are
  // based at the group's first k and bounded by its last, so rows and k past
  // the group read as zero.
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
  typedef typename std::conditional<A_KC, KcDma<BM, NW, BK>, TDma<BM, NW, BK>>::type LdA;
  typedef typename std::conditional<B_KC, KcDma<BN, NW, BK>, TDma<BN, NW, BK>>::type LdB;
  auto init_a = [&](LdA& la, int vw) {
    if constexpr (A_KC) {
      const int rows = ti.m_end - ti.m0;
      la.init([&](int r) { return r < rows ? r : -1; }, p.lda, vw, lane);
    } else {
      la.init(ti.m0, ti.m_end, vw, lane);
    }
  };
  auto init_b = [&](LdB& lb, int vw) {
    if constexpr (B_KC) {
      const int n0 = ti.n0, N = p.N;
      if constexpr (EPI == EPI_SUM3) {
        // B = [piece 0; piece 1; piece 2], each N rows; tile row c feeds wave
        // c / 96, piece (c % 96) / 32, output column n0 + 32 * wave + c % 32
        lb.init([&](int c) {
          const int w = c / Cfg::WN, cc = c % Cfg::WN;
          const int col = n0 + 32 * w + (cc & 31);
          return col < N ? (cc >> 5) * N + col : -1;
        }, p.ldb, vw, lane);
      } else {
        lb.init([&](int c) { return n0 + c < N ? n0 + c : -1; }, p.ldb, vw, lane);
      }
    } else {
      lb.init(ti.n0, p.N, vw, lane);
    }
  };
  LdA la0;
  LdB lb0;
  init_a(la0, wave);
  init_b(lb0, wave);

  f32x16 acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int klen = ti.k_hi - ti.k_lo;
  const int nk = klen > 0 ? (klen + BK - 1) / BK : 0;
  const uint32_t lds0 = lds_addr(smem);
  // descriptors of GM_RED start at k_lo; the others at k = 0
  const int kd0 = (GM == GM_RED) ? 0 : ti.k_lo;
  const int kd_hi = ti.k_hi - ((GM == GM_RED) ? ti.k_lo : 0);

  // DMA instruction J (0 .. D-1) of stage kt: A's instructions, then B's.
  auto dma_share = [&](int kt, auto jc, const LdA& la, const LdB& lb, int vw) {
    constexpr int J = decltype(jc)::value;
    const uint32_t st = lds0 + (uint32_t)((kt % NS) * Cfg::STAGE_BYTES);
    const int k0 = kd0 + kt * BK;
    if constexpr (J < Cfg::A_INSTR) {
      if constexpr (A_KC) la.template issue1<J>(rsA, st, k0, kd_hi, k0 + BK > kd_hi, vw);
      else la.template issue1<J>(rsA, st, k0, p.lda, vw);
    } else {
      constexpr int JB = J - Cfg::A_INSTR;
      if constexpr (B_KC) lb.template issue1<JB>(rsB, st + Cfg::A_BYTES, k0, kd_hi, k0 + BK > kd_hi, vw);
      else lb.template issue1<JB>(rsB, st + Cfg::A_BYTES, k0, p.ldb, vw);
    }
  };
  auto dma_one = [&](int kt, auto jc) { dma_share(kt, jc, la0, lb0, wave); };
  auto issue = [&](int kt) { static_for<0, D>([&](auto jc) { dma_one(kt, jc); }); };

  const int a_row0 = wm * Cfg::WM, b_row0 = wn * Cfg::WN;
  // Fragments of k-substep ks (16 deep) of the stage at sa / sb.
  auto load_frags = [&](const char* sa, const char* sb, int ks, bf16x8 (&af)[MI], bf16x8 (&bfr)[NI]) {
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      if constexpr (A_KC) af[i] = kc_frag<BK>(sa, a_row0 + i * 32 + (lane & 31), ks * 2 + (lane >> 5));
      else af[i] = t_frag<BM>(sa, a_row0 + i * 32, ks * 16, lane);
    }
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      if constexpr (B_KC) bfr[j] = kc_frag<BK>(sb, b_row0 + j * 32 + (lane & 31), ks * 2 + (lane >> 5));
      else bfr[j] = t_frag<BN>(sb, b_row0 + j * 32, ks * 16, lane);
    }
  };
  constexpr int KS = BK / 16;
  static_assert(KS % 2 == 0, "fragment double buffer assumes an even number of substeps");
  // MFMAs of a stage before its end-of-stage barrier; the D DMAs of the stage
  // being refilled are spread evenly among them (several follow one MFMA when
  // a stage has more DMAs than MFMAs).
  constexpr int TOTM = (KS - 1) * MI * NI;
  static_assert(TOTM >= 1, "the DMAs of a stage need MFMA slots");

  // MFMAs of substep KSC (a compile-time constant); with DMA_ST >= 0 the DMAs
  // of stage DMA_ST whose slots fall in this substep follow their MFMA.
  auto substep = [&](auto ksc, const bf16x8 (&af)[MI], const bf16x8 (&bfr)[NI], int dma_st) {
    constexpr int KSI = decltype(ksc)::value;
    static_for<0, MI * NI>([&](auto mc) {
      constexpr int M = decltype(mc)::value;
      acc[M / NI][M % NI] = mfma16<typename Cfg::Tc>(af[M / NI], bfr[M % NI], acc[M / NI][M % NI]);
      constexpr int G = KSI * MI * NI + M;  // MFMA index within the stage
      static_for<0, D>([&](auto dc) {
        constexpr int DI = decltype(dc)::value;
        if constexpr ((DI * TOTM) / D == G) {
          if (dma_st >= 0) dma_one(dma_st, dc);
        }
      });
    });
  };

  // ---- pipeline. The prologue fills all NS ring slots. During stage kt the
  // DMAs of stage kt-1+NS (into the slot stage kt-1 used) are interleaved
  // with the MFMAs, so address issue overlaps matrix work. At the end of each
  // stage but the last (before its last substep's MFMAs) every wave waits for
  // stage kt+1 and the block synchronises (which also retires every read of
  // stage kt and makes stage kt+1 visible); the first fragments of stage kt+1
  // are read while the last MFMAs of stage kt run. The loop body is
  // straight-line code; the last stage is peeled.
#pragma unroll
  for (int s0 = 0; s0 < NS; ++s0)
    if (s0 < nk) issue(s0);
  bf16x8 af[2][MI], bfr[2][NI];
  if (nk > 0) {
    wait_stages<D, NS>(min(NS, nk) - 1);
    lds_barrier();
    load_frags(smem, smem + Cfg::A_BYTES, 0, af[0], bfr[0]);
  }
  for (int kt = 0; kt + 1 < nk; ++kt) {
    const char* sa = smem + (kt % NS) * Cfg::STAGE_BYTES;
    const char* sb = sa + Cfg::A_BYTES;
    const int dma_st = (kt >= 1 && kt - 1 + NS < nk) ? kt - 1 + NS : -1;
    static_for<0, KS - 1>([&](auto ksc) {
      constexpr int KSI = decltype(ksc)::value;
      load_frags(sa, sb, KSI + 1, af[(KSI + 1) & 1], bfr[(KSI + 1) & 1]);
      substep(ksc, af[KSI & 1], bfr[KSI & 1], dma_st);
    });
    // stages kt+2 .. min(kt+NS-1, nk-1) may stay in flight
    wait_stages<D, NS>(min(NS - 1, nk - 1 - kt) - 1);
    lds_barrier();
    const char* na = smem + ((kt + 1) % NS) * Cfg::STAGE_BYTES;
    load_frags(na, na + Cfg::A_BYTES, 0, af[0], bfr[0]);
    substep(std::integral_constant<int, KS - 1>(), af[1], bfr[1], -1);
  }
  if (nk > 0) {
    const char* sa = smem + ((nk - 1) % NS) * Cfg::STAGE_BYTES;
    const char* sb = sa + Cfg::A_BYTES;
    static_for<0, KS>([&](auto ksc) {
      constexpr int KSI = decltype(ksc)::value;
      if constexpr (KSI + 1 < KS) load_frags(sa, sb, KSI + 1, af[(KSI + 1) & 1], bfr[(KSI + 1) & 1]);
      substep(ksc, af[KSI & 1], bfr[KSI & 1], -1);
    });
  }
  wait_vmcnt<0>();
  lds_barrier();
  store_tile_dma<Cfg, Tout, GM, EPI>(acc, reinterpret_cast<float*>(smem), ti, p, wave, wm, wn, lane);
}

template <class Cfg, bool A_KC, bool B_KC, int GM, int EPI, typename Tout = bf16_t>
hipError_t launch_gemm_dma(const GemmParams& p, hipStream_t s) {
  constexpr int TN = EPI == EPI_SUM3 ? Cfg::BN / 3 : Cfg::BN;
  const int ntn = (p.N + TN - 1) / TN;
  int64_t slots;
  if (GM == GM_ROWS) slots = (p.M + Cfg::BM - 1) / Cfg::BM + p.groups;
  else if (GM == GM_RED || GM == GM_BATCH) slots = (int64_t)p.groups * ((p.M + Cfg::BM - 1) / Cfg::BM);
  else slots = (p.M + Cfg::BM - 1) / Cfg::BM;
  int64_t grid = slots * ntn;
  if (grid <= 0) return hipSuccess;
  if (GM == GM_ROWS) grid = (grid + 7) / 8 * 8;  // xcd_tile spreads up to 8*ceil(tiles/8) blocks
  if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL((grouped_gemm_dma_kernel<Cfg, Tout, A_KC, B_KC, GM, EPI>), dim3((unsigned)grid), dim3(Cfg::NT), 0,
                     s, p);
  return hipGetLastError();
}

}  // namespace pmoe
