// Persistent grouped GEMM for the six expert GEMMs (GM_ROWS and GM_RED) and
// the router's input gradient (GM_ROWS, one group).
//
// One block per CU loops over the tiles of its XCD. The tile list holds each
// group's tiles together (GM_ROWS: n-tile major, see rows_tile; GM_RED: m-tile
// major); XCD x owns a contiguous share of it, and block i of the XCD takes
// tiles i, i + nb, i + 2 nb, ... of that share (nb = blocks on the XCD), so at
// any moment the XCD's CUs work on neighbouring tiles that share operands in
// its L2 (GM_RED under skew deals them differently, see below). Per block, the
// expert offsets are read into LDS and scanned once; a tile's group is then a
// binary search in LDS.
//
// The k loop is the ring pipeline of grouped_gemm_dma_kernel with a global
// stage counter, so ring slots carry over from one tile to the next: stage
// kt+NS-1 is issued during stage kt, and in a tile's last NS-1 stages that is
// one of the next tile's first stages, so the next tile's data lands while
// this tile finishes and stores. The epilogue stages accumulators through a
// separate per-wave LDS region of 16- or 8-row slabs and never touches the
// ring. The expert GEMMs run on a four-slot ring, the router's input gradient
// (one tile per CU) on three.
#pragma once

#include "gemm_dma.h"

namespace pmoe {

template <class Cfg>
struct PersistLayout {
  static constexpr int EPI_LD = Cfg::WN + 4;  // floats per staged fp32 row
  static_assert(EPI_LD % 4 == 0, "16-byte aligned staging rows");
};

// Lane l receives lane (l ^ 1)'s value (DPP quad permutation 1, 0, 3, 2).
__device__ __forceinline__ float swap_lane_pair(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));
}

// Epilogue through per-wave slabs of SLAB rows (16, or 8 where fp32 staging
// sits beside a four-slot ring): slab (i, s) holds rows SLAB s .. SLAB s +
// SLAB - 1 of the wave's 32-row block i. In the MFMA 32x32 layout lane half h
// holds rows 8 q + 4 h + r (r = 0..3) of a block, so slab s gathers the SLAB /
// 8 values of q from (SLAB / 8) s on: local row 8 (q - (SLAB / 8) s) + 4 h + r.
// Each lane then reads 8 consecutive outputs and stores 16 bytes.
//
// bf16 outputs (all but the SwiGLU backward's) round in registers and stage
// packed: lanes 2c and 2c + 1 hold columns 2c and 2c + 1 of the same four
// rows, so they swap half of their values and each writes two dwords of
// (column 2c, 2c + 1) pairs, rows 0-1 from the even lane and rows 2-3 from
// the odd one. Packed rows are
// WN / 2 + 8 dwords apart, so the four rows one write instruction touches
// start 16 banks apart. The rounding is the v_cvt_pk_bf16_f32 the fp32 path
// applies after staging, so both give the same bits; the packed staging
// takes half the LDS of the fp32 one (measured: the same speed), which the
// four-slot ring needs.
template <class Cfg, bool PACK, int SLAB>
struct EpiStage {
  static constexpr int ROW = PACK ? Cfg::WN / 2 + 8 : PersistLayout<Cfg>::EPI_LD;  // 4-byte words per staged row
  static constexpr int WORDS = Cfg::NW * SLAB * ROW;
  static_assert(SLAB == 8 || SLAB == 16, "slabs of one or two MFMA row groups");
  static_assert(ROW % 4 == 0, "16-byte aligned staging rows");
};

// 16-byte global store of 8 outputs (bf16 packed in a u32x4, or half of 8
// fp32). NT: non-temporal, so the output streams past L2 instead of evicting
// the operand rows that the stages in flight read through it.
template <bool NT>
__device__ __forceinline__ void st16(void* p, const u32x4& v) {
  if constexpr (NT) __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
  else *reinterpret_cast<u32x4*>(p) = v;
}
template <bool NT>
__device__ __forceinline__ void st_out8(bf16_t* p, const float* v) { st16<NT>(p, Out8<bf16_t>::pack(v)); }
template <bool NT>
__device__ __forceinline__ void st_out8(f16_t* p, const float* v) { st16<NT>(p, Out8<f16_t>::pack(v)); }
template <bool NT>
__device__ __forceinline__ void st_out8(float* p, const float* v) {
  st16<NT>(p, u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])});
  st16<NT>(p + 4, u32x4{__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]), __float_as_uint(v[7])});
}

// Which epilogues store non-temporally: the weight gradients (GM_RED), whose
// outputs (an expert's whole weight block per tile, 0.8 GB at the
// Qwen3-30B-A3B shape) would otherwise push the gathered rows the next tiles
// read out of L2 (measured on a walk of the gate_up weight-gradient loads:
// 64 GB/s per CU without stores, 29 with cached stores, 50 with
// non-temporal ones).
template <int GM>
constexpr bool nt_epilogue() { return GM == GM_RED; }

// Epilogue of a plain-store tile (EPI_STORE) whose columns all lie inside N,
// the common case. Each 8-row slab of a wave's 32-row block goes through the
// wave's LDS region in fp32, written straight from the MFMA layout (lane
// half h holds rows 4 h + r of the slab for its column: no lane exchange) and
// read back as 8 consecutive outputs per lane, which one 16-byte raw buffer
// store writes (two for fp32 outputs). The buffer covers the wave's valid
// rows only, so rows past the tile's last row are dropped by the hardware's
// bound check: no per-lane branch and no 64-bit address arithmetic. A wave's
// LDS operations run in order, so each slab's reads follow its writes, and the
// next slab's writes follow those reads, without a wait between them.
// Per lane per slab: 4 write2, 2 ds_read_b128, 4 conversions, 1-2 stores.
// 8-row fp32 staging of one MFMA row group in 64-float rows: lanes 0-31 write
// a row and lanes 32-63 the row four below, then 8 lanes read each row as two
// 16-byte halves. Columns are XORed with 4 on odd rows and with 32 on rows 4-7,
// so both the writes and the 16-lane groups of the reads hit distinct banks
// (a padded row of 68 floats left the writes 2-way conflicted).
__device__ __forceinline__ int stage_swz(int row) { return ((row & 1) << 2) | ((row & 4) << 3); }
__device__ __forceinline__ void stage_put(float* stage, int row, int col, float v) {
  stage[row * 64 + (col ^ stage_swz(row))] = v;
}
__device__ __forceinline__ void stage_get8(const float* stage, int row, int c, float (&v)[8]) {
  const int sw = stage_swz(row);
  const f32x4 a = *reinterpret_cast<const f32x4*>(stage + row * 64 + (c ^ sw));
  const f32x4 b = *reinterpret_cast<const f32x4*>(stage + row * 64 + ((c + 4) ^ sw));
  v[0] = a[0]; v[1] = a[1]; v[2] = a[2]; v[3] = a[3];
  v[4] = b[0]; v[5] = b[1]; v[6] = b[2]; v[7] = b[3];
}

template <class Cfg, typename Tout, int GM, bool NT>
__device__ __forceinline__ void store_tile_full_cols(const f32x16 (&acc)[Cfg::MI][Cfg::NI], float* stage,
                                                     const TileInfo& ti, const GemmParams& p, int wm, int wn,
                                                     int lane) {
  constexpr int MI = Cfg::MI, NI = Cfg::NI, WM = Cfg::WM, WN = Cfg::WN;
  constexpr int CPR = WN / 8;  // 8-output chunks per row
  static_assert(PersistLayout<Cfg>::EPI_LD >= 64, "the staged rows hold 64 floats");
  static_assert(8 * CPR == kWave, "one chunk per lane per 8-row slab (64-column wave tiles)");
  Tout* C = reinterpret_cast<Tout*>(p.C);
  if constexpr (GM == GM_RED) C += (int64_t)ti.group * p.strideC;
  // uniform by construction; said so, or the descriptor lives in VGPRs and
  // every buffer access becomes a readfirstlane loop
  const int row0 = __builtin_amdgcn_readfirstlane(ti.m0 + wm * WM);
  const int rows = __builtin_amdgcn_readfirstlane(min(max(ti.m_end - row0, 0), WM));
  Tout* base = C + (int64_t)row0 * p.ldc + ti.n0 + wn * WN;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      base, (short)0, rows > 0 ? (int)(((int64_t)(rows - 1) * p.ldc + WN) * (int64_t)sizeof(Tout)) : 0, 0x00020000);
  const int half = lane >> 5, col_l = lane & 31;
  const int r = lane / CPR, c = (lane % CPR) * 8;
  const int ld_bytes = (int)(p.ldc * sizeof(Tout));
  constexpr int AUX = NT ? 2 : 0;  // nt
#pragma unroll
  for (int i = 0; i < MI; ++i) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
      for (int j = 0; j < NI; ++j)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) stage_put(stage, 4 * half + rr, j * 32 + col_l, acc[i][j][4 * q + rr]);
      float v[8];
      stage_get8(stage, r, c, v);
      const int off = (i * 32 + 8 * q + r) * ld_bytes + c * (int)sizeof(Tout);
      if constexpr (sizeof(Tout) == 2) {
        __builtin_amdgcn_raw_buffer_store_b128(Out8<Tout>::pack(v), rs, off, 0, AUX);
      } else {
        const u32x4 lo = {__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])};
        const u32x4 hi = {__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]), __float_as_uint(v[7])};
        __builtin_amdgcn_raw_buffer_store_b128(lo, rs, off, 0, AUX);
        __builtin_amdgcn_raw_buffer_store_b128(hi, rs, off + 16, 0, AUX);
      }
    }
  }
}

// Epilogue of the SwiGLU backward (down dgrad, EPI_SWIGLU_BWD) for a tile
// whose columns all lie inside N. Each output needs its row's saved gate and
// up pre-activations and routing weight, which live in HBM. They are loaded
// PF slabs ahead through bounded raw buffer loads (rows past the tile's end
// read zero), the slabs go through the wave's fp32 LDS rows as in
// store_tile_full_cols, and the outputs and routing-weight partials leave
// through bounded buffer stores (rows past the end dropped). The descriptors
// must be wave-uniform (else each access becomes a readfirstlane loop) and
// the per-slab row offsets go in the SGPR offset (else the unrolled slabs
// hold one VGPR offset each and the 256x256 kernel spills). Measured on
// MI355X at config 2: 0.300 ms against 0.321 ms for the slab loop in
// store_slabs, with PF = 1, 2 and 3 alike. The arithmetic and its order are
// those of that slab loop.
template <class Cfg, bool NT>
__device__ __forceinline__ void store_tile_swiglu_bwd(const f32x16 (&acc)[Cfg::MI][Cfg::NI], float* stage,
                                                      const TileInfo& ti, const GemmParams& p, int wm, int wn,
                                                      int lane) {
  constexpr int MI = Cfg::MI, NI = Cfg::NI, WM = Cfg::WM, WN = Cfg::WN;
  constexpr int CPR = WN / 8;
  typedef typename Cfg::Tc T16;
  static_assert(WN == 64 && 8 * CPR == kWave, "one 8-column chunk per lane per 8-row slab, 64-column partials");
  constexpr int NSLAB = MI * 4, PF = 2;  // slabs per wave, slabs loaded ahead
  const int row0 = __builtin_amdgcn_readfirstlane(ti.m0 + wm * WM);  // uniform: scalar descriptors
  const int rows = __builtin_amdgcn_readfirstlane(min(max(ti.m_end - row0, 0), WM));
  const int col0 = __builtin_amdgcn_readfirstlane(ti.n0 + wn * WN);
  const int r = lane / CPR, c = (lane % CPR) * 8;
  const int ldaux = (int)p.ldaux, ldc = (int)p.ldc;
  const T16* GU = reinterpret_cast<const T16*>(p.aux) + (int64_t)row0 * p.ldaux;
  T16* DG = reinterpret_cast<T16*>(p.C) + (int64_t)row0 * p.ldc;
  const __amdgpu_buffer_rsrc_t rs_gu =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<T16*>(GU), (short)0, rows * ldaux * 2, 0x00020000);
  const __amdgpu_buffer_rsrc_t rs_dg = __builtin_amdgcn_make_buffer_rsrc(DG, (short)0, rows * ldc * 2, 0x00020000);
  const bool has_w = p.row_w != nullptr, has_part = p.part != nullptr;
  const __amdgpu_buffer_rsrc_t rs_w = __builtin_amdgcn_make_buffer_rsrc(
      has_w ? const_cast<float*>(p.row_w) + row0 : nullptr, (short)0, has_w ? rows * 4 : 0, 0x00020000);
  const __amdgpu_buffer_rsrc_t rs_part = __builtin_amdgcn_make_buffer_rsrc(
      has_part ? p.part + (int64_t)row0 * p.part_ld : nullptr, (short)0, has_part ? rows * p.part_ld * 4 : 0,
      0x00020000);
  constexpr int AUX = NT ? 2 : 0;
  const int half = lane >> 5, col_l = lane & 31;
  u32x4 pg[PF], pu[PF];
  float pw[PF];
  // slab s: rows 32 (s / 4) + 8 (s % 4) .. +7 of the wave; this lane's row in it is r
  // per-lane offsets are fixed; the slab's first row and the column block go
  // in the uniform (SGPR) offset, so the unrolled slabs share four VGPRs
  const int vo_gu = (r * ldaux + c) * 2, vo_dg = (r * ldc + c) * 2, vo_w = r * 4, vo_part = r * p.part_ld * 4;
  auto fetch = [&](auto sc) {
    constexpr int S = decltype(sc)::value;
    constexpr int R0 = (S / 4) * 32 + 8 * (S % 4);
    const int so = (R0 * ldaux + col0) * 2;
    pg[S % PF] = __builtin_amdgcn_raw_buffer_load_b128(rs_gu, vo_gu, so, 0);
    pu[S % PF] = __builtin_amdgcn_raw_buffer_load_b128(rs_gu, vo_gu, so + (int)p.inter * 2, 0);
    pw[S % PF] = has_w ? __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs_w, vo_w, R0 * 4, 0)) : 1.0f;
  };
  static_for<0, PF>([&](auto sc) { fetch(sc); });
  static_for<0, NSLAB>([&](auto sc) {
    constexpr int S = decltype(sc)::value, i = S / 4, q = S % 4;
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) stage_put(stage, 4 * half + rr, j * 32 + col_l, acc[i][j][4 * q + rr]);
    float v[8], g[8], u[8], dg[8], du[8];
    stage_get8(stage, r, c, v);
    unpack8<T16>(pg[S % PF], g);
    unpack8<T16>(pu[S % PF], u);
    const float ws = pw[S % PF];
    if constexpr (S + PF < NSLAB) fetch(std::integral_constant<int, S + PF>());
    float pd = 0.0f;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const float sg = fast_sigmoid(g[t]);
      const float silu = g[t] * sg;
      pd += v[t] * (silu * u[t]);
      const float dm = v[t] * ws;
      dg[t] = dm * u[t] * (sg + silu * (1.0f - sg));
      du[t] = dm * silu;
    }
    constexpr int R0 = i * 32 + 8 * q;
    const int so = (R0 * ldc + col0) * 2;
    __builtin_amdgcn_raw_buffer_store_b128(Out8<T16>::pack(dg), rs_dg, vo_dg, so, AUX);
    __builtin_amdgcn_raw_buffer_store_b128(Out8<T16>::pack(du), rs_dg, vo_dg, so + (int)p.inter * 2, AUX);
    if (has_part) {  // the CPR = 8 lanes of a row are consecutive: sum them in a fixed order
      pd += __shfl_xor(pd, 1);
      pd += __shfl_xor(pd, 2);
      pd += __shfl_xor(pd, 4);
      if ((lane % CPR) == 0)
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(pd), rs_part, vo_part,
                                              (R0 * p.part_ld + col0 / 64) * 4, 0);
    }
  });
}

template <class Cfg, typename Tout, int GM, int EPI, bool PACK, int SLAB>
__device__ __forceinline__ void store_slabs(const f32x16 (&acc)[Cfg::MI][Cfg::NI], float* stage,
                                            const TileInfo& ti, const GemmParams& p, int wm, int wn, int lane) {
  constexpr int MI = Cfg::MI, NI = Cfg::NI, WN = Cfg::WN;
  constexpr int LD = PersistLayout<Cfg>::EPI_LD;
  constexpr int LDW = EpiStage<Cfg, PACK, SLAB>::ROW;  // packed: words per staged row
  constexpr int QPS = SLAB / 8, NSL = 32 / SLAB;         // row groups q per slab, slabs per 32-row block
  static_assert(!PACK || (sizeof(Tout) == 2 && EPI != EPI_SWIGLU_BWD), "packed staging of bf16 outputs");
  static_assert(EPI == EPI_STORE || sizeof(Tout) == 2, "fused epilogues write bf16");
  constexpr bool NT = nt_epilogue<GM>();
  if constexpr (EPI == EPI_SWIGLU_BWD && GM == GM_ROWS && Cfg::WN == 64) {
    if (ti.n0 + Cfg::BN <= p.N && (int64_t)Cfg::WM * p.ldaux * 2 < ((int64_t)1 << 31) &&
        (int64_t)Cfg::WM * p.ldc * 2 < ((int64_t)1 << 31)) {
      store_tile_swiglu_bwd<Cfg, NT>(acc, stage, ti, p, wm, wn, lane);
      return;
    }
  }
  if constexpr (EPI == EPI_STORE && Cfg::WN == 64) {
    if (ti.n0 + Cfg::BN <= p.N && (int64_t)Cfg::WM * p.ldc * (int64_t)sizeof(Tout) < ((int64_t)1 << 31)) {
      store_tile_full_cols<Cfg, Tout, GM, NT>(acc, stage, ti, p, wm, wn, lane);
      return;
    }
  }
  Tout* C = reinterpret_cast<Tout*>(p.C);
  if constexpr (GM == GM_RED) C += (int64_t)ti.group * p.strideC;
  const int half = lane >> 5, col_l = lane & 31;
  uint32_t* st32 = reinterpret_cast<uint32_t*>(stage);
  // SwiGLU forward: the routing weights of every row this lane writes, loaded
  // before the first slab rather than one global load (and its latency) per slab
  constexpr int SW_CPR = WN / 2 / 8, SW_NE = (SLAB * SW_CPR + 63) / 64;
  float wsp[MI][NSL][SW_NE];
  if constexpr (EPI == EPI_SWIGLU) {
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int hs = 0; hs < NSL; ++hs)
#pragma unroll
        for (int ei = 0; ei < SW_NE; ++ei) {
          const int e = lane + 64 * ei;
          const int row = ti.m0 + wm * Cfg::WM + i * 32 + SLAB * hs + e / SW_CPR;
          wsp[i][hs][ei] = (p.row_w != nullptr && e < SLAB * SW_CPR && row < ti.m_end) ? p.row_w[row] : 1.0f;
        }
  }
#pragma unroll
  for (int i = 0; i < MI; ++i) {
#pragma unroll
    for (int hs = 0; hs < NSL; ++hs) {
      if constexpr (PACK) {
        const bool odd = lane & 1;
#pragma unroll
        for (int qq = 0; qq < QPS; ++qq)
#pragma unroll
          for (int j = 0; j < NI; ++j) {
            const int q0 = 4 * (QPS * hs + qq);
            const float v0 = acc[i][j][q0], v1 = acc[i][j][q0 + 1], v2 = acc[i][j][q0 + 2], v3 = acc[i][j][q0 + 3];
            const float r0 = swap_lane_pair(odd ? v0 : v2), r1 = swap_lane_pair(odd ? v1 : v3);
            const uint32_t p0 = odd ? Fmt16<Tout>::pack2(r0, v2) : Fmt16<Tout>::pack2(v0, r0);
            const uint32_t p1 = odd ? Fmt16<Tout>::pack2(r1, v3) : Fmt16<Tout>::pack2(v1, r1);
            const int row = 8 * qq + 4 * half + (odd ? 2 : 0);
            st32[row * LDW + j * 16 + (col_l >> 1)] = p0;
            st32[(row + 1) * LDW + j * 16 + (col_l >> 1)] = p1;
          }
      } else {
#pragma unroll
        for (int qq = 0; qq < QPS; ++qq)
#pragma unroll
          for (int j = 0; j < NI; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              stage[(8 * qq + 4 * half + r) * LD + j * 32 + col_l] = acc[i][j][4 * (QPS * hs + qq) + r];
      }
      __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0): slab written
      asm volatile("" ::: "memory");
      const int row_base = ti.m0 + wm * Cfg::WM + i * 32 + SLAB * hs;
      if constexpr (EPI == EPI_SWIGLU) {
        constexpr int H2 = WN / 2, CPR = H2 / 8;
        Tout* MID = reinterpret_cast<Tout*>(p.C2);
#pragma unroll
        for (int ei = 0; ei < SW_NE; ++ei) {
          const int e = lane + 64 * ei;
          if (e >= SLAB * CPR) break;
          const int r = e / CPR, c = (e % CPR) * 8;
          const int row = row_base + r, col = ti.n0 + wn * H2 + c;
          if (row < ti.m_end && col < p.inter) {
            static_assert(PACK, "the SwiGLU forward stages bf16");
            float g[8], u[8], m[8];
            const u32x4 gw = *reinterpret_cast<const u32x4*>(st32 + r * LDW + c / 2);
            const u32x4 uw = *reinterpret_cast<const u32x4*>(st32 + r * LDW + H2 / 2 + c / 2);
            st16<NT>(C + (int64_t)row * p.ldc + col, gw);
            st16<NT>(C + (int64_t)row * p.ldc + p.inter + col, uw);
            unpack8<Tout>(gw, g);  // the activation uses the stored (rounded) pre-activations
            unpack8<Tout>(uw, u);
            const float ws = wsp[i][hs][ei];  // the routing weight
#pragma unroll
            for (int t = 0; t < 8; ++t) m[t] = g[t] * fast_sigmoid(g[t]) * u[t] * ws;
            st_out8<NT>(MID + (int64_t)row * p.ldc2 + col, m);
          }
        }
      } else {
        constexpr int CPR = WN / 8;
        static_assert(EPI != EPI_SWIGLU_BWD || WN == 64, "routing-weight partials are per 64-column block");
        const int col_base = ti.n0 + wn * WN;
#pragma unroll
        for (int e = lane; e < SLAB * CPR; e += 64) {
          const int r = e / CPR, c = (e % CPR) * 8;
          const int row = row_base + r, col = col_base + c;
          float pd = 0.0f;  // this lane's share of <acc, silu(g) u> (EPI_SWIGLU_BWD with row_w)
          if (row < ti.m_end && col < p.N) {
            float v[8];
            if constexpr (PACK) {
              const u32x4 w = *reinterpret_cast<const u32x4*>(st32 + r * LDW + c / 2);
              if (col + 8 <= p.N) {
                st16<NT>(C + (int64_t)row * p.ldc + col, w);
              } else {
                unpack8<Tout>(w, v);
                for (int t = 0; col + t < p.N; ++t) store_scalar<Tout>(C + (int64_t)row * p.ldc + col + t, v[t]);
              }
            } else if constexpr (EPI == EPI_SWIGLU_BWD) {
              // v = d(mid), or with row_w d(w * mid): then d(mid) = w v and d(w) += v . mid
              Vec8<float>::load(stage + r * LD + c, v);
              const Tout* GU = reinterpret_cast<const Tout*>(p.aux) + (int64_t)row * p.ldaux;
              float g[8], u[8], dg[8], du[8];
              Vec8<Tout>::load(GU + col, g);
              Vec8<Tout>::load(GU + p.inter + col, u);
              const float ws = p.row_w != nullptr ? p.row_w[row] : 1.0f;
#pragma unroll
              for (int t = 0; t < 8; ++t) {
                const float sg = fast_sigmoid(g[t]);
                const float silu = g[t] * sg;
                pd += v[t] * (silu * u[t]);
                const float dm = v[t] * ws;
                dg[t] = dm * u[t] * (sg + silu * (1.0f - sg));
                du[t] = dm * silu;
              }
              st_out8<NT>(C + (int64_t)row * p.ldc + col, dg);
              st_out8<NT>(C + (int64_t)row * p.ldc + p.inter + col, du);
            } else {
              Vec8<float>::load(stage + r * LD + c, v);
              if (col + 8 <= p.N) {
                st_out8<NT>(C + (int64_t)row * p.ldc + col, v);
              } else {
                for (int t = 0; col + t < p.N; ++t) store_scalar<Tout>(C + (int64_t)row * p.ldc + col + t, v[t]);
              }
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
      // (the next slab's writes follow these reads in the wave's LDS order)
    }
  }
}

// Of D DMAs placed after MFMA slots (i * TOTM) / D, those before slot PRE.
template <int D, int TOTM, int PRE>
constexpr int dmas_before() {
  int c = 0;
  for (int i = 0; i < D; ++i) c += (i * TOTM) / D < PRE ? 1 : 0;
  return c;
}

// Slot of DMA DI among the TOTM MFMA slots of a stage: the D DMAs at
// (DI * TOTM) / D.
template <int D, int TOTM>
constexpr int dma_slot(int di) {
  return (di * TOTM) / D;
}

// Tile `local` of an expert (a row group) with r m-tiles (the last may be
// partial) over ntn n-tiles. The tiles go n-tile major, an n-tile's m-tiles
// side by side so that they share its weight block in L2. An expert with more
// m-tiles than n-tiles (its rows then outweigh its weights) goes in
// super-blocks of mb m-tiles, mb x ntn tiles that run together on one XCD
// (mb = the XCD's blocks / ntn): its rows are then staged from past L2 once
// rather than once per n-tile, its weight blocks once per super-block.
__device__ __forceinline__ void rows_tile(int local, int r, int ntn, int mb, int& tn, int& mt) {
  const int k = (r > ntn && r > mb) ? (r - 1) / mb : 0;  // full super-blocks before the last
  const int first = k * mb * ntn;
  if (local < first) {
    const int sb = local / (mb * ntn), q = local % (mb * ntn);
    tn = q / mb;
    mt = sb * mb + q % mb;
    return;
  }
  local -= first;
  const int h = r - k * mb, m0 = k * mb;  // the last super-block's m-tiles
  tn = local / h;
  mt = m0 + local % h;
}

// GM_RED cost model: a tile of group g runs max(ceil(rows_g / BK), NS - 1)
// k-stages plus an epilogue worth about kRedEpiStages stages (measured: a
// 256x256 bf16 tile drains in ~3 stage times). s_cost[g] = cost of one tile of
// each group before g (inclusive scan to groups + 1 entries, computed by wave
// 0), *s_cmax = the largest cost of one tile; every thread gets s_cost[groups].
constexpr int kRedEpiStages = 3;
template <int BK, int NS>
__device__ __forceinline__ int red_cost_scan(const int32_t* offs, int groups, int* s_cost, int* s_cmax) {
  const int tid = threadIdx.x, lane = tid & 63;
  if (tid < 64) {
    int carry = 0, cmax = 0;
    for (int base = 0; base < groups; base += 64) {
      const int g = base + lane;
      int c = 0;
      if (g < groups) {
        const int rows = offs[g] - (g == 0 ? 0 : offs[g - 1]);
        c = max((rows + BK - 1) / BK, NS - 1) + kRedEpiStages;
      }
      cmax = max(cmax, c);
      const int inc = wave_incl_scan(c, lane) + carry;
      if (g < groups) s_cost[g + 1] = inc;
      carry = __shfl(inc, 63, kWave);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) cmax = max(cmax, __shfl_xor(cmax, o, kWave));
    if (lane == 0) {
      s_cost[0] = 0;
      *s_cmax = cmax;
    }
  }
  __syncthreads();
  return s_cost[groups];
}

// First tile (in list order: group-major, tpg tiles per group) whose
// cumulative cost reaches `target` (0 <= target <= total cost).
__device__ __forceinline__ int red_cost_tile(const int* s_cost, int groups, int tpg, int64_t target) {
  int lo = 0, hi = groups - 1;  // the last group g with s_cost[g] * tpg <= target
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if ((int64_t)s_cost[mid] * tpg <= target) lo = mid;
    else hi = mid - 1;
  }
  const int64_t c = s_cost[lo + 1] - s_cost[lo];  // cost of one tile of group lo (> 0)
  const int64_t k = (target - (int64_t)s_cost[lo] * tpg + c - 1) / c;
  return lo * tpg + (int)min<int64_t>(k, tpg);
}

// Dealing of GM_RED tiles under skewed routing. The tiles are taken in order
// of descending cost (s_order: groups sorted by the cost of one tile, each
// group's tpg tiles consecutive) and dealt in rounds: round 0 gives tile p to
// the block at position p; in each later round only the blocks whose load is
// still below the mean share take part (all of them when none is), in
// ascending position order on even rounds and descending order on odd ones,
// each taking the next tile. Against the plain snake (every block in every
// round) this keeps a block that drew a heavy tile from also drawing its share
// of the small ones: on config 4's routing a simulation of the two deals puts
// the heaviest block at 1.05x (down wgrad) and 1.01x (gate_up wgrad) the mean
// share, against 1.37x and 1.06x. Every block runs the same integer simulation
// (thread p simulates position p; a round is one ballot and one barrier) and
// keeps the list indices of its own tiles. The costs are staged in `scratch`
// (the ring's LDS, unused until the first DMA); s_cost (the inclusive scan of
// red_cost_scan) is overwritten by this block's list, ended by -1 when it is
// shorter than kMaxDealt. Returns whether the deal fits (at most kMaxDealt
// tiles for every block, at most kMaxRounds rounds, no more blocks than
// threads; the same outcome in every block): otherwise the caller falls back
// to the snake, in every block alike.
constexpr int kMaxDealt = 1024;
constexpr int kMaxRounds = 4096;
template <int NT>
__device__ __forceinline__ bool deal_below_mean(const unsigned short* s_order, int* s_cost, int groups, int tpg,
                                            int total, int64_t c_all, int nb, int spos, char* scratch,
                                            int* s_result) {
  constexpr int NW = NT / 64;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (nb > NT) return false;  // uniform: the grid is the same for every block
  int* c_sorted = reinterpret_cast<int*>(scratch);                 // [groups]
  uint64_t* s_mask = reinterpret_cast<uint64_t*>(scratch + 4096);  // [2][NW]
  for (int r = tid; r < groups; r += NT) {
    const int g = s_order[r];
    c_sorted[r] = s_cost[g + 1] - s_cost[g];
  }
  if (tid == 0) s_result[1] = 0;
  __syncthreads();  // the costs are staged; s_cost is free for the list
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int64_t load = 0;
  int cnt = 0, j0 = 0, round = 0;
  while (j0 < total && round < kMaxRounds) {
    bool act = tid < nb && (round == 0 || load * nb < c_all);
    const uint64_t m = __ballot(act);
    if (lane == 0) s_mask[(round & 1) * NW + wave] = m;
    __syncthreads();
    int a = 0, below = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const int c = __popcll(s_mask[(round & 1) * NW + w]);
      a += c;
      below += w < wave ? c : 0;
    }
    below += __popcll(m & lt_mask);
    if (a == 0) {  // every block has reached the mean: all take part
      act = tid < nb;
      a = nb;
      below = tid;
    }
    if (act) {
      const int j = j0 + ((round & 1) ? a - 1 - below : below);
      if (j < total) {
        load += c_sorted[j / tpg];
        if (tid == spos && cnt < kMaxDealt) s_cost[cnt] = j;
        ++cnt;
      }
    }
    j0 += a;
    ++round;
  }
  // end this block's list; flag any block whose list does not fit (uniform outcome)
  if (tid == spos && cnt < kMaxDealt) s_cost[cnt] = -1;
  if (cnt > kMaxDealt) atomicOr(&s_result[1], 1);
  __syncthreads();
  return s_result[1] == 0 && j0 >= total;
}

// The block's tiles form one continuous stream of k-stages: stage g lives in
// ring slot g % NS, and the DMAs issued during stage g fetch stream stage
// g + NS - 1, which in a tile's last NS - 1 stages is one of the next tile's
// first stages. The pipeline therefore stays full across tile boundaries (the
// next tile's first stages land while this tile's last stages and epilogue
// run) and every stage issues the same DMAs (no branches in the k-loop). A
// tile's first NS - 1 stages have fully landed before its stage 0 (the
// prologue, and each epilogue, waits for them), so stage 0 goes straight to
// its barrier and every later stage waits for the same vmcnt.
// The DMA instructions per stage of the operand whose k-rows are gathered
// (one token per lane per instruction), and whether its tile shape has the
// two k-rows per instruction (lanes 0-31, 32-63) the token reads assume.
template <bool KG, class LdA, class LdB, bool ON_B>
struct KGatherInfo {
  static constexpr int INSTR = 1;
  static constexpr bool ok = true;
};
template <class LdA, class LdB, bool ON_B>
struct KGatherInfo<true, LdA, LdB, ON_B> {
  typedef typename std::conditional<ON_B, LdB, LdA>::type L;
  static constexpr int INSTR = L::INSTR;
  static constexpr bool ok = L::KPI == 2 && L::CPR == 32;
};

// GATH: which operand's rows are gathered through an index table (see
// GemmParams): 0 none, GA_ROWS (GM_ROWS: A's rows; indices once per tile),
// GA_KROWS / GB_KROWS (GM_RED: A's / B's k-rows; the indices of the DMAs of
// stage g + 1 are read through the scalar cache during stage g, and once per
// tile for its first stage).
enum GatherKind { G_NONE = 0, GA_ROWS = 1, GA_KROWS = 2, GB_KROWS = 3 };

template <class Cfg, typename Tout, bool A_KC, bool B_KC, int GM, int EPI, int GATH>
__global__ __launch_bounds__(Cfg::NT, 1) void grouped_gemm_persist_kernel(GemmParams p) {
  constexpr int BM = Cfg::BM, BN = Cfg::BN, BK = Cfg::BK, NW = Cfg::NW, NS = Cfg::NS, D = Cfg::D;
  constexpr int MI = Cfg::MI, NI = Cfg::NI;
  constexpr int SLOT = Cfg::STAGE_BYTES;  // ring slot bytes
  // bf16 outputs stage packed (the SwiGLU backward reads its fp32 accumulators back)
  constexpr bool PACK = sizeof(Tout) == 2 && (EPI == EPI_SWIGLU || EPI == EPI_STORE);
  static_assert(PACK || EPI != EPI_SWIGLU, "the SwiGLU forward stages packed bf16");
  // (a plain store may round to the other 16-bit format: the router's input
  // gradient from bf16 pieces of an fp16 weight)
  static_assert(sizeof(Tout) == 4 || std::is_same<Tout, typename Cfg::Tc>::value || EPI == EPI_STORE,
                "16-bit outputs of the fused epilogues are in the operands' format");
  static_assert(GM == GM_ROWS || GM == GM_RED, "persistent kernel serves the expert GEMMs");
  static_assert(!(GM == GM_RED && (A_KC || B_KC)), "GM_RED expects [k][m] and [k][n] operands");
  static_assert(EPI != EPI_SWIGLU || (B_KC && GM == GM_ROWS && Cfg::WN % 32 == 0), "SwiGLU epilogue layout");
  static_assert(GATH == G_NONE || (GATH == GA_ROWS && GM == GM_ROWS && A_KC) ||
                    ((GATH == GA_KROWS || GATH == GB_KROWS) && GM == GM_RED),
                "gathers: A's rows in GM_ROWS, A's or B's k-rows in GM_RED");

  __shared__ __attribute__((aligned(1024))) char smem[NS * SLOT];
  // fp32 staging beside a four-slot ring takes 8-row slabs (16 KiB less LDS)
  constexpr int SLAB = (NS >= 4 && !PACK) ? 8 : 16;
  __shared__ __attribute__((aligned(16))) float s_epi[EpiStage<Cfg, PACK, SLAB>::WORDS];
  __shared__ int s_scan[1025];
  __shared__ int s_offs[1024];
  __shared__ unsigned short s_order[1024];  // GM_RED under skew: groups by tile cost, descending
  __shared__ int s_cmax;
  __shared__ int s_deal[2];                  // GM_RED under skew: the deal's overflow flag

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / Cfg::WAVES_N, wn = wave % Cfg::WAVES_N;
  const int groups = p.groups;

  // ---- tile list: GM_ROWS m-tiles follow the per-group row counts
  // offs null: one group of all M rows (a plain GEMM on the same engine)
  for (int g = tid; g < groups; g += Cfg::NT) s_offs[g] = p.offs != nullptr ? p.offs[g] : p.M;
  __syncthreads();
  const int ntiles_n = (EPI == EPI_SWIGLU) ? (p.inter + BN / 2 - 1) / (BN / 2) : (p.N + BN - 1) / BN;
  const int mt_red = (p.M + BM - 1) / BM;  // GM_RED: m-tiles per group
  int total;
  if constexpr (GM == GM_ROWS) total = rows_scan<BM>(s_offs, groups, s_scan) * ntiles_n;
  else total = groups * mt_red * ntiles_n;
  // XCD x (blocks with blockIdx % 8 == x) takes a contiguous share of the tiles
  // and its blocks walk it in a stride of their count. GM_ROWS tiles all run
  // the full reduction, so the shares hold equal tile counts; a GM_RED tile
  // runs its group's reduction range, so there the shares hold equal cost.
  // Under skewed routing (GM_RED, one tile costing more than half a block's
  // mean share) the shares cannot balance: a heavy group's tiles crowd one
  // XCD's blocks. Then the tiles are taken in order of descending cost and
  // dealt in rounds to the blocks still below the mean share
  // (deal_below_mean), positions XCD-major so that a group's tiles still run
  // side by side on one XCD; when that deal does not fit its bounds, in a
  // snake (round k gives tile k*NB + p to the block at position p, or
  // k*NB + NB-1-p for odd k).
  const int xcd = blockIdx.x & 7;
  const int nb = ((int)gridDim.x - xcd + 7) >> 3;  // blocks on this XCD
  const int bi = blockIdx.x >> 3;                  // this block's position on its XCD
  // m-tiles per super-block of a row-heavy expert: the same for every block
  // (the tile list must be), from the grid's blocks per XCD
  const int mb = max(1, ((int)gridDim.x >> 3) / ntiles_n);
  int cnt = 0, start = 0, tpg = 1, spos = 0;
  bool skew = false;
  if (total == 0) {
    return;
  } else if constexpr (GM == GM_RED) {
    tpg = mt_red * ntiles_n;  // tiles per group
    const int64_t c_all = red_cost_scan<BK, NS>(s_offs, groups, s_scan, &s_cmax) * (int64_t)tpg;
    skew = (int64_t)s_cmax * 2 * gridDim.x > c_all;
    if (skew) {
      for (int g = tid; g < groups; g += Cfg::NT) {
        const int c = s_scan[g + 1] - s_scan[g];
        int r = 0;
        for (int h = 0; h < groups; ++h) {
          const int ch = s_scan[h + 1] - s_scan[h];
          r += (ch > c || (ch == c && h < g)) ? 1 : 0;
        }
        s_order[r] = g;
      }
      __syncthreads();
      for (int x = 0; x < xcd; ++x) spos += ((int)gridDim.x - x + 7) >> 3;
      spos += bi;
      // spos < 0 from here on: this block's tiles are the list in s_scan
      if (deal_below_mean<Cfg::NT>(s_order, s_scan, groups, tpg, total, c_all, (int)gridDim.x, spos, smem, s_deal))
        spos = -1;
    } else {
      const int b0 = red_cost_tile(s_scan, groups, tpg, c_all * xcd / 8);
      const int b1 = xcd == 7 ? total : red_cost_tile(s_scan, groups, tpg, c_all * (xcd + 1) / 8);
      start = b0;
      cnt = b1 - b0;
    }
  } else {
    const int per = total >> 3, rem = total & 7;
    cnt = per + (xcd < rem ? 1 : 0);
    start = xcd * per + (xcd < rem ? xcd : rem);
  }
  // The k-th tile of this block (k = 0, 1, ...) as a list index, or -1 past its last.
  auto tile_at = [&](int k) -> int {
    if (skew) {
      if (spos < 0) {
        const int j = k < kMaxDealt ? s_scan[k] : -1;  // this block's k-th tile in the cost order
        return j < 0 ? -1 : s_order[j / tpg] * tpg + j % tpg;
      }
      const int NB = (int)gridDim.x;
      const int j = k * NB + ((k & 1) ? NB - 1 - spos : spos);
      return j < total ? s_order[j / tpg] * tpg + j % tpg : -1;
    }
    const int b = bi + k * nb;
    return b < cnt ? start + b : -1;
  };
  if (tile_at(0) < 0) return;

  const uint32_t lds0 = lds_addr(smem);
  float* stage = s_epi + wave * SLAB * EpiStage<Cfg, PACK, SLAB>::ROW;
  const bf16_t* A0 = reinterpret_cast<const bf16_t*>(p.A);
  const bf16_t* B0 = reinterpret_cast<const bf16_t*>(p.B);
  typedef typename std::conditional<A_KC, KcDma<BM, NW, BK>, TDma<BM, NW, BK>>::type LdA;
  typedef typename std::conditional<B_KC, KcDma<BN, NW, BK>, TDma<BN, NW, BK>>::type LdB;
  constexpr int KS = BK / 16;
  static_assert(KS % 2 == 0, "fragment double buffer assumes an even number of substeps");
  constexpr bool kInterleaveFrags = true;
  // A tile's stages run as two loops (DMAs into this tile, then into the
  // next) in the input-gradient GEMMs ([k][n] weights): gate_up dgrad -2.5 %
  // measured; the forward GEMMs measured 3.5 % slower that way and the weight
  // gradients no faster, so they select the DMA source stage by stage.
  constexpr bool kSplitStages = GM == GM_ROWS && !B_KC;
  // DMAs of stage g + NS - 1 ride on the MFMAs of the first SPREAD substeps
  // of stage g. Spread over all KS substeps, the last of which runs after the
  // stage's barrier: the gate_up forward (measured: -3 % on three slots, and
  // keeping them before the barrier costs 7 % on four) and, on the four-slot
  // ring, the other row-grouped GEMMs (down dgrad -1.6 %, gate_up dgrad
  // -1.4 % on one box; on three slots they lost 5-9 %). The weight gradients
  // keep them before the barrier (spread: +1 % on four slots, +3 % on three).
  // At least three slots: a tile's stage 0 does not wait, because its first
  // NS - 1 >= 2 stages were fetched before it started; with two slots stage 1
  // would be issued during stage 0 and read before it had landed.
  static_assert(NS >= 3, "the persistent ring needs three slots or more");
  constexpr int SPREAD = ((EPI == EPI_SWIGLU && KS == 2) || (NS == 4 && GM == GM_ROWS)) ? KS : KS - 1;
  constexpr int TOTM = SPREAD * MI * NI;  // MFMA slots the DMAs are spread over (several may share one)
  static_assert(SPREAD >= 1, "the DMAs of a stage need MFMA slots");
  // The stage's DMAs issued before its barrier. At that barrier stream stage
  // g + 1 must have landed; issued after its last DMA are the full stages
  // g + 2 .. g + NS - 2 and these D_PRE of stage g + NS - 1, so that many may
  // stay outstanding.
  constexpr int D_PRE = dmas_before<D, TOTM, (KS - 1) * MI * NI>();
  constexpr int WAIT_N = (NS - 3) * D + D_PRE;
  static_assert(WAIT_N >= 0 && D_PRE >= 1, "stage accounting");
  const int a_row0 = wm * Cfg::WM, b_row0 = wn * Cfg::WN;

  // k-row gathers: the gathered [k][r] operand's DMA instructions per stage,
  // each covering KPI = 2 k-rows (lanes 0-31 the first, 32-63 the second).
  constexpr bool KGATH = GATH == GA_KROWS || GATH == GB_KROWS;
  typedef KGatherInfo<KGATH, LdA, LdB, GATH == GB_KROWS> KGI;
  constexpr int GI = KGI::INSTR;
  static_assert(KGI::ok, "k-row gather expects 256-column [k][r] tiles");
  const int32_t* gidx = GATH == GB_KROWS ? p.b_index : p.a_index;

  // What the DMAs of one tile need. nk is padded to at least NS - 1 stages
  // (the extra stages read zeros), so the DMAs of a tile's last NS - 1 stages
  // always fetch the following tile's first stages.
  struct LoadTile {
    TileInfo ti;
    BufRsrc rsA, rsB;
    LdA la;
    LdB lb;
    int nk, kd0, kd_hi;
    int klo;  // first reduction index of the tile (wave-uniform; k-row gathers)
  };
  // Tile t of the list (t < 0: past the block's last tile; its descriptors
  // are empty, so every DMA reads zeros).
  auto setup = [&](int t, LoadTile& T) {
    T.ti.group = 0; T.ti.m0 = 0; T.ti.m_end = 0; T.ti.n0 = 0; T.ti.k_lo = 0; T.ti.k_hi = 0;
    T.nk = NS - 1;
    T.kd0 = 0;
    T.kd_hi = 0;
    T.klo = 0;
    const bf16_t* a_base = A0;
    const bf16_t* b_base = B0;
    uint64_t a_bytes = 0, b_bytes = 0;
    if (t >= 0) {
      int tn = t % ntiles_n, slot = t / ntiles_n;
      if constexpr (GM == GM_ROWS) {
        const int g = rows_group(s_scan, groups, slot);
        const int lo = g == 0 ? 0 : s_offs[g - 1];
        int mt;
        rows_tile(t - s_scan[g] * ntiles_n, s_scan[g + 1] - s_scan[g], ntiles_n, mb, tn, mt);
        T.ti.group = g; T.ti.m0 = lo + mt * BM; T.ti.m_end = s_offs[g];
        T.ti.k_lo = 0; T.ti.k_hi = p.K;
        b_base = B0 + (int64_t)g * p.strideB;
        b_bytes = p.b_bytes;
      } else {
        const int g = slot / mt_red;
        T.ti.group = g; T.ti.m0 = (slot % mt_red) * BM; T.ti.m_end = p.M;
        T.ti.k_lo = g == 0 ? 0 : s_offs[g - 1];
        T.ti.k_hi = s_offs[g];
      }
      T.ti.n0 = (EPI == EPI_SWIGLU) ? tn * (BN / 2) : tn * BN;
      if constexpr (A_KC) {
        if constexpr (GATH == GA_ROWS) {
          a_bytes = p.a_bytes;  // the whole gathered storage
        } else {
          a_base = A0 + (int64_t)T.ti.m0 * p.lda;
          a_bytes = (uint64_t)(T.ti.m_end - T.ti.m0) * p.lda * 2;
        }
      } else if constexpr (GATH == GA_KROWS) {
        a_bytes = p.a_bytes;
      } else {
        a_base = A0 + (int64_t)T.ti.k_lo * p.lda;
        a_bytes = (uint64_t)(T.ti.k_hi - T.ti.k_lo) * p.lda * 2;
      }
      if constexpr (GM == GM_RED) {
        if constexpr (GATH == GB_KROWS) {
          b_bytes = p.b_bytes;
        } else {
          b_base = B0 + (int64_t)T.ti.k_lo * p.ldb;
          b_bytes = (uint64_t)(T.ti.k_hi - T.ti.k_lo) * p.ldb * 2;
        }
      }
      const int klen = T.ti.k_hi - T.ti.k_lo;
      T.nk = max((klen + BK - 1) / BK, NS - 1);
      T.kd0 = (GM == GM_RED) ? 0 : T.ti.k_lo;
      T.kd_hi = T.ti.k_hi - ((GM == GM_RED) ? T.ti.k_lo : 0);
      T.klo = __builtin_amdgcn_readfirstlane(T.ti.k_lo);
    }
    T.rsA = make_rsrc(a_base, a_bytes);
    T.rsB = make_rsrc(b_base, b_bytes);
    // B rows (columns) of the tile: with SwiGLU, wave column block w holds
    // WN/2 gate columns then the matching up columns
    const int n0 = T.ti.n0, N = p.N, I = p.inter;
    auto b_row_of = [&](int c) {
      if constexpr (EPI == EPI_SWIGLU) {
        const int w = c / Cfg::WN, cc = c % Cfg::WN, h = Cfg::WN / 2;
        const int gcol = n0 + w * h + (cc % h);
        if (gcol >= I) return -1;
        return cc < h ? gcol : I + gcol;
      } else {
        return n0 + c < N ? n0 + c : -1;
      }
    };
    if constexpr (A_KC) {
      const int rows = T.ti.m_end - T.ti.m0;
      if constexpr (GATH == GA_ROWS)
        T.la.init_gather(p.a_index, p.n_index, __builtin_amdgcn_readfirstlane(T.ti.m0), rows, p.lda, wave, lane);
      else
        T.la.init([&](int r) { return r < rows ? r : -1; }, p.lda, wave, lane);
    } else {
      T.la.init(T.ti.m0, T.ti.m_end, wave, lane);
    }
    if constexpr (B_KC) T.lb.init(b_row_of, p.ldb, wave, lane);
    else T.lb.init(T.ti.n0, p.N, wave, lane);
  };

  // Tokens of the gathered k-rows of tile-local stage ls of T: instruction i
  // covers two k-rows, tok[i][0] for lanes 0-31 and tok[i][1] for 32-63. They
  // are read through the scalar cache and stay wave-uniform (the per-lane
  // pick happens at the DMA), so a read issued a stage ahead is not waited
  // for until that stage. Index arithmetic in 32 unsigned bits: the table
  // holds at most 2^31 - 1 entries and q stays a few stages past its end.
  auto tokens = [&](const LoadTile& T, int ls, int (&tok)[GI][2]) {
    if constexpr (KGATH) {
      typedef const __attribute__((address_space(4))) int32_t cint;
      cint* ci = (cint*)gidx;
      const uint32_t last = (uint32_t)(p.n_index - 1);
      const uint32_t q0 = (uint32_t)T.klo + (uint32_t)(ls * BK) + (uint32_t)(wave * 2);
#pragma unroll
      for (int i = 0; i < GI; ++i) {
        const uint32_t q = q0 + (uint32_t)(i * NW * 2);
        tok[i][0] = ci[min(q, last)];
        tok[i][1] = ci[min(q + 1u, last)];
      }
    }
  };
  const uint32_t lda2 = (uint32_t)(p.lda * 2), ldb2 = (uint32_t)(p.ldb * 2);  // gathered rows' bytes

  int gs = 0;  // stream stage of the current tile's stage 0
  auto slot_of = [&](int g) { return ((uint32_t)g % NS) * SLOT; };  // g >= 0
  // DMA J of stage ls of tile T, into the ring slot of stream stage g; tok:
  // the gathered k-rows' tokens of that stage.
  auto dma_one = [&](const LoadTile& T, int ls, int g, const int (&tok)[GI][2], auto jc) {
    constexpr int J = decltype(jc)::value;
    const uint32_t st = lds0 + slot_of(g);
    const int k0 = T.kd0 + ls * BK;
    if constexpr (J < Cfg::A_INSTR) {
      if constexpr (A_KC) T.la.template issue1<J>(T.rsA, st, k0, T.kd_hi, k0 + BK > T.kd_hi, wave);
      else if constexpr (GATH == GA_KROWS)
        T.la.template issue1_rows<J>(T.rsA, st, k0, T.kd_hi, tok[J][0], tok[J][1], lda2, wave, lane);
      else T.la.template issue1<J>(T.rsA, st, k0, p.lda, wave);
    } else {
      constexpr int JB = J - Cfg::A_INSTR;
      if constexpr (B_KC)
        T.lb.template issue1<JB, Cfg::STREAM_B>(T.rsB, st + Cfg::A_BYTES, k0, T.kd_hi, k0 + BK > T.kd_hi, wave);
      else if constexpr (GATH == GB_KROWS)
        T.lb.template issue1_rows<JB>(T.rsB, st + Cfg::A_BYTES, k0, T.kd_hi, tok[JB][0], tok[JB][1], ldb2, wave,
                                       lane);
      else T.lb.template issue1<JB>(T.rsB, st + Cfg::A_BYTES, k0, p.ldb, wave);
    }
  };
  // Lane offsets of the [k][r] operands' fragments within a slot, computed
  // once (t_lane_off): a fragment read is then the slot base plus one of
  // these plus an immediate.
  uint32_t toff_a[MI], toff_b[NI];
#pragma unroll
  for (int f = 0; f < MI; ++f) toff_a[f] = A_KC ? 0u : t_lane_off<BM>(a_row0 + f * 32, lane);
#pragma unroll
  for (int j = 0; j < NI; ++j) toff_b[j] = B_KC ? 0u : t_lane_off<BN>(b_row0 + j * 32, lane);
  // Fragment F of substep ks from the slot at sa: F < MI the A rows of block
  // F, then the B rows of block F - MI.
  auto load_frag = [&](const char* sa, int ks, auto fc, bf16x8 (&af)[MI], bf16x8 (&bfr)[NI]) {
    constexpr int F = decltype(fc)::value;
    if constexpr (F < MI) {
      if constexpr (A_KC) af[F] = kc_frag<BK>(sa, a_row0 + F * 32 + (lane & 31), ks * 2 + (lane >> 5));
      else af[F] = t_frag_at<BM>(sa, toff_a[F], ks);
    } else {
      const char* sb = sa + Cfg::A_BYTES;
      constexpr int J = F - MI;
      if constexpr (B_KC) bfr[J] = kc_frag<BK>(sb, b_row0 + J * 32 + (lane & 31), ks * 2 + (lane >> 5));
      else bfr[J] = t_frag_at<BN>(sb, toff_b[J], ks);
    }
  };
  auto load_frags = [&](const char* sa, int ks, bf16x8 (&af)[MI], bf16x8 (&bfr)[NI]) {
    static_for<0, MI + NI>([&](auto fc) { load_frag(sa, ks, fc, af, bfr); });
  };

  f32x16 acc[MI][NI];
  // One 16-k substep; the stage's D DMAs ride on its MFMAs, and the MI + NI
  // fragments of the next substep (substep ksn of the slot at sn, into afn /
  // bfn) are read one after each MFMA rather than all before the first: a wave
  // issues in order, so a burst of fragment reads that waits for room in the
  // LDS queue (every wave reads at once after a barrier) would hold back the
  // MFMAs behind it.
  auto substep = [&](auto ksc, const bf16x8 (&af)[MI], const bf16x8 (&bfr)[NI], const LoadTile& T, int ls,
                     int g, const int (&tok)[GI][2], const char* sn, int ksn, bf16x8 (&afn)[MI], bf16x8 (&bfn)[NI]) {
    constexpr int KSI = decltype(ksc)::value;
    // The weight gradients (short k-loops, an epilogue per 16 stages) gain
    // from letting the wave that issues its MFMAs keep the SIMD (measured
    // ~1.5 %); the row-grouped GEMMs lose about as much, so only GM_RED raises it.
    if constexpr (GM == GM_RED) __builtin_amdgcn_s_setprio(1);
    static_for<0, MI * NI>([&](auto mc) {
      constexpr int M = decltype(mc)::value;
      acc[M / NI][M % NI] = mfma16<typename Cfg::Tc>(af[M / NI], bfr[M % NI], acc[M / NI][M % NI]);
      if constexpr (kInterleaveFrags) {
        // the fragments left when this is the last MFMA (fewer MFMAs than fragments)
        constexpr int F1 = M + 1 < MI * NI ? M + 1 : MI + NI;
        static_for<M, (F1 < MI + NI ? F1 : MI + NI)>([&](auto fc) { load_frag(sn, ksn, fc, afn, bfn); });
      }
      constexpr int G = KSI * MI * NI + M;
      static_for<0, D>([&](auto dc) {
        constexpr int DI = decltype(dc)::value;
        if constexpr (dma_slot<D, TOTM>(DI) == G) {
          dma_one(T, ls, g, tok, dc);
          // keep the DMA between its MFMAs (MFMAs are not memory operations,
          // so the DMA's memory clobber alone would let them drift past it)
          __builtin_amdgcn_sched_barrier(0);
        }
      });
      // pin each MFMA's fragment reads behind it
      if constexpr (kInterleaveFrags) __builtin_amdgcn_sched_barrier(0);
    });
    if constexpr (GM == GM_RED) __builtin_amdgcn_s_setprio(0);
  };

  LoadTile cur, nxt;
  int kt_tile = 0;  // this block's tile counter
  setup(tile_at(0), cur);
  setup(tile_at(1), nxt);
  int tok[GI][2], tok_next[GI][2];
  // prologue: stream stages 0 .. NS-2 (all in the first tile: nk >= NS - 1)
  for (int s0 = 0; s0 < NS - 1; ++s0) {
    tokens(cur, s0, tok);
    static_for<0, D>([&](auto jc) { dma_one(cur, s0, s0, tok, jc); });
  }
  wait_vmcnt<0>();  // stages 0 .. NS-2 have landed: a tile's stage 0 never waits
  lds_barrier();
  bf16x8 af[2][MI], bfr[2][NI];
  load_frags(smem, 0, af[0], bfr[0]);

  for (;;) {
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NI; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    const int nk = cur.nk;
    // tokens of stage 0's DMAs (stream stage gs + NS - 1: this tile's stage NS - 1, or the next tile's)
    if constexpr (KGATH) tokens(NS - 1 >= nk ? nxt : cur, NS - 1 >= nk ? NS - 1 - nk : NS - 1, tok);
    // One stage; its DMAs fetch stream stage g + NS - 1 (stage ls of tile T),
    // which lies in the next tile in a tile's last NS - 1 stages.
    auto run_stage = [&](int kt, const LoadTile& T, int ls) {
      const int g = gs + kt;
      const char* sa = smem + slot_of(g);
      const int s = kt + NS - 1;
      if constexpr (KGATH) {
        // The token reads of the k-row gathers are scalar loads, which return
        // out of order: while one is outstanding the compiler can only wait
        // for an LDS fragment with lgkmcnt(0), which would also wait for the
        // fragments of the next substep just issued. Waiting here, where the
        // tokens (issued a substep ago) and this substep's fragments have
        // landed, leaves no scalar load in flight, so the fragment waits below
        // count LDS reads exactly. (Measured at the Qwen3-30B-A3B shape: the
        // same speed either way; this loop is bound by its loads.)
        __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0)
      }
      static_for<0, KS - 1>([&](auto ksc) {
        constexpr int KSI = decltype(ksc)::value;
        if constexpr (!kInterleaveFrags) load_frags(sa, KSI + 1, af[(KSI + 1) & 1], bfr[(KSI + 1) & 1]);
        substep(ksc, af[KSI & 1], bfr[KSI & 1], T, ls, g + NS - 1, tok, sa, KSI + 1, af[(KSI + 1) & 1],
                bfr[(KSI + 1) & 1]);
      });
      // stream stage g + 1 has landed (this wave's share): outstanding are
      // only the full stages g + 2 .. g + NS - 2 and the DMAs this stage
      // issued before here
      if (kt > 0) wait_vmcnt<WAIT_N>();
      lds_barrier();               // ... every wave's share; every wave is done with slot g but for registers
      if constexpr (KGATH) {
        // the next stage's DMAs (stream stage g + NS: within this tile or the
        // next, since the next tile has at least NS - 1 stages); read here so
        // that the scalar reads run under this stage's last MFMAs rather than
        // in front of a fragment wait (LDS and scalar reads share a counter)
        if (kt + 1 < nk) {
          const bool nn = s + 1 >= nk;
          tokens(nn ? nxt : cur, nn ? s + 1 - nk : s + 1, tok_next);
        }
      }
      // stream stage g + 1: this tile's next stage, or the next tile's first
      if constexpr (!kInterleaveFrags) load_frags(smem + slot_of(g + 1), 0, af[0], bfr[0]);
      substep(std::integral_constant<int, KS - 1>(), af[1], bfr[1], T, ls, g + NS - 1, tok, smem + slot_of(g + 1), 0,
              af[0], bfr[0]);
      if constexpr (KGATH) {
#pragma unroll
        for (int i = 0; i < GI; ++i) {
          tok[i][0] = tok_next[i][0];
          tok[i][1] = tok_next[i][1];
        }
      }
    };
    if constexpr (kSplitStages) {
      // two loops, so that neither selects between the tiles' descriptors
      // and DMA offsets stage by stage
      const int kt_next = nk - (NS - 1);  // >= 0: nk >= NS - 1
#pragma unroll 1
      for (int kt = 0; kt < kt_next; ++kt) run_stage(kt, cur, kt + NS - 1);
#pragma unroll 1
      for (int kt = kt_next; kt < nk; ++kt) run_stage(kt, nxt, kt + NS - 1 - nk);
    } else {
      for (int kt = 0; kt < nk; ++kt) {
        const bool in_next = kt + NS - 1 >= nk;
        LoadTile T;
#pragma unroll
        for (int w = 0; w < 4; ++w) {  // uniform: the descriptors stay in SGPRs
          T.rsA[w] = __builtin_amdgcn_readfirstlane(in_next ? nxt.rsA[w] : cur.rsA[w]);
          T.rsB[w] = __builtin_amdgcn_readfirstlane(in_next ? nxt.rsB[w] : cur.rsB[w]);
        }
        T.la.select(in_next, nxt.la, cur.la);
        T.lb.select(in_next, nxt.lb, cur.lb);
        T.kd0 = in_next ? nxt.kd0 : cur.kd0;
        T.kd_hi = in_next ? nxt.kd_hi : cur.kd_hi;
        run_stage(kt, T, in_next ? kt + NS - 1 - nk : kt + NS - 1);
      }
    }
    // The next tile's first NS - 1 stages were issued during this tile's last
    // stages; wait for them before the epilogue issues its stores. The vector
    // memory counter also counts stores, so a wait placed after them (at the
    // next tile's stage 0) would hold every wave until its stores drained;
    // here the stores get a whole stage to drain before the next wait.
    wait_vmcnt<0>();
    store_slabs<Cfg, Tout, GM, EPI, PACK, SLAB>(acc, stage, cur.ti, p, wm, wn, lane);
    gs += nk;
    ++kt_tile;
    if (tile_at(kt_tile) < 0) break;
    cur = nxt;
    setup(tile_at(kt_tile + 1), nxt);
  }
  wait_vmcnt<0>();  // the zero-reading DMAs past the last tile
}

// Tout defaults to the configuration's 16-bit operand format.
template <class Cfg, bool A_KC, bool B_KC, int GM, int EPI, typename Tout = typename Cfg::Tc, int GATH = G_NONE>
hipError_t launch_gemm_persist(const GemmParams& p, int num_cus, hipStream_t s) {
  if (p.groups > 1024) return hipErrorInvalidValue;
  const int grid = num_cus > 0 ? num_cus : 256;
  hipLaunchKernelGGL((grouped_gemm_persist_kernel<Cfg, Tout, A_KC, B_KC, GM, EPI, GATH>), dim3(grid), dim3(Cfg::NT), 0,
                     s, p);
  return hipGetLastError();
}

// The two forward expert GEMMs on the persistent kernel (the tile shapes used
// for few-token batches serve the forward only). Operands and outputs are in
// the configuration's 16-bit format T16.
template <class Cfg, typename T16 = typename Cfg::Tc>
hipError_t expert_gemm_persist_fwd(int kind, const T16* A, const T16* B, T16* C, T16* C2, const int32_t* offs, int P,
                                   int E, int H, int I, const ExpertGather& xg, int num_cus, hipStream_t s) {
  GemmParams p = expert_params<T16>(kind, A, B, nullptr, C, C2, offs, P, E, H, I, xg);
  switch (kind) {
    case EG_GATE_UP_FWD:
      if (p.a_index != nullptr)
        return launch_gemm_persist<Cfg, true, true, GM_ROWS, EPI_SWIGLU, T16, GA_ROWS>(p, num_cus, s);
      return launch_gemm_persist<Cfg, true, true, GM_ROWS, EPI_SWIGLU>(p, num_cus, s);
    case EG_DOWN_FWD: return launch_gemm_persist<Cfg, true, true, GM_ROWS, EPI_STORE>(p, num_cus, s);
  }
  return hipErrorInvalidValue;
}

// The row-grouped expert GEMMs (forward and dgrad) on the persistent kernel;
// a tile shape that serves only them (the weight gradients' k-row gathers
// take 256-row tiles) is instantiated through this alone.
template <class Cfg, typename T16 = typename Cfg::Tc>
hipError_t expert_gemm_persist_rows(int kind, const T16* A, const T16* B, const T16* aux, T16* C, T16* C2,
                                    const int32_t* offs, int P, int E, int H, int I, const ExpertGather& xg,
                                    int num_cus, hipStream_t s) {
  GemmParams p = expert_params(kind, A, B, aux, C, C2, offs, P, E, H, I, xg);
  const bool gath = xg.index != nullptr;
  switch (kind) {
    case EG_GATE_UP_FWD:
      if (gath) return launch_gemm_persist<Cfg, true, true, GM_ROWS, EPI_SWIGLU, T16, GA_ROWS>(p, num_cus, s);
      return launch_gemm_persist<Cfg, true, true, GM_ROWS, EPI_SWIGLU>(p, num_cus, s);
    case EG_DOWN_FWD: return launch_gemm_persist<Cfg, true, true, GM_ROWS, EPI_STORE>(p, num_cus, s);
    case EG_DOWN_DGRAD:
      if (gath) return launch_gemm_persist<Cfg, true, false, GM_ROWS, EPI_SWIGLU_BWD, T16, GA_ROWS>(p, num_cus, s);
      return launch_gemm_persist<Cfg, true, false, GM_ROWS, EPI_SWIGLU_BWD>(p, num_cus, s);
    case EG_GATE_UP_DGRAD: return launch_gemm_persist<Cfg, true, false, GM_ROWS, EPI_STORE>(p, num_cus, s);
  }
  return hipErrorInvalidValue;
}

// The six expert GEMMs on the persistent kernel; Tw is the weight gradients'
// type (the operands' 16-bit format, or fp32 for fp32 master weights: the
// accumulators stored unrounded). A gathered operand takes the GATH instance
// of its GEMM.
template <class Cfg, typename Tw = typename Cfg::Tc, typename T16 = typename Cfg::Tc>
hipError_t expert_gemm_persist(int kind, const T16* A, const T16* B, const T16* aux, T16* C, T16* C2, Tw* Cw,
                               const int32_t* offs, int P, int E, int H, int I, const ExpertGather& xg, int num_cus,
                               hipStream_t s) {
  if (kind != EG_DOWN_WGRAD && kind != EG_GATE_UP_WGRAD)
    return expert_gemm_persist_rows<Cfg>(kind, A, B, aux, C, C2, offs, P, E, H, I, xg, num_cus, s);
  GemmParams p = expert_params(kind, A, B, aux, C, C2, offs, P, E, H, I, xg);
  p.C = Cw;
  if (xg.index == nullptr) return launch_gemm_persist<Cfg, false, false, GM_RED, EPI_STORE, Tw>(p, num_cus, s);
  if (kind == EG_DOWN_WGRAD) return launch_gemm_persist<Cfg, false, false, GM_RED, EPI_STORE, Tw, GA_KROWS>(p, num_cus, s);
  return launch_gemm_persist<Cfg, false, false, GM_RED, EPI_STORE, Tw, GB_KROWS>(p, num_cus, s);
}

}  // namespace pmoe
