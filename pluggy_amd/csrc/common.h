// Shared types and device helpers for the pmoe HIP kernels (gfx950 / CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

namespace pmoe {

typedef uint16_t bf16_t;  // bf16 storage: the upper 16 bits of an fp32
typedef _Float16 f16_t;   // IEEE binary16 (fp16)
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// The six grouped GEMMs of the expert FFN (forward, dgrad, wgrad of gate_up and down).
enum ExpertGemm {
  EG_GATE_UP_FWD = 0,  // gu, mid <- x_perm . W_gu[e]^T, SwiGLU epilogue
  EG_DOWN_FWD = 1,     // y <- mid . W_dn[e]^T
  EG_DOWN_DGRAD = 2,   // dgu <- SwiGLU'(gu) * (dy . W_dn[e])
  EG_DOWN_WGRAD = 3,   // dW_dn[e] <- dy_e^T . mid_e
  EG_GATE_UP_DGRAD = 4,  // dx_perm <- dgu . W_gu[e]
  EG_GATE_UP_WGRAD = 5,  // dW_gu[e] <- dgu_e^T . x_perm_e
};

// The token-major side of an expert GEMM, when its expert-sorted rows are
// gathered instead of materialised: the sorted row p of the operand that
// holds tokens (x in EG_GATE_UP_FWD / EG_GATE_UP_WGRAD, the output gradient in
// EG_DOWN_DGRAD / EG_DOWN_WGRAD) is row index[p] of a (rows, .) tensor.
// row_w / part: the routing weight of each sorted row and the partials of its
// gradient (EG_GATE_UP_FWD scales mid by row_w; EG_DOWN_DGRAD takes the
// gradient of the scaled mid and writes the partials).
struct ExpertGather {
  const int32_t* index = nullptr;
  int64_t rows = 0;
  const float* row_w = nullptr;
  float* part = nullptr;
  int part_ld = 0;
};


// ---------------------------------------------------------------- bf16 ----

__device__ __forceinline__ float bf16_to_f32(bf16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Round-to-nearest-even fp32 -> bf16 (NaN stays NaN), written out in integer
// arithmetic so the rounding rule is explicit and identical on every target.
__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<bf16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<bf16_t>(u >> 16);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return static_cast<uint32_t>(f32_to_bf16(lo)) | (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
}

__device__ __forceinline__ float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Load/store 8 consecutive elements of type T as fp32. load_nt: a
// non-temporal load, for rows read once (gathered rows of the row movers).
template <typename T> struct Vec8;

template <> struct Vec8<bf16_t> {
  __device__ static __forceinline__ void load(const bf16_t* p, float* v) {
    u32x4 w = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) { v[2 * i] = bf16lo(w[i]); v[2 * i + 1] = bf16hi(w[i]); }
  }
  __device__ static __forceinline__ void load_nt(const bf16_t* p, float* v) {
    const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
#pragma unroll
    for (int i = 0; i < 4; ++i) { v[2 * i] = bf16lo(w[i]); v[2 * i + 1] = bf16hi(w[i]); }
  }
  __device__ static __forceinline__ void store(bf16_t* p, const float* v) {
    u32x4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
    *reinterpret_cast<u32x4*>(p) = w;
  }
};

template <> struct Vec8<float> {
  __device__ static __forceinline__ void load(const float* p, float* v) {
    f32x4 a = *reinterpret_cast<const f32x4*>(p);
    f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) { v[i] = a[i]; v[4 + i] = b[i]; }
  }
  __device__ static __forceinline__ void load_nt(const float* p, float* v) {
    const f32x4 a = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
    const f32x4 b = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p + 4));
#pragma unroll
    for (int i = 0; i < 4; ++i) { v[i] = a[i]; v[4 + i] = b[i]; }
  }
  __device__ static __forceinline__ void store(float* p, const float* v) {
    f32x4 a, b;
#pragma unroll
    for (int i = 0; i < 4; ++i) { a[i] = v[i]; b[i] = v[4 + i]; }
    *reinterpret_cast<f32x4*>(p) = a;
    *reinterpret_cast<f32x4*>(p + 4) = b;
  }
};

// ---------------------------------------------------------------- fp16 ----
// Conversions follow IEEE rules: fp16 -> fp32 is exact, fp32 -> fp16 rounds to
// nearest even (overflow to +-inf, NaN stays NaN), in the hardware converters.

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float f16lo(uint32_t w) { return (float)__builtin_bit_cast(f16x2_t, w)[0]; }
__device__ __forceinline__ float f16hi(uint32_t w) { return (float)__builtin_bit_cast(f16x2_t, w)[1]; }

// Two fp32 -> packed fp16 (lo in bits 0-15).
__device__ __forceinline__ uint32_t cvt_pk_f16(float lo, float hi) {
  const f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2_t));
}

template <> struct Vec8<f16_t> {
  __device__ static __forceinline__ void load(const f16_t* p, float* v) {
    u32x4 w = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) { v[2 * i] = f16lo(w[i]); v[2 * i + 1] = f16hi(w[i]); }
  }
  __device__ static __forceinline__ void load_nt(const f16_t* p, float* v) {
    const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
#pragma unroll
    for (int i = 0; i < 4; ++i) { v[2 * i] = f16lo(w[i]); v[2 * i + 1] = f16hi(w[i]); }
  }
  __device__ static __forceinline__ void store(f16_t* p, const float* v) {
    u32x4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = cvt_pk_f16(v[2 * i], v[2 * i + 1]);
    *reinterpret_cast<u32x4*>(p) = w;
  }
};

template <typename T> __device__ __forceinline__ float load_scalar(const T* p);
template <> __device__ __forceinline__ float load_scalar<float>(const float* p) { return *p; }
template <> __device__ __forceinline__ float load_scalar<bf16_t>(const bf16_t* p) { return bf16_to_f32(*p); }
template <> __device__ __forceinline__ float load_scalar<f16_t>(const f16_t* p) { return (float)*p; }

template <typename T> __device__ __forceinline__ void store_scalar(T* p, float v);
template <> __device__ __forceinline__ void store_scalar<float>(float* p, float v) { *p = v; }
template <> __device__ __forceinline__ void store_scalar<bf16_t>(bf16_t* p, float v) { *p = f32_to_bf16(v); }
template <> __device__ __forceinline__ void store_scalar<f16_t>(f16_t* p, float v) { *p = (f16_t)v; }

// ------------------------------------------------------------- wave ops ----

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// Inclusive scan over a wave (64 lanes).
__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    int t = __shfl_up(v, o, kWave);
    if (lane >= o) v += t;
  }
  return v;
}

// SiLU and its derivative in fp32: silu(g) = g * sigmoid(g).
__device__ __forceinline__ float sigmoidf_(float g) { return 1.0f / (1.0f + expf(-g)); }

// sigmoid from the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32; each
// about 1 ulp): 1 / (1 + 2^(-g log2 e)). Saturates to 0 / 1 without NaN for
// large |g|.
__device__ __forceinline__ float fast_sigmoid(float g) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -1.4426950408889634f));
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Two fp32 -> packed bf16 (lo in bits 0-15), round to nearest even, with the
// gfx950 conversion instruction (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi) {
  const f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// The 16-bit storage formats of the MFMA paths: packing of two rounded
// values into a dword and the two halves of a dword back to fp32.
template <typename T> struct Fmt16;
template <> struct Fmt16<bf16_t> {
  __device__ static __forceinline__ uint32_t pack2(float lo, float hi) { return cvt_pk_bf16(lo, hi); }
  __device__ static __forceinline__ float lo(uint32_t w) { return bf16lo(w); }
  __device__ static __forceinline__ float hi(uint32_t w) { return bf16hi(w); }
};
template <> struct Fmt16<f16_t> {
  __device__ static __forceinline__ uint32_t pack2(float lo, float hi) { return cvt_pk_f16(lo, hi); }
  __device__ static __forceinline__ float lo(uint32_t w) { return f16lo(w); }
  __device__ static __forceinline__ float hi(uint32_t w) { return f16hi(w); }
};

__device__ __forceinline__ int ceil_div(int a, int b) { return (a + b - 1) / b; }

}  // namespace pmoe
