// Shared device helpers for the Spider-MoE block kernels (gfx950 / CDNA4).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "smoe.h"

namespace smoe {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// ---------------------------------------------------------------- bf16 ----
__device__ __forceinline__ float bf2f(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}
__device__ __forceinline__ uint16_t f2bf(float f) {  // RNE (v_cvt_pk_bf16_f32)
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  return static_cast<uint32_t>(f2bf(lo)) | (static_cast<uint32_t>(f2bf(hi)) << 16);
}

// ------------------------------------------------------------ fp8 e4m3 ----
// OCP e4m3fn (bias 7, no infinities, S.1111.111 = NaN) — the format of
// torch.float8_e4m3fn.  Decoded exactly to float: the 7 magnitude bits are
// placed at float bit 20 (exponent low bits + mantissa high bits), which
// reads as 2^(e-127) * 1.m (or m * 2^-129 for e == 0), then rebiased by an
// exact multiply with 2^120.  Every e4m3 value is exactly representable in
// bf16, so the bf16 of the result is exact too.
__device__ __forceinline__ float fp8_to_f32(uint32_t byte) {
  const uint32_t mag = byte & 0x7Fu;
  float v = __uint_as_float(mag << 20) * 0x1p120f;
  v = (mag == 0x7Fu) ? __uint_as_float(0x7FC00000u) : v;
  return (byte & 0x80u) ? -v : v;
}

// 4 packed e4m3 codes -> 4 bf16 (as 2 u32), exact.
__device__ __forceinline__ u32x2 fp8x4_to_bf16x4(uint32_t w) {
  // v_cvt_pk_f32_fp8 on gfx950 decodes the OCP e4m3 format; the decode is
  // checked against the full 256-code table by the GPU tests.
  f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), false);
  f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), true);
  // exact values: truncating to the high 16 bits is exact
  u32x2 r;
  r.x = __builtin_amdgcn_perm(__float_as_uint(lo.y), __float_as_uint(lo.x), 0x07060302u);
  r.y = __builtin_amdgcn_perm(__float_as_uint(hi.y), __float_as_uint(hi.x), 0x07060302u);
  return r;
}

// ---------------------------------------------------------------- int4 ----
// 8 signed nibbles of one u32 (element 2i in the low nibble of byte i) times
// one scale -> 8 bf16 (RNE of q * s computed in fp32).
__device__ __forceinline__ u32x4 int4x8_to_bf16x8(uint32_t w, float s) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int b = static_cast<int>((w >> (8 * i)) & 0xFFu);
    const int lo = ((b & 0xF) ^ 8) - 8;
    const int hi = (((b >> 4) & 0xF) ^ 8) - 8;
    r[i] = pack_bf2(static_cast<float>(lo) * s, static_cast<float>(hi) * s);
  }
  return r;
}

__device__ __forceinline__ float load_scale(const void* p, int64_t i, int is_f16) {
  if (is_f16) return static_cast<float>(reinterpret_cast<const _Float16*>(p)[i]);
  return reinterpret_cast<const float*>(p)[i];
}

// ----------------------------------------------------------- reductions ----
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
// (value, index) arg-max over the wave; ties -> lowest index.  NaN never wins.
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(v, o);
    const int oi = __shfl_xor(i, o);
    if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
  }
}

// erf by Abramowitz & Stegun, Handbook of Mathematical Functions, eq. 7.1.26:
// erf(a) = 1 - (a1 t + a2 t^2 + a3 t^3 + a4 t^4 + a5 t^5) exp(-a^2),
// t = 1 / (1 + p a), a >= 0, |error| <= 1.5e-7 (far below the bf16 rounding of
// the values it feeds).
__device__ __forceinline__ float erf_as(float x) {
  const float a = fabsf(x);
  const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f, a, 1.0f));
  float y = fmaf(1.061405429f, t, -1.453152027f);
  y = fmaf(y, t, 1.421413741f);
  y = fmaf(y, t, -0.284496736f);
  y = fmaf(y, t, 0.254829592f);
  y = 1.0f - y * t * __expf(-a * a);
  return copysignf(y, x);
}
__device__ __forceinline__ float gelu_erf(float x) {  // nn.GELU() default (exact-erf GELU)
  return 0.5f * x * (1.0f + erf_as(x * 0.70710678118654752f));
}
__device__ __forceinline__ float silu(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x));
}

}  // namespace smoe
