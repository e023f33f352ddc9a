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
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// ------------------------------------------------- separately rounded ----
// A product and a sum each rounded on its own, as a CPU computes a * b + c
// without fma.  HIP's __fmul_rn / __fadd_rn are the plain operators, which
// -ffp-contract=fast fuses into one fma; operations written under
// contract(off) carry no contraction flag, so they stay apart after inlining.
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}
__device__ __forceinline__ double mul_rn(double a, double b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ double add_rn(double a, double b) {
#pragma clang fp contract(off)
  return a + b;
}

// ---------------------------------------------------------------- bf16 ----
__device__ __forceinline__ float bf2f(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}
__device__ __forceinline__ uint16_t f2bf(float f) {  // RNE (v_cvt_pk_bf16_f32)
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
// Two floats -> two RNE bf16 in one u32 (lo in the low half), as one
// v_cvt_pk_bf16_f32 (two scalar conversions would add shifts and ors).
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  typedef float f32v2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16v2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32v2{lo, hi}, bf16v2));
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
// one scale -> 8 bf16 (RNE of q * s computed in fp32).  A nibble n holds
// q = n - 16 [n >= 8]; u = n ^ 8 = q + 8 in 0..15 sits alone in a byte after
// one xor and a mask (low nibbles) or a shift and a mask (high nibbles), is
// widened by a byte-to-float conversion, and q * s = fma(u, s, -8 s) with one
// rounding (-8 s is exact), the same bits as float(q) * s.  The empty asm
// hides the masks from the optimizer, which would otherwise fold each byte
// back into a bit-field extract ahead of a byte-0 conversion (two VALU
// operations per element instead of one v_cvt_f32_ubyteN).
__device__ __forceinline__ u32x4 int4x8_to_bf16x8(uint32_t w, float s) {
  const uint32_t x = w ^ 0x88888888u;
  uint32_t lo = x & 0x0F0F0F0Fu, hi = (x >> 4) & 0x0F0F0F0Fu;
  asm("" : "+v"(lo), "+v"(hi));
  const float m = -8.f * s;
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float fl = static_cast<float>((lo >> (8 * i)) & 0xFFu);
    const float fh = static_cast<float>((hi >> (8 * i)) & 0xFFu);
    r[i] = pack_bf2(__builtin_fmaf(fl, s, m), __builtin_fmaf(fh, s, m));
  }
  return r;
}

__device__ __forceinline__ float load_scale(const void* p, int64_t i, int is_f16) {
  if (is_f16) return static_cast<float>(reinterpret_cast<const _Float16*>(p)[i]);
  return reinterpret_cast<const float*>(p)[i];
}

// ----------------------------------------------------------- reductions ----
// Wave reductions: within each 16-lane row by DPP (quad_perm xor 1, xor 2,
// row_half_mirror, row_mirror: after them every lane holds its row's
// result), then the four rows' results read from lanes 0, 16, 32, 48 and
// combined uniformly.  A DPP step costs a few cycles where a ds_bpermute
// shuffle waits on LDS.  Every lane of the wave must be active.
template <int CTRL>
__device__ __forceinline__ int dpp_i(int x) {
  return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __int_as_float(dpp_i<CTRL>(__float_as_int(x)));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7 - i within 8
constexpr int kDppMirror = 0x140;      // lane i <-> 15 - i within 16
__device__ __forceinline__ float lane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f<kDppXor1>(v);
  v += dpp_f<kDppXor2>(v);
  v += dpp_f<kDppHalfMirror>(v);
  v += dpp_f<kDppMirror>(v);
  return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f<kDppXor1>(v));
  v = fmaxf(v, dpp_f<kDppXor2>(v));
  v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_f<kDppMirror>(v));
  return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}
// (value, index) arg-max over the wave; ties -> lowest index.  NaN never wins.
// Branch-free (bitwise, no short circuit): a branch here becomes exec-mask
// bookkeeping whose scalar ops wait on each vector compare.
__device__ __forceinline__ void argmax_take(float& v, int& i, float ov, int oi) {
  const bool take = (ov > v) | ((ov == v) & (oi < i));
  v = take ? ov : v;
  i = take ? oi : i;
}
template <int CTRL>
__device__ __forceinline__ void argmax_dpp(float& v, int& i) {
  argmax_take(v, i, dpp_f<CTRL>(v), dpp_i<CTRL>(i));
}
// Reductions over aligned segments of SEG lanes (SEG = 16, 32 or 64): the
// 16-lane row by the DPP steps above, then xor 16 / xor 32 shuffles; every
// lane gets its segment's result.  Ties of the arg-max go to the lowest
// index; the order of the sum is fixed (deterministic).
template <int SEG>
__device__ __forceinline__ float seg_max(float v) {
  static_assert(SEG == 16 || SEG == 32 || SEG == 64, "segment");
  v = fmaxf(v, dpp_f<kDppXor1>(v));
  v = fmaxf(v, dpp_f<kDppXor2>(v));
  v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_f<kDppMirror>(v));
  if constexpr (SEG >= 32) v = fmaxf(v, __shfl_xor(v, 16));
  if constexpr (SEG >= 64) v = fmaxf(v, __shfl_xor(v, 32));
  return v;
}
template <int SEG>
__device__ __forceinline__ float seg_sum(float v) {
  static_assert(SEG == 16 || SEG == 32 || SEG == 64, "segment");
  v += dpp_f<kDppXor1>(v);
  v += dpp_f<kDppXor2>(v);
  v += dpp_f<kDppHalfMirror>(v);
  v += dpp_f<kDppMirror>(v);
  if constexpr (SEG >= 32) v += __shfl_xor(v, 16);
  if constexpr (SEG >= 64) v += __shfl_xor(v, 32);
  return v;
}
template <int SEG>
__device__ __forceinline__ void seg_argmax(float& v, int& i) {
  static_assert(SEG == 16 || SEG == 32 || SEG == 64, "segment");
  argmax_dpp<kDppXor1>(v, i);
  argmax_dpp<kDppXor2>(v, i);
  argmax_dpp<kDppHalfMirror>(v, i);
  argmax_dpp<kDppMirror>(v, i);
  if constexpr (SEG >= 32) argmax_take(v, i, __shfl_xor(v, 16), __shfl_xor(i, 16));
  if constexpr (SEG >= 64) argmax_take(v, i, __shfl_xor(v, 32), __shfl_xor(i, 32));
}

// More than 64 entries per token (experts / destinations, up to 256): one
// wave per token, lane l holding entries l, l + 64, .. (V slots).
constexpr int kWideBig = 1 << 20;  // index of "no candidate"
// The arg-max takes the lane's best candidate (the lowest index
// on ties) into the wave's arg-max, so ties still go to the lowest index.
template <int V>
__device__ __forceinline__ void wide_argmax(const float (&x)[V], const bool (&cand)[V], float& cv,
                                            int& ci) {
  const int lane = threadIdx.x & 63;
  cv = -INFINITY;
  ci = kWideBig;
#pragma unroll
  for (int v = 0; v < V; ++v)
    if (cand[v] && (ci == kWideBig || x[v] > cv)) {
      cv = x[v];
      ci = lane + 64 * v;
    }
  seg_argmax<64>(cv, ci);
}

// Distinct selected ids ascending across the V lane slots: slot v of lane l
// holds id l + 64 v, so the rank counts the earlier slots' selections and
// this slot's lower lanes.  Returns the number selected.
template <int V>
__device__ __forceinline__ int wide_ranks(const bool (&sel)[V], int (&rank)[V]) {
  const int lane = threadIdx.x & 63;
  const uint64_t lt = (1ull << lane) - 1ull;
  int base = 0;
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const uint64_t m = __ballot(sel[v]);
    rank[v] = base + __popcll(m & lt);
    base += __popcll(m);
  }
  return base;
}

// Inclusive prefix sum over the wave in lane order: Hillis-Steele within
// each 16-lane row (DPP row_shr 1, 2, 4, 8, zero fill), then row_bcast15 /
// row_bcast31 carry the row totals into the rows above.
template <int CTRL>
__device__ __forceinline__ int dpp_shr0(int x) {  // out-of-row sources read 0
  return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xF, 0xF, true);
}
__device__ __forceinline__ int wave_incl_scan(int v) {
  v += dpp_shr0<0x111>(v);
  v += dpp_shr0<0x112>(v);
  v += dpp_shr0<0x114>(v);
  v += dpp_shr0<0x118>(v);
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast15 -> rows 1, 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast31 -> rows 2, 3
  return v;
}

// Workgroup barrier ordering LDS only: waits for the wave's LDS accesses
// (lgkmcnt) but not for its global stores, which no other wave of the
// workgroup reads back.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// s_waitcnt vmcnt(n) (gfx9 encoding; expcnt / lgkmcnt left at "no wait")
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (0xF << 8));
}
// s_waitcnt lgkmcnt(0) (vmcnt / expcnt left at "no wait")
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// address spaces of global_load_lds's operands
typedef __attribute__((address_space(3))) void* lds_vptr;
typedef __attribute__((address_space(1))) void* gbl_vptr;

// LDS rows of 16*CPR bytes: logical 16-byte chunk c of row r sits at chunk
// c ^ ((r / (16 / CPR)) % CPR), so the 16 rows one ds_read phase touches
// cover all 64 banks once (the map is an involution)
template <int CPR>
__device__ __forceinline__ int sw_chunk(int r, int c) {
  return c ^ ((r / (16 / CPR)) & (CPR - 1));
}

__device__ __forceinline__ void wave_argmax(float& v, int& i) {
  argmax_dpp<kDppXor1>(v, i);
  argmax_dpp<kDppXor2>(v, i);
  argmax_dpp<kDppHalfMirror>(v, i);
  argmax_dpp<kDppMirror>(v, i);
  float bv = lane_f(v, 0);
  int bi = __builtin_amdgcn_readlane(i, 0);
#pragma unroll
  for (int r = 16; r < 64; r += 16) argmax_take(bv, bi, lane_f(v, r), __builtin_amdgcn_readlane(i, r));
  v = bv;
  i = bi;
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
