// Per-token row helpers shared by the combine kernels and the decode front:
// 16-byte row loads / stores in bf16 or f32, a batched gather-add of rows,
// and the block epilogue LN(h + alpha * sum_e y + beta * x0) of one token
// row held by one wave (lane l: columns (l + 64 c) * 8 .. + 7, c < CPL).
// Every user computes the LayerNorm through ln_row, so the operations, and
// their order, are the same wherever a row is normalised: the decode front
// that normalises the previous loop's rows gives the bits k_epilogue gives.
#pragma once
#include <type_traits>

#include "smoe_common.hpp"

namespace smoe {

// 8 consecutive elements of a bf16 or f32 array <-> 8 floats, as 16-byte
// vectors.  The dtype is a template argument: a run-time dtype branch would
// make each load wait before the branches join.
template <int DT>
__device__ __forceinline__ void load8(const void* base, int64_t off, float* v) {
  if constexpr (DT == SMOE_F32) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(base) + off);
    const f32x4 b = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(base) + off + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = a[i];
      v[4 + i] = b[i];
    }
  } else {
    const u32x4 a = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(base) + off);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(a[i] << 16);
      v[2 * i + 1] = __uint_as_float(a[i] & 0xFFFF0000u);
    }
  }
}

template <int DT>
__device__ __forceinline__ void store8(void* base, int64_t off, const float* v) {
  if constexpr (DT == SMOE_F32) {
    float* p = reinterpret_cast<float*>(base) + off;
    *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4*>(p + 4) = f32x4{v[4], v[5], v[6], v[7]};
  } else {
    u32x4 a;
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = pack_bf2(v[2 * i], v[2 * i + 1]);
    *reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(base) + off) = a;
  }
}

// Keeps a loaded value live here, so the compiler issues the loads of a
// batch together instead of sinking each into the branch that consumes it.
__device__ __forceinline__ void pin(float x) { asm volatile("" : : "v"(x)); }

// acc += the rows named by the set bits of `live` (lane j of my_row holds a
// row index when bit j is set), in ascending bit order.  Loads of a batch of
// rows are issued together; a batch slot past the last row loads row 0 and
// is not added.
template <int CPL, int DT>
__device__ __forceinline__ void gather_add(const void* __restrict__ base, int H,
                                           int my_row, uint64_t live, float (&acc)[CPL][8]) {
  constexpr int B = CPL >= 8 ? 1 : 8 / CPL;  // rows per batch (<= 8 x 16 B loads per lane)
  const int lane = threadIdx.x & 63;
  while (live) {
    float v[B][CPL][8];
    bool use[B];
#pragma unroll
    for (int b = 0; b < B; ++b) {
      use[b] = live != 0;
      const int src = use[b] ? __ffsll(static_cast<unsigned long long>(live)) - 1 : 0;
      live &= live - 1;
      const int r = __shfl(my_row, src);
      const int64_t row = use[b] ? r : 0;
#pragma unroll
      for (int c = 0; c < CPL; ++c) {  // columns past H load column 0 (not stored)
        const int col = (lane + 64 * c) * 8;
        load8<DT>(base, row * H + (col < H ? col : 0), v[b][c]);
      }
    }
#pragma unroll
    for (int b = 0; b < B; ++b)
#pragma unroll
      for (int c = 0; c < CPL; ++c)
#pragma unroll
        for (int i = 0; i < 8; ++i) pin(v[b][c][i]);
#pragma unroll
    for (int b = 0; b < B; ++b)
#pragma unroll
      for (int c = 0; c < CPL; ++c)
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[c][i] += use[b] ? v[b][c][i] : 0.f;
  }
}

// The residual rows of token t: h, x0 and the LayerNorm parameters (1 / 0
// where null), loaded before the routing-dependent rows.
template <int CPL, int ADT>
__device__ __forceinline__ void ln_load(const void* __restrict__ h, const void* __restrict__ x0,
                                        const float* __restrict__ ln_w,
                                        const float* __restrict__ ln_b, int t, int H,
                                        float (&hv)[CPL][8], float (&xv)[CPL][8],
                                        float (&gw)[CPL][8], float (&gb)[CPL][8]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {  // columns past H load column 0 (not stored)
    const int col = (lane + 64 * c) * 8;
    const int cc = col < H ? col : 0;
    const int64_t o = static_cast<int64_t>(t) * H + cc;
    load8<ADT>(h, o, hv[c]);
    load8<ADT>(x0, o, xv[c]);
    if (ln_w) load8<SMOE_F32>(ln_w, cc, gw[c]);
    else
#pragma unroll
      for (int i = 0; i < 8; ++i) gw[c][i] = 1.f;
    if (ln_b) load8<SMOE_F32>(ln_b, cc, gb[c]);
    else
#pragma unroll
      for (int i = 0; i < 8; ++i) gb[c][i] = 0.f;
  }
}

// out = LayerNorm(h + alpha * d + beta * x0) of the wave's row; d holds the
// summed expert rows on entry and is overwritten.  model.py:317.
template <int CPL>
__device__ __forceinline__ void ln_row(const float (&hv)[CPL][8], const float (&xv)[CPL][8],
                                       const float (&gw)[CPL][8], const float (&gb)[CPL][8],
                                       float (&d)[CPL][8], int H, float alpha, float beta,
                                       float eps, float (&out)[CPL][8]) {
  const int lane = threadIdx.x & 63;
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int col = (lane + 64 * c) * 8;
    if (col < H)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        d[c][i] = (hv[c][i] + alpha * d[c][i]) + beta * xv[c][i];
        s += d[c][i];
      }
  }
  const float mean = wave_sum(s) / static_cast<float>(H);
  float q = 0.f;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int col = (lane + 64 * c) * 8;
    if (col < H)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float z = d[c][i] - mean;
        q += z * z;
      }
  }
  const float rstd = 1.0f / sqrtf(wave_sum(q) / static_cast<float>(H) + eps);
#pragma unroll
  for (int c = 0; c < CPL; ++c)
#pragma unroll
    for (int i = 0; i < 8; ++i) out[c][i] = (d[c][i] - mean) * rstd * gw[c][i] + gb[c][i];
}

// dtype code (SMOE_F32 / SMOE_BF16) -> compile-time constant
template <typename F>
int by_dt(int dt, F&& f) {
  if (dt == SMOE_F32) return f(std::integral_constant<int, SMOE_F32>{});
  if (dt == SMOE_BF16) return f(std::integral_constant<int, SMOE_BF16>{});
  return SMOE_EUNSUPPORTED;
}
// 8-element chunks per lane for a row of H: H <= 512 * CPL
template <typename F>
int by_cpl(int H, F&& f) {
  if (H <= 0 || H % 8) return SMOE_EINVAL;
  if (H <= 512) return f(std::integral_constant<int, 1>{});
  if (H <= 1024) return f(std::integral_constant<int, 2>{});
  if (H <= 2048) return f(std::integral_constant<int, 4>{});
  if (H <= 4096) return f(std::integral_constant<int, 8>{});
  return SMOE_EINVAL;
}

}  // namespace smoe
