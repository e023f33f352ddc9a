// fp8 x fp8 path of the Forge GEMM (forge/gemm/fp8.py:22-76 with
// quantize_input=True): activations quantized per tensor to e4m3 on the
// device, then a GEMM whose both operands are e4m3 codes, on gfx950's
// v_mfma_f32_16x16x128_f8f6f4, the two per-tensor scales applied in the
// epilogue.  The instruction multiplies the codes exactly but sums each
// block of 128 products below f32 precision (measured: within 2^-14 of the
// block's largest product); the blocks accumulate in f32.
#include "smoe_common.hpp"
#include "smoe_internal.hpp"

namespace smoe {
namespace {

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void* lds_ptr;
typedef __attribute__((address_space(1))) void* gbl_ptr;

constexpr float kE4m3Max = 448.0f;

// max that keeps a NaN once seen (torch's amax propagates NaN)
__device__ __forceinline__ float nan_max(float m, float a) { return (a > m || a != a) ? a : m; }

__device__ __forceinline__ float wave_nan_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = nan_max(v, __shfl_xor(v, o));
  return v;
}

// float -> OCP e4m3fn code, round to nearest even, not saturating: the cast
// torch.Tensor.to(torch.float8_e4m3fn) performs (|v| > 464 and NaN -> the
// NaN code S.1111.111; 464 itself ties to 448).
__device__ __forceinline__ uint32_t f32_to_e4m3(float v) {
  const uint32_t b = __float_as_uint(v);
  const uint32_t sign = (b >> 24) & 0x80u;
  const uint32_t a = b & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7fu;              // NaN
  const float av = __uint_as_float(a);
  if (av < 0.015625f) {                                  // below 2^-6: subnormal codes m * 2^-9
    const float q = __builtin_rintf(av * 512.0f);        // exact scaling, RNE to 0 .. 8
    return sign | static_cast<uint32_t>(q);              // 8 reads as the smallest normal
  }
  int e = static_cast<int>(a >> 23) - 127;               // >= -6
  uint32_t m = (a >> 20) & 7u;
  const uint32_t rem = a & 0xfffffu;
  if (rem > 0x80000u || (rem == 0x80000u && (m & 1u))) ++m;
  if (m == 8u) {
    m = 0;
    ++e;
  }
  if (e > 8 || (e == 8 && m == 7u)) return sign | 0x7fu;  // above 464: NaN (inf too)
  return sign | (static_cast<uint32_t>(e + 7) << 3) | m;
}

template <int XDT>
__device__ __forceinline__ float load_x(const void* x, int64_t i) {
  if constexpr (XDT == SMOE_F32) return reinterpret_cast<const float*>(x)[i];
  else if constexpr (XDT == SMOE_BF16) return bf2f(reinterpret_cast<const uint16_t*>(x)[i]);
  else return static_cast<float>(reinterpret_cast<const _Float16*>(x)[i]);
}

// Partial amax |x| of each workgroup's grid-stride share.
template <int XDT>
__global__ __launch_bounds__(256) void k_amax_partial(const void* __restrict__ x, int64_t n,
                                                      float* __restrict__ partial) {
  __shared__ float red[4];
  float m = 0.f;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * 256)
    m = nan_max(m, fabsf(load_x<XDT>(x, i)));
  m = wave_nan_max(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0)
    partial[blockIdx.x] = nan_max(nan_max(red[0], red[1]), nan_max(red[2], red[3]));
}

// scale = max(amax / 448, 1e-12) (quant.py:30-33), codes = e4m3(x / scale)
// (quant.py:52), 4 codes per thread; columns cols .. ld_out-1 of each row
// are written as code 0 (value 0: the GEMM's K padding).
template <int XDT>
__global__ __launch_bounds__(256) void k_quant_fp8(const void* __restrict__ x, int rows, int cols,
                                                   int ld_out, const float* __restrict__ partial,
                                                   int nparts, uint8_t* __restrict__ codes,
                                                   float* __restrict__ scale_out) {
  __shared__ float s_scale;
  if (threadIdx.x < 64) {
    float m = 0.f;
    for (int i = threadIdx.x; i < nparts; i += 64) m = nan_max(m, partial[i]);
    m = wave_nan_max(m);
    if (threadIdx.x == 0) {
      float sc = __fdiv_rn(m, kE4m3Max);
      sc = sc < 1e-12f ? 1e-12f : sc;  // clamp_min (a NaN scale stays NaN)
      s_scale = sc;
      if (blockIdx.x == 0) *scale_out = sc;
    }
  }
  __syncthreads();
  const float sc = s_scale;
  const int quads = ld_out >> 2;
  const int64_t total = static_cast<int64_t>(rows) * quads;
  for (int64_t q = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; q < total;
       q += static_cast<int64_t>(gridDim.x) * 256) {
    const int r = static_cast<int>(q / quads);
    const int c0 = static_cast<int>(q - static_cast<int64_t>(r) * quads) * 4;
    uint32_t word = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = c0 + i;
      if (c < cols) {
        const float v = load_x<XDT>(x, static_cast<int64_t>(r) * cols + c);
        word |= f32_to_e4m3(__fdiv_rn(v, sc)) << (8 * i);
      }
    }
    *reinterpret_cast<uint32_t*>(codes + static_cast<int64_t>(r) * ld_out + c0) = word;
  }
}

// Per-row scales (quant.py:146-169 with a per-row amax, the block's fp8
// expert format): one wave per row, scale[r] = max(amax_r / 448, 1e-12),
// codes = e4m3(x / scale[r]); columns cols .. ld_out-1 get code 0.
template <int XDT>
__global__ __launch_bounds__(256) void k_quant_fp8_rows(const void* __restrict__ x, int rows,
                                                        int cols, int ld_out,
                                                        uint8_t* __restrict__ codes,
                                                        float* __restrict__ scale) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;  // wave-uniform
  const int64_t rb = static_cast<int64_t>(r) * cols;
  float m = 0.f;
  for (int c = lane; c < cols; c += 64) m = nan_max(m, fabsf(load_x<XDT>(x, rb + c)));
  m = wave_nan_max(m);
  float sc = __fdiv_rn(m, kE4m3Max);
  sc = sc < 1e-12f ? 1e-12f : sc;
  if (lane == 0) scale[r] = sc;
  for (int q = lane; q < (ld_out >> 2); q += 64) {
    uint32_t word = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = 4 * q + i;
      if (c < cols) word |= f32_to_e4m3(__fdiv_rn(load_x<XDT>(x, rb + c), sc)) << (8 * i);
    }
    *reinterpret_cast<uint32_t*>(codes + static_cast<int64_t>(r) * ld_out + 4 * q) = word;
  }
}

// LDS rows of 64 B, chunk c of row r at c ^ ((r >> 1) & 3) (the ring
// kernels' conflict-free layout).
__device__ __forceinline__ int swz64(int row, int chunk) {
  return row * 64 + ((chunk ^ ((row >> 1) & 3)) << 4);
}

template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (0xF << 8));
}
__device__ __forceinline__ void wait_lgkm() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// out[m, n] = act(xs * ws * sum_k X[m, k] W[n, k] + bias[n]) over e4m3
// codes X [N, ldx], W [N_out, ldw] (K a multiple of 256, zero-padded).
//
// 128 x 128 block tile, 4 waves in a 2 x 2 grid (wave tile 64 x 64), K
// advancing 128 per stage through a 3-stage LDS ring (32 KB a stage) fed
// by global_load_lds_dwordx4.  A stage keeps each operand as two 64-byte
// halves of its 128-byte k slice ([X k 0-63][X k 64-127][W k 0-63][W k
// 64-127], 8 KB each, the swizzle above); a lane's 32-byte MFMA fragment
// (row l % 16, k bytes 32 (l / 16) ..) is two ds_read_b128 from one half.
// Both operands use the same lane -> k assignment, so every lane group
// multiplies matching k.  Fragments of stage s+1 are read into a second
// register set while stage s's 16 MFMAs run.
template <int EPI, int ODT>
__global__ __launch_bounds__(256) void k_gemm_f8f8(const uint8_t* __restrict__ X, int ldx,
                                                   const uint8_t* __restrict__ W, int ldw,
                                                   const float* __restrict__ xs,
                                                   const float* __restrict__ ws,
                                                   const float* __restrict__ bias, int N, int K,
                                                   int N_out, void* __restrict__ out, int ldo,
                                                   int tiles_m) {
  constexpr int BM = 128, BN = 128, NS = 3, SUB = 128 * 64, STAGE = 4 * SUB, LD = 8;
  __shared__ __attribute__((aligned(1024))) uint8_t ring[NS * STAGE];
  const int tm = blockIdx.x % tiles_m, tn = blockIdx.x / tiles_m;
  const int m0 = tm * BM, n0 = tn * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // DMA: instruction q = wave + 4 j (j < 8) of a stage covers operand q >> 4
  // (0 X, 1 W), half (q >> 3) & 1, rows 16 (q & 7) ..; lane i: row i / 4,
  // physical chunk i % 4, loading the logical chunk the swizzle puts there
  const uint8_t* src[LD];
  int dst[LD];
  {
    const int pr = lane >> 2, pc = lane & 3;
#pragma unroll
    for (int j = 0; j < LD; ++j) {
      const int q = wave + 4 * j;
      const int op = q >> 4, half = (q >> 3) & 1, rb = q & 7;
      const int r = rb * 16 + pr;
      const int lc = pc ^ ((r >> 1) & 3);
      if (op == 0) {
        const int row = m0 + r < N ? m0 + r : N - 1;  // rows past the end: valid data, never stored
        src[j] = X + static_cast<int64_t>(row) * ldx + 64 * half + 16 * lc;
      } else {
        const int row = n0 + r < N_out ? n0 + r : N_out - 1;
        src[j] = W + static_cast<int64_t>(row) * ldw + 64 * half + 16 * lc;
      }
      dst[j] = (op * 2 + half) * SUB + rb * 1024;
    }
  }
  auto issue = [&](int stage) {
    uint8_t* base = ring + (stage % NS) * STAGE;
    const int k0 = stage * 128;
#pragma unroll
    for (int j = 0; j < LD; ++j)
      __builtin_amdgcn_global_load_lds((gbl_ptr)(src[j] + k0), (lds_ptr)(base + dst[j]), 16, 0, 0);
  };

  const int fr = lane & 15, g = lane >> 4;
  const int half = g >> 1, c0 = 2 * (g & 1);
  i32x8 xa[4], wa[4], xb[4], wb[4];
  auto read_frags = [&](int stage, i32x8 (&xf)[4], i32x8 (&wf)[4]) {
    const uint8_t* sx = ring + (stage % NS) * STAGE + half * SUB;
    const uint8_t* sw = sx + 2 * SUB;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = wm * 64 + i * 16 + fr;
      const u32x4 lo = *reinterpret_cast<const u32x4*>(sx + swz64(r, c0));
      const u32x4 hi = *reinterpret_cast<const u32x4*>(sx + swz64(r, c0 + 1));
      xf[i] = __builtin_bit_cast(i32x8, (uint32_t __attribute__((ext_vector_type(8)))){
                                            lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w});
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = wn * 64 + j * 16 + fr;
      const u32x4 lo = *reinterpret_cast<const u32x4*>(sw + swz64(r, c0));
      const u32x4 hi = *reinterpret_cast<const u32x4*>(sw + swz64(r, c0 + 1));
      wf[j] = __builtin_bit_cast(i32x8, (uint32_t __attribute__((ext_vector_type(8)))){
                                            lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w});
    }
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[j][i] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int KT = K / 128;  // even: K % 256 == 0
  auto step = [&](int s, i32x8 (&xc)[4], i32x8 (&wc)[4], i32x8 (&xn)[4], i32x8 (&wn_)[4]) {
    if (s + 1 < KT) {
      if (s + NS - 1 < KT) wait_vm<(NS - 2) * LD>();
      else wait_vm<0>();
      wait_lgkm();
      __builtin_amdgcn_s_barrier();
      if (s + NS < KT) issue(s + NS);  // into stage s's slot: its fragments are in registers
      read_frags(s + 1, xn, wn_);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        acc[j][i] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wc[j], xc[i], acc[j][i], 0, 0, 0,
                                                                     0, 0, 0);
  };

#pragma unroll
  for (int st = 0; st < NS; ++st)
    if (st < KT) issue(st);
  if (KT >= NS) wait_vm<(NS - 1) * LD>();
  else wait_vm<0>();
  __builtin_amdgcn_s_barrier();
  read_frags(0, xa, wa);
  for (int s = 0; s < KT; s += 2) {
    step(s, xa, wa, xb, wb);
    step(s + 1, xb, wb, xa, wa);
  }

  // epilogue: lane holds channels n .. n+3 (4 (l / 16) + v) of row m (l % 16)
  const float sc = xs[0] * ws[0];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int n = n0 + wn * 64 + j * 16 + 4 * g;
    float b4[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) b4[v] = (bias && n + v < N_out) ? bias[n + v] : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = m0 + wm * 64 + i * 16 + fr;
      if (m >= N) continue;
      float o[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float y = acc[j][i][v] * sc + b4[v];
        o[v] = EPI == 1 ? gelu_erf(y) : y;
      }
      const int64_t base = static_cast<int64_t>(m) * ldo + n;
      if (ODT == SMOE_F32) {
        float* po = reinterpret_cast<float*>(out) + base;
        if (n + 3 < N_out && (base & 3) == 0) {
          *reinterpret_cast<f32x4*>(po) = f32x4{o[0], o[1], o[2], o[3]};
        } else {
#pragma unroll
          for (int v = 0; v < 4; ++v)
            if (n + v < N_out) po[v] = o[v];
        }
      } else {
        uint16_t* po = reinterpret_cast<uint16_t*>(out) + base;
        if (n + 3 < N_out && (base & 3) == 0) {
          *reinterpret_cast<u32x2*>(po) = u32x2{pack_bf2(o[0], o[1]), pack_bf2(o[2], o[3])};
        } else {
#pragma unroll
          for (int v = 0; v < 4; ++v)
            if (n + v < N_out) po[v] = f2bf(o[v]);
        }
      }
    }
  }
}

int rc() { return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP; }

constexpr int kAmaxParts = 1024;

}  // namespace

size_t quantize_fp8_workspace_bytes() { return kAmaxParts * sizeof(float); }

int launch_quantize_fp8(const void* x, int xdt, int rows, int cols, int ld_out, int per_row,
                        uint8_t* codes, float* scale, void* workspace, hipStream_t s) {
  if (rows < 1 || cols < 1 || ld_out < cols || ld_out % 4) return SMOE_EINVAL;
  if (per_row) {
    auto go = [&](auto xd) {
      hipLaunchKernelGGL((k_quant_fp8_rows<decltype(xd)::value>), dim3((rows + 3) / 4), dim3(256),
                         0, s, x, rows, cols, ld_out, codes, scale);
      return rc();
    };
    switch (xdt) {
      case SMOE_F32: return go(std::integral_constant<int, SMOE_F32>{});
      case SMOE_BF16: return go(std::integral_constant<int, SMOE_BF16>{});
      case SMOE_F16: return go(std::integral_constant<int, SMOE_F16>{});
      default: return SMOE_EUNSUPPORTED;
    }
  }
  const int64_t n = static_cast<int64_t>(rows) * cols;
  const int parts = static_cast<int>(std::min<int64_t>(kAmaxParts, (n + 4095) / 4096));
  float* partial = static_cast<float*>(workspace);
  const int64_t quads = static_cast<int64_t>(rows) * (ld_out / 4);
  const int qblocks = static_cast<int>(std::min<int64_t>(4096, (quads + 255) / 256));
  auto run = [&](auto xd) {
    constexpr int XD = decltype(xd)::value;
    hipLaunchKernelGGL((k_amax_partial<XD>), dim3(parts), dim3(256), 0, s, x, n, partial);
    hipLaunchKernelGGL((k_quant_fp8<XD>), dim3(qblocks), dim3(256), 0, s, x, rows, cols, ld_out,
                       partial, parts, codes, scale);
    return rc();
  };
  switch (xdt) {
    case SMOE_F32: return run(std::integral_constant<int, SMOE_F32>{});
    case SMOE_BF16: return run(std::integral_constant<int, SMOE_BF16>{});
    case SMOE_F16: return run(std::integral_constant<int, SMOE_F16>{});
    default: return SMOE_EUNSUPPORTED;
  }
}

int launch_gemm_f8f8(const uint8_t* xq, int ldx, const float* xs, const uint8_t* wq, int ldw,
                     const float* ws, const float* bias, int N, int K, int N_out, int gelu,
                     void* out, int odt, int ldo, hipStream_t s) {
  if (N < 0 || K <= 0 || K % 256 || N_out <= 0 || ldx < K || ldw < K || ldx % 16 || ldw % 16 ||
      ldo < N_out)
    return SMOE_EINVAL;
  if (N == 0) return SMOE_OK;
  const int tiles_m = (N + 127) / 128, tiles_n = (N_out + 127) / 128;
  const dim3 grid(tiles_m * tiles_n), block(256);
  auto go = [&](auto epi, auto od) {
    SMOE_LAUNCH((k_gemm_f8f8<decltype(epi)::value, decltype(od)::value>), grid, block, 0, s, xq,
                ldx, wq, ldw, xs, ws, bias, N, K, N_out, out, ldo, tiles_m);
    return rc();
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using OF = std::integral_constant<int, SMOE_F32>;
  using OB = std::integral_constant<int, SMOE_BF16>;
  if (odt == SMOE_F32) return gelu ? go(I1{}, OF{}) : go(I0{}, OF{});
  if (odt == SMOE_BF16) return gelu ? go(I1{}, OB{}) : go(I0{}, OB{});
  return SMOE_EUNSUPPORTED;
}

}  // namespace smoe
