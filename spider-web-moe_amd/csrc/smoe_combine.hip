// Per-token combines of the Spider-MoE block (one wave per token row).
//
//  msg[t]  = sum over the token's destination rows (ascending destination)
//            of proj[row] (= c * W_edge[d] h, model.py:277-288)
//  h'[t]   = LayerNorm(h + alpha * delta + beta * x0)  (model.py:317), with
//            delta = sum over the token's expert rows with weight > 0
//            (ascending expert, as sparse_experts.py:51-63 accumulates) of
//            y[row] (= w * FFN_e(msg), the down-GEMM epilogue)
//
// A fixed summation order per token and no atomics make every output
// bit-reproducible run to run.  Rows are read as 16-byte vectors; H must be
// a multiple of 8.
#include "smoe_common.hpp"
#include "smoe_internal.hpp"

namespace smoe {

__device__ __forceinline__ void load8(const void* base, int dtype, int64_t off, float* v) {
  if (dtype == SMOE_F32) {
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

__device__ __forceinline__ void store8(void* base, int dtype, int64_t off, const float* v) {
  if (dtype == SMOE_F32) {
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

// CPL = 8-element chunks per lane (H <= 512 * CPL)
// Lane j (< S) fetches the token's j-th (destination, row) entry; the rows
// are then broadcast and all their loads issued before any is consumed.
template <int CPL>
__global__ __launch_bounds__(256) void k_msg_combine(const void* __restrict__ proj, int pdt,
                                                     const int32_t* __restrict__ tok_d,
                                                     const int32_t* __restrict__ d_tokrow, int N,
                                                     int S, int H, void* __restrict__ msg,
                                                     int mdt) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= N) return;
  const int64_t e = static_cast<int64_t>(t) * S + lane;
  const int my_row = (lane < S && tok_d[e] >= 0) ? d_tokrow[e] : -1;
  const int n = __popcll(__ballot(my_row >= 0));  // entries are packed first (ascending destination)
  float acc[CPL][8];
#pragma unroll
  for (int c = 0; c < CPL; ++c)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[c][i] = 0.f;
  for (int j = 0; j < n; ++j) {
    const int64_t row = __shfl(my_row, j);
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int col = (lane + 64 * c) * 8;
      if (col < H) {
        float v[8];
        load8(proj, pdt, row * H + col, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[c][i] += v[i];
      }
    }
  }
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int col = (lane + 64 * c) * 8;
    if (col < H) store8(msg, mdt, static_cast<int64_t>(t) * H + col, acc[c]);
  }
}

template <int CPL>
__global__ __launch_bounds__(256) void k_epilogue(
    const void* __restrict__ h, const void* __restrict__ x0, int adt, const void* __restrict__ y,
    int ydt, const int32_t* __restrict__ tok_e, const float* __restrict__ tok_ew,
    const int32_t* __restrict__ e_tokrow, int N, int K, int H, float alpha, float beta,
    const float* __restrict__ ln_w, const float* __restrict__ ln_b, float eps,
    void* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= N) return;
  // lane j (< K): the token's j-th expert row if its weight is > 0 (rows
  // with weight <= 0 are dropped from the FFN, sparse_experts.py:56)
  const int64_t e = static_cast<int64_t>(t) * K + lane;
  int my_row = -1;
  if (lane < K && tok_e[e] >= 0 && tok_ew[e] > 0.f) my_row = e_tokrow[e];
  uint64_t live = __ballot(my_row >= 0);
  float hv[CPL][8], xv[CPL][8], d[CPL][8];
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int col = (lane + 64 * c) * 8;
#pragma unroll
    for (int i = 0; i < 8; ++i) d[c][i] = 0.f;
    if (col < H) {
      load8(h, adt, static_cast<int64_t>(t) * H + col, hv[c]);
      load8(x0, adt, static_cast<int64_t>(t) * H + col, xv[c]);
    }
  }
  while (live) {  // ascending expert order (tok_e is ascending)
    const int j = __ffsll(static_cast<unsigned long long>(live)) - 1;
    live &= live - 1;
    const int64_t row = __shfl(my_row, j);
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int col = (lane + 64 * c) * 8;
      if (col < H) {
        float v[8];
        load8(y, ydt, row * H + col, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) d[c][i] += v[i];
      }
    }
  }
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
  for (int c = 0; c < CPL; ++c) {
    const int col = (lane + 64 * c) * 8;
    if (col < H) {
      float o[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        o[i] = (d[c][i] - mean) * rstd * (ln_w ? ln_w[col + i] : 1.f) + (ln_b ? ln_b[col + i] : 0.f);
      store8(out, adt, static_cast<int64_t>(t) * H + col, o);
    }
  }
}

template <int CPL>
__global__ __launch_bounds__(256) void k_delta_combine(const void* __restrict__ y, int ydt,
                                                       const int32_t* __restrict__ tok_row, int N,
                                                       int K, int H, void* __restrict__ out,
                                                       int odt) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= N) return;
  float d[CPL][8];
#pragma unroll
  for (int c = 0; c < CPL; ++c)
#pragma unroll
    for (int i = 0; i < 8; ++i) d[c][i] = 0.f;
  for (int j = 0; j < K; ++j) {
    const int row = tok_row[static_cast<int64_t>(t) * K + j];
    if (row < 0) continue;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int col = (lane + 64 * c) * 8;
      if (col < H) {
        float v[8];
        load8(y, ydt, static_cast<int64_t>(row) * H + col, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) d[c][i] += v[i];
      }
    }
  }
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int col = (lane + 64 * c) * 8;
    if (col < H) store8(out, odt, static_cast<int64_t>(t) * H + col, d[c]);
  }
}

namespace {
template <typename F>
int by_cpl(int H, F&& f) {
  if (H <= 0 || H % 8) return SMOE_EINVAL;
  if (H <= 512) return f(std::integral_constant<int, 1>{});
  if (H <= 1024) return f(std::integral_constant<int, 2>{});
  if (H <= 2048) return f(std::integral_constant<int, 4>{});
  if (H <= 4096) return f(std::integral_constant<int, 8>{});
  return SMOE_EINVAL;
}
int last_rc() { return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP; }
}  // namespace

int launch_msg_combine(const void* proj, int pdt, const int32_t* tok_d, const int32_t* d_tokrow,
                       int N, int S, int H, void* msg, int mdt, hipStream_t s) {
  if (N <= 0) return SMOE_OK;
  return by_cpl(H, [&](auto cpl) {
    hipLaunchKernelGGL((k_msg_combine<decltype(cpl)::value>), dim3((N + 3) / 4), dim3(256), 0, s,
                       proj, pdt, tok_d, d_tokrow, N, S, H, msg, mdt);
    return last_rc();
  });
}

int launch_epilogue(const void* h, const void* x0, int adt, const void* y, int ydt,
                    const int32_t* tok_e, const float* tok_ew, const int32_t* e_tokrow, int N,
                    int K, int H, float alpha, float beta, const float* ln_w, const float* ln_b,
                    float eps, void* out, hipStream_t s) {
  if (N <= 0) return SMOE_OK;
  return by_cpl(H, [&](auto cpl) {
    hipLaunchKernelGGL((k_epilogue<decltype(cpl)::value>), dim3((N + 3) / 4), dim3(256), 0, s, h,
                       x0, adt, y, ydt, tok_e, tok_ew, e_tokrow, N, K, H, alpha, beta, ln_w, ln_b,
                       eps, out);
    return last_rc();
  });
}

int launch_delta_combine(const void* y, int ydt, const int32_t* tok_row, int N, int K, int H,
                         void* out, int odt, hipStream_t s) {
  if (N <= 0) return SMOE_OK;
  return by_cpl(H, [&](auto cpl) {
    hipLaunchKernelGGL((k_delta_combine<decltype(cpl)::value>), dim3((N + 3) / 4), dim3(256), 0,
                       s, y, ydt, tok_row, N, K, H, out, odt);
    return last_rc();
  });
}

}  // namespace smoe
