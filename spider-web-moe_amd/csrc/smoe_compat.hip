// The reference's device ABI (include/spider_cuda.h) over gfx950 kernels:
// the fp32 "native" loop of the torch-free path, with the reference's
// layouts and semantics (see the header).  Each sum runs in a fixed order
// and the products / sums the reference's scalar library forms in single or
// double precision are formed the same way here (explicit _rn operations
// where the compiler would otherwise contract a multiply-add), so the
// outputs follow the scalar library to the last bit or two.
#include <math.h>

#include <type_traits>

#include "smoe_common.hpp"
#include "smoe_internal.hpp"
#include "spider_cuda.h"

namespace smoe {
namespace {

constexpr int kRefBig = 1 << 20;

__device__ __forceinline__ float fmul(float a, float b) { return mul_rn(a, b); }
__device__ __forceinline__ float fadd(float a, float b) { return add_rn(a, b); }

// ---------------------------------------------------------------- router ----
// Segment of SEG lanes per row (lane e: expert e).  p = exp(l + b - max) /
// sum; the k-th pick is the largest p not taken yet, the lowest index among
// equal p (spider_kernels.cu:8-26 takes the first strictly greater);
// weights renormalised by max(sum of picks, 1e-20).
template <int SEG>
__device__ __forceinline__ void ref_route_seg(float v, int b, bool ok, int E, int K,
                                              float* __restrict__ w, int32_t* __restrict__ idx) {
  const int lane = threadIdx.x & 63;
  const int e = lane & (SEG - 1);
  const bool in = e < E;
  v = in ? v : -INFINITY;
  const float mx = seg_max<SEG>(v);
  const float ex = in ? expf(v - mx) : 0.f;
  const float denom = seg_sum<SEG>(ex);
  const float p = ex / denom;
  bool used = false;
  float chosen = 0.f, slot_w = 0.f;
  int slot_i = 0;
#pragma unroll 1
  for (int k = 0; k < K; ++k) {
    float cv = (in && !used) ? p : -INFINITY;
    int ci = (in && !used) ? e : kRefBig;
    seg_argmax<SEG>(cv, ci);
    used = used || e == ci;
    slot_w = e == k ? cv : slot_w;
    slot_i = e == k ? ci : slot_i;
    chosen = fadd(chosen, cv);
  }
  const float d = fmaxf(chosen, 1e-20f);
  if (ok && e < K) {
    w[static_cast<int64_t>(b) * K + e] = slot_w / d;
    idx[static_cast<int64_t>(b) * K + e] = slot_i;
  }
}

template <int SEG>
__global__ __launch_bounds__(256) void k_ref_router(const float* __restrict__ logits,
                                                    const float* __restrict__ bias, int B, int E,
                                                    int K, float* __restrict__ w,
                                                    int32_t* __restrict__ idx) {
  constexpr int TPW = 64 / SEG;
  const int lane = threadIdx.x & 63;
  const int b0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * TPW;
  if (b0 >= B) return;  // wave-uniform
  const int e = lane & (SEG - 1);
  const int b = b0 + lane / SEG;
  const bool ok = b < B;
  const int ec = e < E ? e : E - 1;
  const float v = fadd(logits[static_cast<int64_t>(ok ? b : B - 1) * E + ec], bias[ec]);
  ref_route_seg<SEG>(v, b, ok, E, K, w, idx);
}

// Loop step: logits = h . router_w ([H, E]) in double (products and sums as
// scalar_phase1_1.cpp:77-84 forms them), then the router.  One wave per row.
__global__ __launch_bounds__(64) void k_ref_logits_router(const float* __restrict__ h,
                                                          const float* __restrict__ router_w,
                                                          const float* __restrict__ bias, int B,
                                                          int H, int E, int K,
                                                          float* __restrict__ w,
                                                          int32_t* __restrict__ idx) {
  const int b = blockIdx.x;
  const int e = threadIdx.x;
  const int ec = e < E ? e : E - 1;
  double acc = 0.0;
  for (int i = 0; i < H; ++i)
    acc = add_rn(acc, mul_rn(static_cast<double>(h[static_cast<int64_t>(b) * H + i]),
                                   static_cast<double>(router_w[static_cast<int64_t>(i) * E + ec])));
  const float v = fadd(static_cast<float>(acc), bias[ec]);
  ref_route_seg<64>(v, b, true, E, K, w, idx);
}

// -------------------------------------------------------------- graph v1 ----
// messages[b, j] = sum over the row's valid sources and their edges of
// (edge_w * route_w) * h[b, j], sources in slot order, edges in CSR order
// (spider_kernels.cu:28-40; the scalar form is scalar.cpp:36-53).
__global__ __launch_bounds__(256) void k_ref_graph(const float* __restrict__ h, int B, int H,
                                                   int E, int K, const int32_t* __restrict__ rp,
                                                   const float* __restrict__ ew, int nnz, int loop,
                                                   const int32_t* __restrict__ assign,
                                                   const float* __restrict__ rw,
                                                   float* __restrict__ out) {
  const int b = blockIdx.y;
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= H) return;
  const float hv = h[static_cast<int64_t>(b) * H + j];
  float acc = 0.f;
  for (int k = 0; k < K; ++k) {
    const int src = assign[b * K + k];
    if (src < 0 || src >= E) continue;
    const float r = rw[b * K + k];
    const int e1 = rp[src + 1];
    for (int e = rp[src]; e < e1; ++e)
      if (e < nnz) acc = fadd(acc, fmul(fmul(ew[static_cast<int64_t>(loop) * nnz + e], r), hv));
  }
  out[static_cast<int64_t>(b) * H + j] = acc;
}

// ------------------------------------------------------------ expert FFN ----
__device__ __forceinline__ float gelu_tanh_ref(float a) {
  const float c = fmul(0.7978845608f, fadd(a, fmul(fmul(fmul(0.044715f, a), a), a)));
  return fmul(fmul(0.5f, a), fadd(1.f, tanhf(c)));
}

// One workgroup per row b: for each slot k with a valid expert e (slot
// order), act[u] = gelu_tanh(sum_i x[i] W_up[e][i][u]) (i ascending), then
// out[j] += (route_w act[u]) W_down[e][u][j] for u ascending — the order in
// which scalar.cpp:55-73 accumulates (spider_expert_v2.cu:13-58 forms the
// same sums with atomics).  act lives in LDS, or in the caller's workspace
// [B, K, U] (act_ws).  CH: output columns per thread.
template <int CH>
__global__ __launch_bounds__(256) void k_ref_expert(const float* __restrict__ x, int H, int U,
                                                    int E, int K, const int32_t* __restrict__ ids,
                                                    const float* __restrict__ rw,
                                                    const float* __restrict__ w_up,
                                                    const float* __restrict__ w_down,
                                                    float* __restrict__ out,
                                                    float* __restrict__ act_ws) {
  extern __shared__ float sm[];
  const int b = blockIdx.x, tid = threadIdx.x;
  float* xs = sm;
  for (int i = tid; i < H; i += 256) xs[i] = x[static_cast<int64_t>(b) * H + i];
  __syncthreads();
  float acc[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) acc[c] = 0.f;
  for (int k = 0; k < K; ++k) {
    const int e = ids[b * K + k];
    if (e < 0 || e >= E) continue;  // uniform
    float* act = act_ws ? act_ws + (static_cast<int64_t>(b) * K + k) * U : sm + H;
    const float* wu = w_up + static_cast<int64_t>(e) * H * U;
    for (int u = tid; u < U; u += 256) {
      float a = 0.f;
      for (int i = 0; i < H; ++i) a = fadd(a, fmul(xs[i], wu[static_cast<int64_t>(i) * U + u]));
      act[u] = gelu_tanh_ref(a);
    }
    __syncthreads();
    const float r = rw[b * K + k];
    const float* wd = w_down + static_cast<int64_t>(e) * U * H;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int j = tid + 256 * c;
      if (j < H)
        for (int u = 0; u < U; ++u)
          acc[c] = fadd(acc[c], fmul(fmul(r, act[u]), wd[static_cast<int64_t>(u) * H + j]));
    }
    __syncthreads();  // act is rewritten by the next slot
  }
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int j = tid + 256 * c;
    if (j < H) out[static_cast<int64_t>(b) * H + j] = acc[c];
  }
}

// -------------------------------------------------------------- epilogue ----
// One workgroup per row: u = (h + alpha d) + beta x0 in fp32, mean and
// variance in double (two passes over the row; the reference runs Welford
// in double, scalar.cpp:75-92), inv = 1 / sqrt(float(m2 / H) + eps), out =
// ((u - float(mean)) inv) gamma + beta_ln.  out may alias d (in-place: every
// u is held in registers before the first store).
__device__ __forceinline__ double block_sum_d(double v, double* red) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = add_rn(v, __shfl_xor(v, o));
  if (lane == 0) red[wave] = v;
  __syncthreads();
  const double s = add_rn(add_rn(red[0], red[1]), add_rn(red[2], red[3]));
  __syncthreads();
  return s;
}

template <int CH>
__global__ __launch_bounds__(256) void k_ref_epilogue(const float* __restrict__ h,
                                                      const float* d,
                                                      const float* __restrict__ x0, int H,
                                                      float alpha, float beta,
                                                      const float* __restrict__ gamma,
                                                      const float* __restrict__ lb, float eps,
                                                      float* out) {
  __shared__ double red[4];
  const int b = blockIdx.x, tid = threadIdx.x;
  const int64_t base = static_cast<int64_t>(b) * H;
  float u[CH];
  double s = 0.0;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int j = tid + 256 * c;
    u[c] = 0.f;
    if (j < H) {
      u[c] = fadd(fadd(h[base + j], fmul(alpha, d[base + j])), fmul(beta, x0[base + j]));
      s = add_rn(s, static_cast<double>(u[c]));
    }
  }
  const double mean = block_sum_d(s, red) / static_cast<double>(H);
  double q = 0.0;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int j = tid + 256 * c;
    if (j < H) {
      const double z = static_cast<double>(u[c]) - mean;
      q = add_rn(q, mul_rn(z, z));
    }
  }
  const double m2 = block_sum_d(q, red);
  const float inv = 1.f / sqrtf(fadd(static_cast<float>(m2 / static_cast<double>(H)), eps));
  const float mf = static_cast<float>(mean);
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int j = tid + 256 * c;
    if (j < H) out[base + j] = fadd(fmul(fmul(fadd(u[c], -mf), inv), gamma[j]), lb[j]);
  }
}

// ------------------------------------------------------------------ exit ----
// One wave per row: dot in double (exact products, fixed order), z =
// float(dot), the overflow-free sigmoid of scalar.cpp:94-104, > threshold.
__global__ __launch_bounds__(64) void k_ref_exit(const float* __restrict__ h,
                                                 const float* __restrict__ proj, int H,
                                                 float threshold, uint8_t* __restrict__ mask) {
  const int b = blockIdx.x, lane = threadIdx.x;
  double acc = 0.0;
  for (int j = lane; j < H; j += 64)
    acc = add_rn(acc, mul_rn(static_cast<double>(h[static_cast<int64_t>(b) * H + j]),
                                   static_cast<double>(proj[j])));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) acc = add_rn(acc, __shfl_xor(acc, o));
  if (lane == 0) {
    const float z = static_cast<float>(acc);
    const float conf = z >= 0.f ? 1.f / (1.f + expf(-z)) : expf(z) / (1.f + expf(z));
    mask[b] = conf > threshold ? 1 : 0;
  }
}

__global__ void k_ref_zero_u8(uint8_t* __restrict__ p, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0;
}

__global__ void k_ref_copy_f32(const float* __restrict__ src, float* __restrict__ dst, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) dst[i] = src[i];
}

// ---------------------------------------------------------------- launch ----
int rc_last() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : static_cast<int>(e);
}

int seg_for(int E) { return E <= 16 ? 16 : (E <= 32 ? 32 : 64); }

int launch_router(const float* logits, const float* bias, int B, int E, int K, float* w,
                  int32_t* idx, hipStream_t s) {
  const int seg = seg_for(E), per = 4 * (64 / seg);
  const dim3 grid((B + per - 1) / per), block(256);
  if (seg == 16) hipLaunchKernelGGL(k_ref_router<16>, grid, block, 0, s, logits, bias, B, E, K, w, idx);
  else if (seg == 32) hipLaunchKernelGGL(k_ref_router<32>, grid, block, 0, s, logits, bias, B, E, K, w, idx);
  else hipLaunchKernelGGL(k_ref_router<64>, grid, block, 0, s, logits, bias, B, E, K, w, idx);
  return rc_last();
}

template <typename F>
int by_ch(int H, F&& f) {
  if (H <= 256) return f(std::integral_constant<int, 1>{});
  if (H <= 512) return f(std::integral_constant<int, 2>{});
  if (H <= 1024) return f(std::integral_constant<int, 4>{});
  if (H <= 2048) return f(std::integral_constant<int, 8>{});
  if (H <= 4096) return f(std::integral_constant<int, 16>{});
  if (H <= 8192) return f(std::integral_constant<int, 32>{});
  return 1;
}

int launch_expert(const float* x, int B, int H, int U, int E, int K, const int32_t* ids,
                  const float* rw, const float* up, const float* down, float* out, float* act_ws,
                  hipStream_t s) {
  const size_t lds = (static_cast<size_t>(H) + (act_ws ? 0 : U)) * sizeof(float);
  if (lds > 64 * 1024) return 1;
  return by_ch(H, [&](auto ch) {
    hipLaunchKernelGGL(k_ref_expert<decltype(ch)::value>, dim3(B), dim3(256), lds, s, x, H, U, E,
                       K, ids, rw, up, down, out, act_ws);
    return rc_last();
  });
}

int launch_epilogue_ref(const float* h, const float* d, const float* x0, int B, int H, float a,
                        float beta, const float* g, const float* lb, float eps, float* out,
                        hipStream_t s) {
  return by_ch(H, [&](auto ch) {
    hipLaunchKernelGGL(k_ref_epilogue<decltype(ch)::value>, dim3(B), dim3(256), 0, s, h, d, x0, H,
                       a, beta, g, lb, eps, out);
    return rc_last();
  });
}

}  // namespace
}  // namespace smoe

using namespace smoe;

extern "C" {

SPIDER_CUDA_API int spider_cuda_router_f32(const float* logits, const float* loop_bias, int B,
                                           int E, int K, int loop_idx, float* out_w,
                                           int32_t* out_idx, void* stream) {
  if (!logits || !loop_bias || !out_w || !out_idx || B <= 0 || E <= 0 || E > 64 || K <= 0 ||
      K > E || loop_idx < 0)
    return 1;
  return launch_router(logits, loop_bias + static_cast<int64_t>(loop_idx) * E, B, E, K, out_w,
                       out_idx, static_cast<hipStream_t>(stream));
}

SPIDER_CUDA_API int spider_cuda_graph_message_passing_f32(
    const float* h, int B, int H, int E, int K, const int32_t* row_ptr, const int32_t* col_idx,
    const float* edge_w, int nnz, int loop_idx, const int32_t* assign, const float* route_w,
    float* messages, void* stream) {
  if (!h || !row_ptr || !col_idx || !edge_w || !assign || !route_w || !messages || B <= 0 ||
      H <= 0 || E <= 0 || K <= 0 || nnz < 0 || loop_idx < 0)
    return 1;
  hipLaunchKernelGGL(k_ref_graph, dim3((H + 255) / 256, B), dim3(256), 0,
                     static_cast<hipStream_t>(stream), h, B, H, E, K, row_ptr, edge_w, nnz,
                     loop_idx, assign, route_w, messages);
  return rc_last();
}

SPIDER_CUDA_API int spider_cuda_expert_grouped_gemm_f32(const float* x, int B, int H, int U,
                                                        int E, int K, const int32_t* assign,
                                                        const float* route_w, const float* W_up,
                                                        const float* W_down, float* out,
                                                        void* stream) {
  if (!x || !assign || !route_w || !W_up || !W_down || !out || B <= 0 || H <= 0 || U <= 0 ||
      E <= 0 || K <= 0 || H > 8192)
    return 1;
  return launch_expert(x, B, H, U, E, K, assign, route_w, W_up, W_down, out, nullptr,
                       static_cast<hipStream_t>(stream));
}

SPIDER_CUDA_API size_t spider_cuda_expert_workspace_bytes(int B, int K, int U) {
  if (B <= 0 || K <= 0 || U <= 0) return 0;
  return static_cast<size_t>(B) * K * U * sizeof(float);
}

SPIDER_CUDA_API int spider_cuda_expert_grouped_gemm_v2_f32(
    const float* x, int B, int H, int U, int E, int K, const int32_t* assign,
    const float* route_w, const float* W_up, const float* W_down, float* out, float* workspace,
    void* stream) {
  if (!x || !assign || !route_w || !W_up || !W_down || !out || !workspace || B <= 0 || H <= 0 ||
      U <= 0 || E <= 0 || K <= 0 || H > 8192)
    return 1;
  return launch_expert(x, B, H, U, E, K, assign, route_w, W_up, W_down, out, workspace,
                       static_cast<hipStream_t>(stream));
}

SPIDER_CUDA_API int spider_cuda_loop_epilogue_f32(const float* h, const float* d,
                                                  const float* x0, int B, int H, float alpha,
                                                  float beta, const float* gamma,
                                                  const float* beta_ln, float eps, float* out,
                                                  void* stream) {
  if (!h || !d || !x0 || !gamma || !beta_ln || !out || B <= 0 || H <= 0 || H > 8192 ||
      !(eps > 0.f))
    return 1;
  return launch_epilogue_ref(h, d, x0, B, H, alpha, beta, gamma, beta_ln, eps, out,
                             static_cast<hipStream_t>(stream));
}

SPIDER_CUDA_API int spider_cuda_early_exit_f32(const float* h, const float* proj, int B, int H,
                                               float threshold, uint8_t* mask, void* stream) {
  if (!h || !proj || !mask || B <= 0 || H <= 0) return 1;
  hipLaunchKernelGGL(k_ref_exit, dim3(B), dim3(64), 0, static_cast<hipStream_t>(stream), h, proj,
                     H, threshold, mask);
  return rc_last();
}

SPIDER_CUDA_API int spider_cuda_moe_loop_step_f32(
    const float* h, const float* x0, int B, int H, int E, int K, int U, int loop_idx,
    const float* router_w, const float* loop_bias, const int32_t* row_ptr,
    const int32_t* col_idx, const float* edge_w, int nnz, const float* W_up,
    const float* W_down, const float* ln_weight, const float* ln_bias, float alpha, float beta,
    float eps, const float* exit_proj, float exit_threshold, float* h_next, uint8_t* exit_mask,
    int32_t* tmp_assign, float* tmp_route, float* tmp_messages, void* stream) {
  if (!h || !x0 || !router_w || !loop_bias || !W_up || !W_down || !ln_weight || !ln_bias ||
      !h_next || !tmp_assign || !tmp_route || !tmp_messages || B <= 0 || H <= 0 || H > 8192 ||
      E <= 0 || E > 64 || K <= 0 || K > E || U <= 0 || loop_idx < 0 || !(eps > 0.f) ||
      h_next == h || h_next == x0)
    return 1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(k_ref_logits_router, dim3(B), dim3(64), 0, s, h, router_w,
                     loop_bias + static_cast<int64_t>(loop_idx) * E, B, H, E, K, tmp_route,
                     tmp_assign);
  int rc = rc_last();
  if (rc) return rc;
  if (row_ptr && col_idx && edge_w && nnz >= 0) {
    hipLaunchKernelGGL(k_ref_graph, dim3((H + 255) / 256, B), dim3(256), 0, s, h, B, H, E, K,
                       row_ptr, edge_w, nnz, loop_idx, tmp_assign, tmp_route, tmp_messages);
  } else {
    const int64_t n = static_cast<int64_t>(B) * H;
    hipLaunchKernelGGL(k_ref_copy_f32, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                       s, h, tmp_messages, n);
  }
  rc = rc_last();
  if (rc) return rc;
  // the expert delta goes to h_next, which the epilogue then overwrites in place
  rc = launch_expert(tmp_messages, B, H, U, E, K, tmp_assign, tmp_route, W_up, W_down, h_next,
                     nullptr, s);
  if (rc) return rc;
  rc = launch_epilogue_ref(h, h_next, x0, B, H, alpha, beta, ln_weight, ln_bias, eps, h_next, s);
  if (rc) return rc;
  if (exit_mask && exit_proj) {
    hipLaunchKernelGGL(k_ref_exit, dim3(B), dim3(64), 0, s, h_next, exit_proj, H, exit_threshold,
                       exit_mask);
  } else if (exit_mask) {
    hipLaunchKernelGGL(k_ref_zero_u8, dim3((B + 255) / 256), dim3(256), 0, s, exit_mask, B);
  }
  return rc_last();
}

}  // extern "C"
