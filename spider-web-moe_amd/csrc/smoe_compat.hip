// The reference's device ABI (include/spider_cuda.h) over gfx950 kernels:
// the fp32 "native" loop of the torch-free path, with the reference's
// layouts and semantics (see the header).  Each sum runs in a fixed order
// and the products / sums the reference's scalar library forms in single or
// double precision are formed the same way here (explicit _rn operations
// where the compiler would otherwise contract a multiply-add), so the
// outputs follow the scalar library to the last bit or two.
#include <math.h>

#include <climits>
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
    const int e1 = min(rp[src + 1], nnz);  // a malformed CSR never reads past its arrays
    for (int e = max(rp[src], 0); e < e1; ++e)
      acc = fadd(acc, fmul(fmul(ew[static_cast<int64_t>(loop) * nnz + e], r), hv));
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

// ------------------------------------------------------ wide arg-max ----
// LDS written by some lanes of a wave, then read by others of the same wave.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// The scalar library's iterative arg-max (scalar.cpp:18-27,
// scalar_phase1_2.cpp:19-30) over one row of up to 64 * VPL values, one
// wave per row: lane l holds index l + 64 c in v[c].  Pick m is the first
// (lowest-index) largest value above `floor` among the indices not picked
// yet — the scalar loop's strict "greater than the best so far" started at
// floor (-1 for router probabilities, -inf for edge logits).  A pick with
// no candidate left is (-1, floor), as there.  Lane 0 writes the picks.
template <int VPL>
__device__ __forceinline__ void wave_pick(const float (&v)[VPL], int n, int picks, float floor,
                                          int32_t* __restrict__ out_i,
                                          float* __restrict__ out_v) {
  const int lane = threadIdx.x & 63;
  unsigned used = 0;
#pragma unroll 1
  for (int m = 0; m < picks; ++m) {
    float bv = -INFINITY;
    int bi = kRefBig;
#pragma unroll
    for (int c = 0; c < VPL; ++c) {
      const int e = lane + 64 * c;
      if (e < n && !((used >> c) & 1u) && v[c] > floor && v[c] > bv) {
        bv = v[c];
        bi = e;
      }
    }
    seg_argmax<64>(bv, bi);
    if (bi != kRefBig && (bi & 63) == lane) used |= 1u << (bi >> 6);
    if (lane == 0) {
      out_i[m] = bi == kRefBig ? -1 : bi;
      out_v[m] = bi == kRefBig ? floor : bv;
    }
  }
}

// Router rows of 64 < E <= 64 * VPL experts (the <= 64 form is
// k_ref_router): p = exp(l + b - max) / sum, K picks of p, weights
// renormalised by max(sum of picks in pick order, 1e-20).  One wave per
// row; the picks go through LDS.
template <int VPL>
__global__ __launch_bounds__(256) void k_ref_router_wide(const float* __restrict__ logits,
                                                         const float* __restrict__ bias, int B,
                                                         int E, int K, float* __restrict__ w,
                                                         int32_t* __restrict__ idx) {
  __shared__ float sv[4][64 * VPL];
  __shared__ int32_t si[4][64 * VPL];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int b = blockIdx.x * 4 + wave;
  if (b >= B) return;  // wave-uniform; no block barrier below
  float v[VPL];
  float mx = -INFINITY;
#pragma unroll
  for (int c = 0; c < VPL; ++c) {
    const int e = lane + 64 * c;
    v[c] = e < E ? fadd(logits[static_cast<int64_t>(b) * E + e], bias[e]) : -INFINITY;
    mx = fmaxf(mx, v[c]);
  }
  mx = seg_max<64>(mx);
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < VPL; ++c) s += lane + 64 * c < E ? expf(v[c] - mx) : 0.f;
  s = seg_sum<64>(s);
#pragma unroll
  for (int c = 0; c < VPL; ++c) v[c] = lane + 64 * c < E ? expf(v[c] - mx) / s : -INFINITY;
  wave_pick<VPL>(v, E, K, -1.f, si[wave], sv[wave]);
  wave_lds_sync();
  float tot = 0.f;
  for (int m = 0; m < K; ++m) tot = fadd(tot, sv[wave][m]);
  const float d = fmaxf(tot, 1e-20f);
  for (int m = lane; m < K; m += 64) {
    w[static_cast<int64_t>(b) * K + m] = sv[wave][m] / d;
    idx[static_cast<int64_t>(b) * K + m] = si[wave][m];
  }
}

// --------------------------------------------------------- edge top-m ----
// spider_edge_topk_f32 (scalar_phase1_2.cpp:11-47): for each (b, src) row
// of E edge logits, M picks of the iterative arg-max, then a softmax over
// the picked values (max, exp, sum in pick order, / max(sum, 1e-20)).  One
// wave per row.
template <int VPL>
__global__ __launch_bounds__(256) void k_ref_edge_topk(const float* __restrict__ logits, int rows,
                                                       int E, int M, int32_t* __restrict__ eidx,
                                                       float* __restrict__ ew) {
  __shared__ float sv[4][64 * VPL];
  __shared__ int32_t si[4][64 * VPL];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = blockIdx.x * 4 + wave;
  if (r >= rows) return;  // wave-uniform
  float v[VPL];
#pragma unroll
  for (int c = 0; c < VPL; ++c) {
    const int e = lane + 64 * c;
    v[c] = e < E ? logits[static_cast<int64_t>(r) * E + e] : -INFINITY;
  }
  wave_pick<VPL>(v, E, M, -INFINITY, si[wave], sv[wave]);
  wave_lds_sync();
  float mx = -INFINITY;
  for (int m = 0; m < M; ++m) mx = fmaxf(mx, sv[wave][m]);
  for (int m = lane; m < M; m += 64) sv[wave][m] = expf(sv[wave][m] - mx);
  wave_lds_sync();
  float sum = 0.f;
  for (int m = 0; m < M; ++m) sum = fadd(sum, sv[wave][m]);
  const float d = fmaxf(sum, 1e-20f);
  for (int m = lane; m < M; m += 64) {
    eidx[static_cast<int64_t>(r) * M + m] = si[wave][m];
    ew[static_cast<int64_t>(r) * M + m] = sv[wave][m] / d;
  }
}

// ------------------------------------------------ graph v2 / dynamic ----
// messages[b, j] = sum over the row's valid sources (slot order) and their
// edges (CSR order, or the M picks of the (b, src) row) of scale *
// projected[b, dst, j] — scalar_phase1_1.cpp:34-60 (scale = the loop's
// edge weight) and scalar_phase1_2.cpp:49-72 (scale = the picked edge
// weight).  Sources or destinations outside [0, E) are skipped (the host
// entry points reject them first, as the scalar library does).
__global__ __launch_bounds__(256) void k_ref_graph_proj(
    const float* __restrict__ proj, int B, int H, int E, int K, const int32_t* __restrict__ rp,
    const int32_t* __restrict__ ci, int nnz, const float* __restrict__ ew, int M,
    const int32_t* __restrict__ eidx, const int32_t* __restrict__ assign,
    float* __restrict__ out) {
  const int b = blockIdx.y;
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= H) return;
  float acc = 0.f;
  for (int k = 0; k < K; ++k) {
    const int src = assign[b * K + k];
    if (src < 0 || src >= E) continue;
    // static CSR (rp != nullptr) or the row's dynamic picks
    // (a malformed CSR never reads past its arrays)
    const int64_t e0 = rp ? max(rp[src], 0) : (static_cast<int64_t>(b) * E + src) * M;
    const int64_t e1 = rp ? min(rp[src + 1], nnz) : e0 + M;
    for (int64_t e = e0; e < e1; ++e) {
      const int dst = rp ? ci[e] : eidx[e];
      if (dst < 0 || dst >= E) continue;
      acc = fadd(acc, fmul(ew[e], proj[(static_cast<int64_t>(b) * E + dst) * H + j]));
    }
  }
  out[static_cast<int64_t>(b) * H + j] = acc;
}

// -------------------------------------------- double-accumulated GEMM ----
// out[b, o] = float(sum over i ascending of double(A[b, i]) * double(W[o, i]))
// with A[b] = [x[b, 0:H], x2[0:n_in - H]] and W row-major [O, n_in]: the
// edge projection (W_edge [E, H, H] as [E*H, H], scalar_phase1_1.cpp:17-32)
// and the edge generator (W_gen [E*E, H + D] over [h; loop_emb],
// scalar_phase1_3.cpp:14-42).  Products of two floats are exact in double,
// so each step rounds only the sum, in the scalar loop's order.  Tiles of
// 64 outputs x 16 rows, 32-wide k steps through LDS; thread: one output of
// 4 rows.
__global__ __launch_bounds__(256) void k_ref_gemm_f64(const float* __restrict__ x, int H,
                                                      const float* __restrict__ x2, int n_in,
                                                      const float* __restrict__ W, int O, int B,
                                                      float* __restrict__ out) {
  __shared__ float sW[32][65];
  __shared__ float sA[16][33];
  const int tid = threadIdx.x, ol = tid & 63, bq = tid >> 6;
  const int o0 = blockIdx.x * 64, b0 = blockIdx.y * 16;
  double acc[4] = {0.0, 0.0, 0.0, 0.0};
  for (int i0 = 0; i0 < n_in; i0 += 32) {
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int id = tid + 256 * r, row = id >> 5, col = id & 31;
      const int o = o0 + row, i = i0 + col;
      sW[col][row] = (o < O && i < n_in) ? W[static_cast<int64_t>(o) * n_in + i] : 0.f;
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int id = tid + 256 * r, row = id >> 5, col = id & 31;
      const int b = b0 + row, i = i0 + col;
      float a = 0.f;
      if (b < B && i < n_in) a = i < H ? x[static_cast<int64_t>(b) * H + i] : x2[i - H];
      sA[row][col] = a;
    }
    __syncthreads();
    const int iend = min(32, n_in - i0);
    for (int ii = 0; ii < iend; ++ii) {
      const double wv = static_cast<double>(sW[ii][ol]);
#pragma unroll
      for (int r = 0; r < 4; ++r)
        acc[r] = add_rn(acc[r], mul_rn(static_cast<double>(sA[bq * 4 + r][ii]), wv));
    }
    __syncthreads();
  }
  const int o = o0 + ol;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int b = b0 + bq * 4 + r;
    if (b < B && o < O) out[static_cast<int64_t>(b) * O + o] = static_cast<float>(acc[r]);
  }
}

// ---------------------------------------------------------------- launch ----
int rc_last() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : static_cast<int>(e);
}

int seg_for(int E) { return E <= 16 ? 16 : (E <= 32 ? 32 : 64); }

int launch_router(const float* logits, const float* bias, int B, int E, int K, float* w,
                  int32_t* idx, hipStream_t s) {
  if (E > 64) {  // one wave per row, up to 4 experts per lane
    const dim3 grid((B + 3) / 4), block(256);
    if (E <= 128) hipLaunchKernelGGL(k_ref_router_wide<2>, grid, block, 0, s, logits, bias, B, E, K, w, idx);
    else hipLaunchKernelGGL(k_ref_router_wide<4>, grid, block, 0, s, logits, bias, B, E, K, w, idx);
    return rc_last();
  }
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

int launch_edge_topk(const float* logits, int rows, int E, int M, int32_t* eidx, float* ew,
                     hipStream_t s) {
  const dim3 grid((rows + 3) / 4), block(256);
  if (E <= 64) hipLaunchKernelGGL(k_ref_edge_topk<1>, grid, block, 0, s, logits, rows, E, M, eidx, ew);
  else if (E <= 128) hipLaunchKernelGGL(k_ref_edge_topk<2>, grid, block, 0, s, logits, rows, E, M, eidx, ew);
  else hipLaunchKernelGGL(k_ref_edge_topk<4>, grid, block, 0, s, logits, rows, E, M, eidx, ew);
  return rc_last();
}

int launch_gemm_f64(const float* x, int H, const float* x2, int n_in, const float* W, int O, int B,
                    float* out, hipStream_t s) {
  hipLaunchKernelGGL(k_ref_gemm_f64, dim3((O + 63) / 64, (B + 15) / 16), dim3(256), 0, s, x, H, x2,
                     n_in, W, O, B, out);
  return rc_last();
}

}  // namespace

// The loop step's pieces for the host entry points (smoe_host_abi.hip).
int ref_logits_router(const float* h, const float* router_w, const float* bias_row, int B, int H,
                      int E, int K, float* w, int32_t* idx, hipStream_t s) {
  if (E > 64) return 1;
  hipLaunchKernelGGL(k_ref_logits_router, dim3(B), dim3(64), 0, s, h, router_w, bias_row, B, H, E,
                     K, w, idx);
  return rc_last();
}

int ref_copy_f32(const float* src, float* dst, int64_t n, hipStream_t s) {
  if (n <= 0) return 0;
  hipLaunchKernelGGL(k_ref_copy_f32, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s,
                     src, dst, n);
  return rc_last();
}

}  // namespace smoe

using namespace smoe;

extern "C" {

SPIDER_CUDA_API int spider_cuda_router_f32(const float* logits, const float* loop_bias, int B,
                                           int E, int K, int loop_idx, float* out_w,
                                           int32_t* out_idx, void* stream) {
  if (!logits || !loop_bias || !out_w || !out_idx || B <= 0 || E <= 0 || E > 256 || K <= 0 ||
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

SPIDER_CUDA_API int spider_cuda_edge_project_f32(const float* h, int B, int H, int E,
                                                 const float* W_edge, float* out_proj,
                                                 void* stream) {
  if (!h || !W_edge || !out_proj || B <= 0 || H <= 0 || E <= 0 ||
      static_cast<int64_t>(E) * H > INT32_MAX)
    return 1;
  return launch_gemm_f64(h, H, nullptr, H, W_edge, E * H, B, out_proj,
                         static_cast<hipStream_t>(stream));
}

SPIDER_CUDA_API int spider_cuda_graph_message_passing_v2_f32(
    const float* projected, int B, int H, int E, int K, const int32_t* row_ptr,
    const int32_t* col_idx, const float* edge_w, int nnz, int loop_idx, const int32_t* assign,
    float* messages, void* stream) {
  if (!projected || !row_ptr || !col_idx || !edge_w || !assign || !messages || B <= 0 || H <= 0 ||
      E <= 0 || K <= 0 || nnz < 0 || loop_idx < 0)
    return 1;
  hipLaunchKernelGGL(k_ref_graph_proj, dim3((H + 255) / 256, B), dim3(256), 0,
                     static_cast<hipStream_t>(stream), projected, B, H, E, K, row_ptr, col_idx,
                     nnz, edge_w + static_cast<int64_t>(loop_idx) * nnz, 0, nullptr, assign,
                     messages);
  return rc_last();
}

SPIDER_CUDA_API int spider_cuda_edge_topk_f32(const float* edge_logits, int B, int E, int M,
                                              int32_t* edge_idx, float* edge_w, void* stream) {
  if (!edge_logits || !edge_idx || !edge_w || B <= 0 || E <= 0 || E > 256 || M <= 0 || M > E ||
      static_cast<int64_t>(B) * E > INT32_MAX)
    return 1;
  return launch_edge_topk(edge_logits, B * E, E, M, edge_idx, edge_w,
                          static_cast<hipStream_t>(stream));
}

SPIDER_CUDA_API int spider_cuda_graph_message_passing_dynamic_f32(
    const float* projected, int B, int H, int E, int K, int M, const int32_t* edge_idx,
    const float* edge_w, const int32_t* assign, float* messages, void* stream) {
  if (!projected || !edge_idx || !edge_w || !assign || !messages || B <= 0 || H <= 0 || E <= 0 ||
      K <= 0 || M <= 0)
    return 1;
  hipLaunchKernelGGL(k_ref_graph_proj, dim3((H + 255) / 256, B), dim3(256), 0,
                     static_cast<hipStream_t>(stream), projected, B, H, E, K, nullptr, nullptr, 0,
                     edge_w, M, edge_idx, assign, messages);
  return rc_last();
}

SPIDER_CUDA_API int spider_cuda_edge_generator_f32(const float* h, int B, int H, int E,
                                                   const float* loop_emb, int loop_emb_dim,
                                                   const float* W_gen, float* out_logits,
                                                   void* stream) {
  if (!h || !loop_emb || !W_gen || !out_logits || B <= 0 || H <= 0 || E <= 0 ||
      loop_emb_dim < 0 || static_cast<int64_t>(E) * E > INT32_MAX)
    return 1;
  return launch_gemm_f64(h, H, loop_emb, H + loop_emb_dim, W_gen, E * E, B, out_logits,
                         static_cast<hipStream_t>(stream));
}

}  // extern "C"
