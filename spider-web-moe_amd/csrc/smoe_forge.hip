// Kernels behind the Forge surfaces (spider_infer/forge/*): the select
// top-k modes and the weighted combine of per-expert output rows.
#include <climits>

#include "smoe_common.hpp"
#include "smoe_internal.hpp"
#include "smoe_rows.hpp"

namespace smoe {
namespace {

constexpr int kSelBig = 1 << 20;

// One segment of SEG lanes per token (lane e: logit e).  MODE 0: the
// router (model.py:255-258): p = softmax(logits) in fp32, top-k on p (ties
// to the lower index), weights p / max(sum, 1e-9).  MODE 1:
// ForgeSelect.route (forge/select/api.py:28-40): top-k on the logits
// (descending, ties to the lower index), weights = softmax over those k
// values (summed in slot order).
template <int SEG, int MODE>
__global__ __launch_bounds__(256) void k_select_topk(const float* __restrict__ logits, int N,
                                                     int E, int K, float* __restrict__ top_w,
                                                     int32_t* __restrict__ top_idx) {
  constexpr int TPW = 64 / SEG;
  const int lane = threadIdx.x & 63;
  const int t0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * TPW;
  if (t0 >= N) return;  // wave-uniform
  const int e = lane & (SEG - 1);
  const int t = t0 + lane / SEG;
  const bool ok = t < N;
  const bool in = e < E;
  float v = logits[static_cast<int64_t>(ok ? t : N - 1) * E + (in ? e : E - 1)];
  v = in ? v : -INFINITY;
  float key = v, mx = 0.f, sum = 1.f;
  if (MODE == 0) {
    mx = seg_max<SEG>(v);
    sum = seg_sum<SEG>(in ? expf(v - mx) : 0.f);
  }
  bool sel = false;
  float first = 0.f, acc = 0.f, slot_v = 0.f;
  int slot_i = 0;
#pragma unroll 1
  for (int j = 0; j < K; ++j) {
    float cv = (in && !sel) ? key : -INFINITY;
    int ci = (in && !sel) ? e : kSelBig;
    seg_argmax<SEG>(cv, ci);
    sel = sel || e == ci;
    first = j == 0 ? cv : first;
    // MODE 0: p of the pick; MODE 1: exp of the pick against the largest
    const float pj = MODE == 0 ? expf(cv - mx) / sum : expf(cv - first);
    slot_v = e == j ? pj : slot_v;
    slot_i = e == j ? ci : slot_i;
    acc += pj;
  }
  const float denom = MODE == 0 ? fmaxf(acc, 1e-9f) : acc;
  if (ok && e < K) {
    top_w[static_cast<int64_t>(t) * K + e] = slot_v / denom;
    top_idx[static_cast<int64_t>(t) * K + e] = slot_i;
  }
}

// k_select_topk for 64 < E <= 64 V: one wave per token, lane l holding
// logits l, l + 64, .. (K <= 64 slots, lane j writes slot j).
template <int V, int MODE>
__global__ __launch_bounds__(256) void k_select_topk_w(const float* __restrict__ logits, int N,
                                                       int E, int K, float* __restrict__ top_w,
                                                       int32_t* __restrict__ top_idx) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= N) return;  // wave-uniform
  float x[V];
  bool in[V], sel[V];
  float mx = -INFINITY;
#pragma unroll
  for (int v = 0; v < V; ++v) {
    in[v] = lane + 64 * v < E;
    x[v] = in[v] ? logits[static_cast<int64_t>(t) * E + lane + 64 * v] : -INFINITY;
    mx = fmaxf(mx, x[v]);
    sel[v] = false;
  }
  float sum = 1.f;
  if (MODE == 0) {
    mx = seg_max<64>(mx);
    float part = 0.f;
#pragma unroll
    for (int v = 0; v < V; ++v) part += in[v] ? expf(x[v] - mx) : 0.f;
    sum = seg_sum<64>(part);
  }
  float first = 0.f, acc = 0.f, slot_v = 0.f;
  int slot_i = 0;
#pragma unroll 1
  for (int j = 0; j < K; ++j) {
    bool cand[V];
#pragma unroll
    for (int v = 0; v < V; ++v) cand[v] = in[v] && !sel[v];
    float cv;
    int ci;
    wide_argmax<V>(x, cand, cv, ci);
#pragma unroll
    for (int v = 0; v < V; ++v) sel[v] = sel[v] || (lane + 64 * v == ci);
    first = j == 0 ? cv : first;
    const float pj = MODE == 0 ? expf(cv - mx) / sum : expf(cv - first);
    slot_v = lane == j ? pj : slot_v;
    slot_i = lane == j ? ci : slot_i;
    acc += pj;
  }
  const float denom = MODE == 0 ? fmaxf(acc, 1e-9f) : acc;
  if (lane < K) {
    top_w[static_cast<int64_t>(t) * K + lane] = slot_v / denom;
    top_idx[static_cast<int64_t>(t) * K + lane] = slot_i;
  }
}

// out[t] = sum over the token's rows (tok_row [N, K], -1 = none) in
// ascending row order — rows are grouped by expert, so this is ascending
// expert order, the order of the per-expert scatter-adds of
// forge/ep/dispatch.py:127-134 — of y[row] * row_w[row], with that code's
// arithmetic: the weight cast to y's dtype, each product rounded to y's
// dtype and each partial sum to out's dtype.  One wave per token; lane j
// holds slot j; each step takes the smallest row left.
template <int CPL, int YDT, int ODT>
__global__ __launch_bounds__(256) void k_combine_rows(const void* __restrict__ y,
                                                      const float* __restrict__ row_w,
                                                      const int32_t* __restrict__ tok_row, int N,
                                                      int K, int H, void* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= N) return;
  const int r = tok_row[static_cast<int64_t>(t) * K + (lane < K ? lane : K - 1)];
  const int my_row = lane < K ? r : -1;
  int left = my_row >= 0 ? my_row : INT_MAX;
  float acc[CPL][8];
#pragma unroll
  for (int c = 0; c < CPL; ++c)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[c][i] = 0.f;
  while (__ballot(left != INT_MAX)) {
    int row = left;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) row = min(row, __shfl_xor(row, m));
    if (left == row) left = INT_MAX;  // rows are distinct: one lane takes it
    float w = row_w ? row_w[row] : 1.f;
    if (YDT == SMOE_BF16) w = bf2f(f2bf(w));
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int col = (lane + 64 * c) * 8;
      float v[8];
      load8<YDT>(y, static_cast<int64_t>(row) * H + (col < H ? col : 0), v);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float p = mul_rn(v[i], w);
        if (YDT == SMOE_BF16) p = bf2f(f2bf(p));
        float s = add_rn(acc[c][i], p);
        if (ODT == SMOE_BF16) s = bf2f(f2bf(s));
        acc[c][i] = s;
      }
    }
  }
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int col = (lane + 64 * c) * 8;
    if (col < H) store8<ODT>(out, static_cast<int64_t>(t) * H + col, acc[c]);
  }
}

// Routed expert ids -> slab slots (Dobu residency); 4 ids per thread.
__global__ __launch_bounds__(256) void k_remap_ids(const int32_t* __restrict__ ids, int64_t n,
                                                   const int32_t* __restrict__ map, int E,
                                                   int32_t* __restrict__ out) {
  const int64_t i0 = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int64_t i = i0 + u;
    if (i < n) {
      const int e = ids[i];
      out[i] = (e >= 0 && e < E) ? map[e] : -1;
    }
  }
}

int rc() { return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP; }

}  // namespace

int launch_select_topk(const float* logits, int N, int E, int K, int mode, float* top_w,
                       int32_t* top_idx, hipStream_t s) {
  if (E < 1 || E > 256 || K < 1 || K > E || K > 64 || (mode != 0 && mode != 1)) return SMOE_EINVAL;
  if (N <= 0) return SMOE_OK;
  if (E > 64) {
    const dim3 grid((N + 3) / 4), block(256);
#define SMOE_SELW(V_)                                                                          \
  do {                                                                                         \
    if (mode == 0)                                                                             \
      hipLaunchKernelGGL((k_select_topk_w<V_, 0>), grid, block, 0, s, logits, N, E, K, top_w, top_idx); \
    else                                                                                       \
      hipLaunchKernelGGL((k_select_topk_w<V_, 1>), grid, block, 0, s, logits, N, E, K, top_w, top_idx); \
  } while (0)
    if (E <= 128) SMOE_SELW(2);
    else if (E <= 192) SMOE_SELW(3);
    else SMOE_SELW(4);
#undef SMOE_SELW
    return rc();
  }
  const int seg = E <= 16 ? 16 : (E <= 32 ? 32 : 64), per = 4 * (64 / seg);
  const dim3 grid((N + per - 1) / per), block(256);
#define SMOE_SEL(SG)                                                                           \
  do {                                                                                         \
    if (mode == 0)                                                                             \
      hipLaunchKernelGGL((k_select_topk<SG, 0>), grid, block, 0, s, logits, N, E, K, top_w, top_idx); \
    else                                                                                       \
      hipLaunchKernelGGL((k_select_topk<SG, 1>), grid, block, 0, s, logits, N, E, K, top_w, top_idx); \
  } while (0)
  if (seg == 16) SMOE_SEL(16);
  else if (seg == 32) SMOE_SEL(32);
  else SMOE_SEL(64);
#undef SMOE_SEL
  return rc();
}

int launch_remap_ids(const int32_t* ids, int64_t n, const int32_t* map, int E, int32_t* out,
                     hipStream_t s) {
  if (n <= 0) return SMOE_OK;
  const int64_t blocks = (n + 1023) / 1024;
  hipLaunchKernelGGL(k_remap_ids, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, ids, n, map,
                     E, out);
  return rc();
}

int launch_combine_rows(const void* y, int ydt, const float* row_w, const int32_t* tok_row,
                        int N, int K, int H, void* out, int odt, hipStream_t s) {
  if (K < 1 || K > 64) return SMOE_EINVAL;
  if (N <= 0) return SMOE_OK;
  return by_cpl(H, [&](auto cpl) {
    return by_dt(ydt, [&](auto yd) {
      return by_dt(odt, [&](auto od) {
        hipLaunchKernelGGL((k_combine_rows<decltype(cpl)::value, decltype(yd)::value,
                                           decltype(od)::value>),
                           dim3((N + 3) / 4), dim3(256), 0, s, y, row_w, tok_row, N, K, H, out);
        return rc();
      });
    });
  });
}

}  // namespace smoe
