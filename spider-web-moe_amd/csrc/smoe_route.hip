// Routing of the Spider-MoE block: router top-k, edge generator top-m with
// per-token destination coefficients, and the stable dispatch plan.
//
// Router (model.py:255-258): logits (fp32, loop bias added by the logits
// GEMM) -> softmax -> top-k -> renorm by max(sum, 1e-9).  One segment of
// SEG = 16 / 32 / 64 lanes per token (the smallest that holds E <= 64; a wave
// holds 64 / SEG tokens), lane e of the segment holds expert e; selection is
// on the logits (softmax is monotonic), ties to the lowest index.
//
// Edges (model.py:261-288): for each of the token's router-selected sources
// s, top-m over the raw edge logits g[s, :] and an fp32 softmax over the m
// values; destination d's coefficient is c[d] = sum of the softmax weights
// of edges s -> d over distinct selected sources (source activity is binary,
// model.py:277-278).  The message is then sum_d c[d] * W_edge[d] h.
//
// Plan (forge/ep/dispatch.py:56-115): entries (token, group, weight) sorted
// by group ascending, token ascending — a stable counting sort: per-block
// counts, an exclusive scan, then a scatter whose within-block ranks come
// from wave ballots (deterministic, no atomics on the output order).
#include "smoe_common.hpp"
#include "smoe_internal.hpp"
#include "smoe_plan64.hpp"
#include "smoe_rows.hpp"
#include "smoe_routing.hpp"

namespace smoe {

constexpr int kPlanMaxGroups = 256;  // experts / destinations a block takes

// ------------------------------------------------------------ router ----
// (topk_seg: smoe_routing.hpp)
template <int SEG>
__global__ __launch_bounds__(256) void k_route_topk(const float* __restrict__ logits, int N, int E,
                                                    int K, int32_t* __restrict__ top_idx,
                                                    float* __restrict__ top_w,
                                                    int32_t* __restrict__ tok_e,
                                                    float* __restrict__ tok_ew,
                                                    const int32_t* __restrict__ active) {
  constexpr int TPW = 64 / SEG;
  const int lane = threadIdx.x & 63;
  const int t0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * TPW;
  if (t0 >= N) return;  // wave-uniform
  const int e = lane & (SEG - 1);
  const int t = t0 + lane / SEG;
  const bool ok = t < N;
  const float v = logits[static_cast<int64_t>(ok ? t : N - 1) * E + (e < E ? e : E - 1)];
  const bool live = !active || active[ok ? t : N - 1] != 0;
  topk_seg<SEG>(v, t, ok, live, E, K, top_idx, top_w, tok_e, tok_ew, nullptr, nullptr);
}

// --------------------------------------------- more than 64 experts ----
// The router of topk_seg for 64 < E <= 64 V: the same softmax, top-k on the
// logits (ties to the lowest index), renorm by max(sum, 1e-9) in slot
// order, tok_e / tok_ew ascending.
template <int V>
__global__ __launch_bounds__(256) void k_route_topk_w(const float* __restrict__ logits, int N,
                                                      int E, int K, int32_t* __restrict__ top_idx,
                                                      float* __restrict__ top_w,
                                                      int32_t* __restrict__ tok_e,
                                                      float* __restrict__ tok_ew,
                                                      const int32_t* __restrict__ active) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= N) return;  // wave-uniform
  const bool live = !active || active[t] != 0;
  float x[V], ex[V];
  bool in[V], sel[V];
  float mx = -INFINITY;
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int e = lane + 64 * v;
    in[v] = e < E;
    x[v] = in[v] ? logits[static_cast<int64_t>(t) * E + e] : -INFINITY;
    mx = fmaxf(mx, x[v]);
    sel[v] = false;
  }
  mx = seg_max<64>(mx);
  float part = 0.f;
#pragma unroll
  for (int v = 0; v < V; ++v) {
    ex[v] = in[v] ? expf(x[v] - mx) : 0.f;
    part += ex[v];
  }
  const float sum = seg_sum<64>(part);
  float psum = 0.f, slot_p = 0.f;
  int slot_i = 0;
#pragma unroll 1
  for (int j = 0; j < K; ++j) {
    bool cand[V];
#pragma unroll
    for (int v = 0; v < V; ++v) cand[v] = in[v] && !sel[v];
    float cv;
    int ci;
    wide_argmax<V>(x, cand, cv, ci);
    const float pj = expf(cv - mx) / sum;
#pragma unroll
    for (int v = 0; v < V; ++v) sel[v] = sel[v] || (lane + 64 * v == ci);
    slot_p = lane == j ? pj : slot_p;
    slot_i = lane == j ? ci : slot_i;
    psum += pj;
  }
  const float denom = fmaxf(psum, 1e-9f);
  if (lane < K) {
    top_idx[static_cast<int64_t>(t) * K + lane] = slot_i;
    top_w[static_cast<int64_t>(t) * K + lane] = slot_p / denom;
  }
  if (!tok_e) return;
  if (live) {
    int rank[V];
    wide_ranks<V>(sel, rank);
#pragma unroll
    for (int v = 0; v < V; ++v)
      if (sel[v]) {
        tok_e[static_cast<int64_t>(t) * K + rank[v]] = lane + 64 * v;
        tok_ew[static_cast<int64_t>(t) * K + rank[v]] = ex[v] / sum / denom;
      }
  } else if (lane < K) {
    tok_e[static_cast<int64_t>(t) * K + lane] = -1;
    tok_ew[static_cast<int64_t>(t) * K + lane] = 0.f;
  }
}

// segment width for E entries per token (E <= 64); lane slots per wave for
// wider E
inline int seg_of(int E) { return E <= 16 ? 16 : (E <= 32 ? 32 : 64); }
inline int wide_of(int E) { return (E + 63) / 64; }

int launch_route_topk(const float* logits, int N, int E, int K, int32_t* top_idx, float* top_w,
                      int32_t* tok_e, float* tok_ew, const int32_t* active, hipStream_t s) {
  if (E < 1 || E > kPlanMaxGroups || K < 1 || K > E || K > 16) return SMOE_EINVAL;
  if (N <= 0) return SMOE_OK;
  if (E > 64) {
    const dim3 grid((N + 3) / 4), block(256);
    switch (wide_of(E)) {
      case 2: hipLaunchKernelGGL(k_route_topk_w<2>, grid, block, 0, s, logits, N, E, K, top_idx, top_w, tok_e, tok_ew, active); break;
      case 3: hipLaunchKernelGGL(k_route_topk_w<3>, grid, block, 0, s, logits, N, E, K, top_idx, top_w, tok_e, tok_ew, active); break;
      default: hipLaunchKernelGGL(k_route_topk_w<4>, grid, block, 0, s, logits, N, E, K, top_idx, top_w, tok_e, tok_ew, active); break;
    }
    return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
  }
  const int seg = seg_of(E), per_block = 4 * (64 / seg);
  const dim3 grid((N + per_block - 1) / per_block), block(256);
  if (seg == 16)
    hipLaunchKernelGGL(k_route_topk<16>, grid, block, 0, s, logits, N, E, K, top_idx, top_w, tok_e, tok_ew, active);
  else if (seg == 32)
    hipLaunchKernelGGL(k_route_topk<32>, grid, block, 0, s, logits, N, E, K, top_idx, top_w, tok_e, tok_ew, active);
  else
    hipLaunchKernelGGL(k_route_topk<64>, grid, block, 0, s, logits, N, E, K, top_idx, top_w, tok_e, tok_ew, active);
  return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
}

// --------------------------------------------------------- slot merge ----
// Arbitrary (idx, w) [N,K] -> distinct groups ascending with merged weights
// (sum over the token's slots of that group, in slot order, from 0 — the
// accumulation of sparse_experts.py:52-55).  Ids outside [0, E) never match
// an expert and are dropped, as in the reference; drop_nonpos also drops
// merged weights <= 0 (sparse_experts.py:56).  w == nullptr: every slot
// weighs 1 (a binary source mask, model.py:277-279).
__global__ __launch_bounds__(256) void k_merge_slots(const int32_t* __restrict__ idx,
                                                     const float* __restrict__ w, int N, int K,
                                                     int E, int drop_nonpos,
                                                     int32_t* __restrict__ tok_g,
                                                     float* __restrict__ tok_w) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= N) return;
  const int32_t* ti = idx + static_cast<int64_t>(t) * K;
  const float* tw = w ? w + static_cast<int64_t>(t) * K : nullptr;
  int out = 0;
  int last = -1;
  // emit groups in ascending order: repeatedly take the smallest id > last
  for (int it = 0; it < K; ++it) {
    int best = kBig;
    for (int s = 0; s < K; ++s) {
      const int e = ti[s];
      if (e > last && e < E && e >= 0 && e < best) best = e;
    }
    if (best == kBig) break;
    float acc = 0.f;
    for (int s = 0; s < K; ++s)
      if (ti[s] == best) acc = acc + (tw ? tw[s] : 1.f);
    last = best;
    if (drop_nonpos && !(acc > 0.f)) continue;
    tok_g[static_cast<int64_t>(t) * K + out] = best;
    tok_w[static_cast<int64_t>(t) * K + out] = acc;
    ++out;
  }
  for (; out < K; ++out) {
    tok_g[static_cast<int64_t>(t) * K + out] = -1;
    tok_w[static_cast<int64_t>(t) * K + out] = 0.f;
  }
}

int launch_merge_slots(const int32_t* idx, const float* w, int N, int K, int E, int drop_nonpos,
                       int32_t* tok_g, float* tok_w, hipStream_t s) {
  if (N <= 0) return SMOE_OK;
  hipLaunchKernelGGL(k_merge_slots, dim3((N + 255) / 256), dim3(256), 0, s, idx, w, N, K, E,
                     drop_nonpos, tok_g, tok_w);
  return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
}

// ------------------------------------------------------------- edges ----
// (topm_seg: smoe_routing.hpp)
// The segment's KB source slots (KB >= K, a compile-time bucket): their
// sources and plan rows (every lane reads the same entries, one load each),
// then all their logit rows at once (rows in expert-plan order; slots past K
// or empty read row 0 and are dropped), so the wave waits on memory twice.
template <int SEG, int KB>
__global__ __launch_bounds__(256) void k_edge_topm(const float* __restrict__ edge_logit,
                                                   const int32_t* __restrict__ tok_e,
                                                   const int32_t* __restrict__ e_tokrow, int N,
                                                   int E, int K, int M, int S,
                                                   int32_t* __restrict__ edge_idx,
                                                   float* __restrict__ edge_w,
                                                   int32_t* __restrict__ tok_d,
                                                   float* __restrict__ tok_dc) {
  constexpr int TPW = 64 / SEG;
  const int lane = threadIdx.x & 63;
  const int t0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * TPW;
  if (t0 >= N) return;  // wave-uniform
  const int d = lane & (SEG - 1);
  const int t = t0 + lane / SEG;
  const bool ok = t < N;
  const int64_t tb = static_cast<int64_t>(ok ? t : N - 1) * K;
  int src[KB], rw[KB];
#pragma unroll
  for (int j = 0; j < KB; ++j) {
    const int jj = j < K ? j : K - 1;
    src[j] = tok_e[tb + jj];
    rw[j] = e_tokrow[tb + jj];
  }
  int row[KB];
  bool live[KB];
  float v[KB];
#pragma unroll
  for (int j = 0; j < KB; ++j) {
    live[j] = ok && j < K && src[j] >= 0;  // sources are packed first (ascending expert)
    row[j] = live[j] ? rw[j] : 0;
    v[j] = edge_logit[static_cast<int64_t>(row[j]) * E + (d < E ? d : E - 1)];
  }
  topm_seg<SEG, KB>(v, row, live, t, ok, E, M, S, edge_idx, edge_w, tok_d, tok_dc, nullptr, nullptr);
}

// topm_seg for 64 < E <= 64 V: one wave per token, lane l holding
// destinations l, l + 64, ..; the same per-source top-m, fp32 softmax over
// the m values in slot order, coefficients summed over the sources in
// ascending order, nonzero destinations ascending into tok_d / tok_dc
// (S <= 64 entries).
template <int V, int KB>
__global__ __launch_bounds__(256) void k_edge_topm_w(const float* __restrict__ edge_logit,
                                                     const int32_t* __restrict__ tok_e,
                                                     const int32_t* __restrict__ e_tokrow, int N,
                                                     int E, int K, int M, int S,
                                                     int32_t* __restrict__ edge_idx,
                                                     float* __restrict__ edge_w,
                                                     int32_t* __restrict__ tok_d,
                                                     float* __restrict__ tok_dc) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= N) return;  // wave-uniform
  const int64_t tb = static_cast<int64_t>(t) * K;
  int src[KB], rw[KB];
#pragma unroll
  for (int j = 0; j < KB; ++j) {
    const int jj = j < K ? j : K - 1;
    src[j] = tok_e[tb + jj];
    rw[j] = e_tokrow[tb + jj];
  }
  bool in[V];
  float c[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    in[v] = lane + 64 * v < E;
    c[v] = 0.f;
  }
#pragma unroll
  for (int j = 0; j < KB; ++j) {
    if (!(j < K && src[j] >= 0)) continue;  // uniform: sources are packed first
    const int row = rw[j];
    float x[V];
    bool sel[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      x[v] = in[v] ? edge_logit[static_cast<int64_t>(row) * E + lane + 64 * v] : -INFINITY;
      sel[v] = false;
    }
    float vmax = 0.f, den = 0.f, rec_v = 0.f;
    int rec_i = 0;
#pragma unroll 1
    for (int i = 0; i < M; ++i) {
      bool cand[V];
#pragma unroll
      for (int v = 0; v < V; ++v) cand[v] = in[v] && !sel[v];
      float cv;
      int ci;
      wide_argmax<V>(x, cand, cv, ci);
#pragma unroll
      for (int v = 0; v < V; ++v) sel[v] = sel[v] || (lane + 64 * v == ci);
      vmax = i == 0 ? cv : vmax;
      rec_v = lane == i ? cv : rec_v;
      rec_i = lane == i ? ci : rec_i;
      den += expf(cv - vmax);
    }
#pragma unroll
    for (int v = 0; v < V; ++v)
      if (sel[v]) c[v] += expf(x[v] - vmax) / den;
    if (lane < M) {
      edge_idx[static_cast<int64_t>(row) * M + lane] = rec_i;
      edge_w[static_cast<int64_t>(row) * M + lane] = expf(rec_v - vmax) / den;
    }
  }
  bool nz[V];
#pragma unroll
  for (int v = 0; v < V; ++v) nz[v] = in[v] && c[v] != 0.f;
  int rank[V];
  const int cnt = wide_ranks<V>(nz, rank);
#pragma unroll
  for (int v = 0; v < V; ++v)
    if (nz[v] && rank[v] < S) {
      tok_d[static_cast<int64_t>(t) * S + rank[v]] = lane + 64 * v;
      tok_dc[static_cast<int64_t>(t) * S + rank[v]] = c[v];
    }
  if (lane >= cnt && lane < S) {
    tok_d[static_cast<int64_t>(t) * S + lane] = -1;
    tok_dc[static_cast<int64_t>(t) * S + lane] = 0.f;
  }
}

int launch_edge_topm(const float* edge_logit, const int32_t* tok_e, const int32_t* e_tokrow,
                     int N, int E, int K, int M, int S, int32_t* edge_idx, float* edge_w,
                     int32_t* tok_d, float* tok_dc, hipStream_t s) {
  if (E < 1 || E > kPlanMaxGroups || M < 1 || M > E || M > 16 || S < 1 || S > 64 || K < 1 ||
      K > 16)
    return SMOE_EINVAL;
  if (N <= 0) return SMOE_OK;
  if (E > 64) {
    const dim3 grid((N + 3) / 4), block(256);
#define SMOE_EDGE_TOPM_W(V_, KB)                                                                   hipLaunchKernelGGL((k_edge_topm_w<V_, KB>), grid, block, 0, s, edge_logit, tok_e, e_tokrow, N,                      E, K, M, S, edge_idx, edge_w, tok_d, tok_dc)
#define SMOE_EDGE_TOPM_WK(V_)                   do {                                            if (K <= 2) SMOE_EDGE_TOPM_W(V_, 2);          else if (K <= 4) SMOE_EDGE_TOPM_W(V_, 4);     else if (K <= 8) SMOE_EDGE_TOPM_W(V_, 8);     else SMOE_EDGE_TOPM_W(V_, 16);              } while (0)
    switch (wide_of(E)) {
      case 2: SMOE_EDGE_TOPM_WK(2); break;
      case 3: SMOE_EDGE_TOPM_WK(3); break;
      default: SMOE_EDGE_TOPM_WK(4); break;
    }
#undef SMOE_EDGE_TOPM_WK
#undef SMOE_EDGE_TOPM_W
    return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
  }
  const int seg = seg_of(E), per_block = 4 * (64 / seg);
  const dim3 grid((N + per_block - 1) / per_block), block(256);
#define SMOE_EDGE_TOPM(SG, KB)                                                                   \
  hipLaunchKernelGGL((k_edge_topm<SG, KB>), grid, block, 0, s, edge_logit, tok_e, e_tokrow, N, E, \
                     K, M, S, edge_idx, edge_w, tok_d, tok_dc)
#define SMOE_EDGE_TOPM_K(SG)           \
  do {                                 \
    if (K <= 1) SMOE_EDGE_TOPM(SG, 1); \
    else if (K <= 2) SMOE_EDGE_TOPM(SG, 2); \
    else if (K <= 4) SMOE_EDGE_TOPM(SG, 4); \
    else if (K <= 8) SMOE_EDGE_TOPM(SG, 8); \
    else SMOE_EDGE_TOPM(SG, 16);       \
  } while (0)
  if (seg == 16) SMOE_EDGE_TOPM_K(16);
  else if (seg == 32) SMOE_EDGE_TOPM_K(32);
  else SMOE_EDGE_TOPM_K(64);
#undef SMOE_EDGE_TOPM_K
#undef SMOE_EDGE_TOPM
  return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
}

// Per-source top-m in the caller's slot order: slot j of token t takes the
// row of its source in the expert plan (the token's merged, ascending
// sources tok_e and their plan rows e_tokrow) and copies that row's m
// destinations and weights; slots without a valid source get -1 / 0.
__global__ __launch_bounds__(256) void k_gather_topm(const int32_t* __restrict__ src_idx,
                                                     const int32_t* __restrict__ tok_e,
                                                     const int32_t* __restrict__ e_tokrow,
                                                     const int32_t* __restrict__ edge_idx,
                                                     const float* __restrict__ edge_w, int N,
                                                     int K, int M, int32_t* __restrict__ out_idx,
                                                     float* __restrict__ out_w) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= static_cast<int64_t>(N) * K) return;
  const int64_t t = i / K;
  const int s = src_idx[i];
  int row = -1;
  for (int q = 0; q < K; ++q)
    if (s >= 0 && tok_e[t * K + q] == s) {
      row = e_tokrow[t * K + q];
      break;
    }
  for (int j = 0; j < M; ++j) {
    out_idx[i * M + j] = row >= 0 ? edge_idx[static_cast<int64_t>(row) * M + j] : -1;
    out_w[i * M + j] = row >= 0 ? edge_w[static_cast<int64_t>(row) * M + j] : 0.f;
  }
}

int launch_gather_topm(const int32_t* src_idx, const int32_t* tok_e, const int32_t* e_tokrow,
                       const int32_t* edge_idx, const float* edge_w, int N, int K, int M,
                       int32_t* out_idx, float* out_w, hipStream_t s) {
  const int64_t n = static_cast<int64_t>(N) * K;
  if (n <= 0) return SMOE_OK;
  hipLaunchKernelGGL(k_gather_topm, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s,
                     src_idx, tok_e, e_tokrow, edge_idx, edge_w, N, K, M, out_idx, out_w);
  return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
}

// Destination coefficients of given edges (model.py:277-288): one wave per
// token, lane d = destination d.  The token's distinct valid sources are
// taken in ascending order (a binary mask: a source listed twice counts
// once) and each adds the weights of its edges into d, as the fused top-m
// does; the nonzero destinations, ascending, fill tok_d / tok_dc (S
// entries per token, -1 / 0 past them).
// V: destinations per lane (lane l holds l, l + 64, ..: E <= 64 V).
template <int V>
__global__ __launch_bounds__(256) void k_dest_coeffs(const int32_t* __restrict__ src_idx,
                                                     const int32_t* __restrict__ eidx,
                                                     const float* __restrict__ ew, int N, int K,
                                                     int M, int E, int S,
                                                     int32_t* __restrict__ tok_d,
                                                     float* __restrict__ tok_dc) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= N) return;  // wave-uniform
  const int32_t* ts = src_idx + static_cast<int64_t>(t) * K;
  float c[V];
#pragma unroll
  for (int v = 0; v < V; ++v) c[v] = 0.f;
  int last = -1;
  for (int it = 0; it < K; ++it) {  // uniform: every lane scans the same slots
    int best = kBig, bj = 0;
    for (int j = 0; j < K; ++j) {
      const int e = ts[j];
      if (e > last && e >= 0 && e < E && e < best) {
        best = e;
        bj = j;
      }
    }
    if (best == kBig) break;
    last = best;
    const int64_t b = (static_cast<int64_t>(t) * K + bj) * M;
    for (int j = 0; j < M; ++j) {
      const int d = eidx[b + j];
#pragma unroll
      for (int v = 0; v < V; ++v)
        if (d == lane + 64 * v) c[v] += ew[b + j];
    }
  }
  bool nz[V];
#pragma unroll
  for (int v = 0; v < V; ++v) nz[v] = lane + 64 * v < E && c[v] != 0.f;
  int rank[V];
  const int cnt = wide_ranks<V>(nz, rank);
#pragma unroll
  for (int v = 0; v < V; ++v)
    if (nz[v] && rank[v] < S) {
      tok_d[static_cast<int64_t>(t) * S + rank[v]] = lane + 64 * v;
      tok_dc[static_cast<int64_t>(t) * S + rank[v]] = c[v];
    }
  if (lane >= cnt && lane < S) {
    tok_d[static_cast<int64_t>(t) * S + lane] = -1;
    tok_dc[static_cast<int64_t>(t) * S + lane] = 0.f;
  }
}

int launch_dest_coeffs(const int32_t* src_idx, const int32_t* eidx, const float* ew, int N, int K,
                       int M, int E, int S, int32_t* tok_d, float* tok_dc, hipStream_t s) {
  if (E < 1 || E > kPlanMaxGroups || S < 1 || S > 64 || K < 1 || M < 1) return SMOE_EINVAL;
  if (N <= 0) return SMOE_OK;
  const dim3 grid((N + 3) / 4), block(256);
  switch (wide_of(E)) {
    case 1: hipLaunchKernelGGL(k_dest_coeffs<1>, grid, block, 0, s, src_idx, eidx, ew, N, K, M, E, S, tok_d, tok_dc); break;
    case 2: hipLaunchKernelGGL(k_dest_coeffs<2>, grid, block, 0, s, src_idx, eidx, ew, N, K, M, E, S, tok_d, tok_dc); break;
    case 3: hipLaunchKernelGGL(k_dest_coeffs<3>, grid, block, 0, s, src_idx, eidx, ew, N, K, M, E, S, tok_d, tok_dc); break;
    default: hipLaunchKernelGGL(k_dest_coeffs<4>, grid, block, 0, s, src_idx, eidx, ew, N, K, M, E, S, tok_d, tok_dc); break;
  }
  return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
}

// -------------------------------------------------------------- plan ----
// (the plan's outline and rank_chunk: smoe_routing.hpp)
// Scatter of one token: row = goff[g] + base[g * bs] + rank (group offset,
// the chunk's prefix inside the group, the rank inside the chunk).
template <typename P>
__device__ __forceinline__ void scatter_token(const int32_t* __restrict__ tok_g,
                                              const float* __restrict__ tok_w, int t, int S,
                                              int G, P base, int bs, const int* goff,
                                              int32_t* __restrict__ rows,
                                              float* __restrict__ roww,
                                              int32_t* __restrict__ tokrow) {
  const int64_t e0 = static_cast<int64_t>(t) * S;
  for (int j0 = 0; j0 < S; j0 += 8) {
    int gv[8], rv[8], bv[8], ov[8];
    float wv[8];
    // every load unconditional (clamped indices), so each batch is one
    // round trip to memory
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int jj = j0 + u < S ? j0 + u : S - 1;
      gv[u] = tok_g[e0 + jj];
      rv[u] = tokrow[e0 + jj];
      wv[u] = tok_w[e0 + jj];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int gc = (gv[u] >= 0 && gv[u] < G) ? gv[u] : 0;
      bv[u] = base[gc * bs];
      ov[u] = goff[gc];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (j0 + u >= S || rv[u] < 0 || gv[u] < 0 || gv[u] >= G) continue;
      const int row = ov[u] + bv[u] + rv[u];
      tokrow[e0 + j0 + u] = row;
      rows[row] = t;
      roww[row] = wv[u];
    }
  }
}

// Exclusive scan of tot[0..G) into goff[0..G].  Every thread of the
// workgroup calls it (it holds barriers); the first 256 do the work.
__device__ __forceinline__ void block_group_offsets(const int32_t* tot, int G, int* goff,
                                                    int* wsum) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool act = tid < 256;
  const int v = (act && tid < G) ? tot[tid] : 0;
  const int incl = wave_incl_scan(v);
  if (act && lane == 63) wsum[wave] = incl;
  __syncthreads();
  if (act) {
    int before = 0;
    for (int w = 0; w < wave; ++w) before += wsum[w];
    if (tid < G) goff[tid] = before + incl - v;
    if (tid == 0) goff[G] = wsum[0] + wsum[1] + wsum[2] + wsum[3];
  }
  __syncthreads();
}

// ccnt / cacnt are [G, C] (group-major).  Wave w of the grid ranks chunk
// w / W for the window w % W (W = ceil(G / 64)).
__global__ __launch_bounds__(256) void k_plan_rank(const int32_t* __restrict__ tok_g,
                                                   const float* __restrict__ tok_w, int N, int S,
                                                   int G, int drop, int C, int W,
                                                   int32_t* __restrict__ ccnt,
                                                   int32_t* __restrict__ cacnt,
                                                   int32_t* __restrict__ tokrow) {
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= C * W) return;
  const int win = (G + W - 1) / W;
  const int chunk = item / W, g0 = (item % W) * win;
  rank_chunk(tok_g, tok_w, N, S, G, drop, chunk * 64, g0, win, ccnt + chunk, cacnt + chunk, C,
             tokrow);
}

// One wave per group: chunk counts -> exclusive chunk prefixes (in place),
// group totals -> cnt, positive-weight totals -> acnt.
__device__ __forceinline__ void scan_group(int g, int C, int32_t* __restrict__ ccnt,
                                           const int32_t* __restrict__ cacnt,
                                           int32_t* __restrict__ cnt, int32_t* __restrict__ acnt) {
  const int lane = threadIdx.x;
  int32_t* row = ccnt + static_cast<int64_t>(g) * C;
  const int32_t* arow = cacnt + static_cast<int64_t>(g) * C;
  int run = 0;  // sum of all earlier passes
  int a = 0;
  for (int c0 = 0; c0 < C; c0 += 256) {
    int v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int c = c0 + lane * 4 + k;
      v[k] = c < C ? row[c] : 0;
      a += c < C ? arow[c] : 0;
    }
    const int s = v[0] + v[1] + v[2] + v[3];
    const int incl = wave_incl_scan(s);
    int p = run + incl - s;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int c = c0 + lane * 4 + k;
      if (c < C) row[c] = p;
      p += v[k];
    }
    run += __builtin_amdgcn_readlane(incl, 63);
  }
  a = __builtin_amdgcn_readlane(wave_incl_scan(a), 63);
  if (lane == 0) {
    cnt[g] = run;
    acnt[g] = a;
  }
}

__global__ __launch_bounds__(64) void k_plan_scan(int C, int32_t* __restrict__ ccnt,
                                                  const int32_t* __restrict__ cacnt,
                                                  int32_t* __restrict__ cnt,
                                                  int32_t* __restrict__ acnt) {
  scan_group(blockIdx.x, C, ccnt, cacnt, cnt, acnt);
}

__global__ __launch_bounds__(256) void k_plan_scatter(const int32_t* __restrict__ tok_g,
                                                      const float* __restrict__ tok_w, int N,
                                                      int S, int G, int C,
                                                      const int32_t* __restrict__ cbase,
                                                      const int32_t* __restrict__ cnt,
                                                      int32_t* __restrict__ off,
                                                      int32_t* __restrict__ rows,
                                                      float* __restrict__ roww,
                                                      int32_t* __restrict__ tokrow) {
  __shared__ int goff[kPlanMaxG + 1], wsum[4];
  block_group_offsets(cnt, G, goff, wsum);
  if (blockIdx.x == 0)
    for (int g = threadIdx.x; g <= G; g += 256) off[g] = goff[g];
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= N) return;
  scatter_token(tok_g, tok_w, t, S, G, cbase + (t >> 6), C, goff, rows, roww, tokrow);
}

// Small N: the three phases in one workgroup of 1024 threads, the [G, C]
// chunk counts in LDS (C <= 64: one chunk per lane in the scan).  Groups are
// cut into windows of `win` so that the rank work spreads over the waves.
constexpr int kSmallMaxCells = 8192;
struct PlanSmem {
  int cc[kSmallMaxCells], ca[kSmallMaxCells];
  int tot[kPlanMaxG], goff[kPlanMaxG + 1], wsum[4];
};

// One workgroup of 16 waves: rank (wave per (chunk, window)), scan (wave per
// group), group offsets, scatter (thread per token).
__global__ __launch_bounds__(1024) void k_plan_small(const int32_t* __restrict__ tok_g,
                                                     const float* __restrict__ tok_w, int N,
                                                     int S, int G, int drop, int win,
                                                     int32_t* __restrict__ cnt,
                                                     int32_t* __restrict__ acnt,
                                                     int32_t* __restrict__ off,
                                                     int32_t* __restrict__ rows,
                                                     float* __restrict__ roww,
                                                     int32_t* __restrict__ tokrow) {
  __shared__ PlanSmem sm;
  int* cc = sm.cc;
  int* ca = sm.ca;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int C = (N + 63) / 64;
  const int W = (G + win - 1) / win;
  for (int item = wave; item < C * W; item += 16) {
    const int c = item / W;
    rank_chunk(tok_g, tok_w, N, S, G, drop, c * 64, (item % W) * win, win, cc + c, ca + c, C,
               tokrow);
  }
  __syncthreads();
  for (int g = wave; g < G; g += 16) {
    const int v = lane < C ? cc[g * C + lane] : 0;
    int a = lane < C ? ca[g * C + lane] : 0;
    const int incl = wave_incl_scan(v);
    a = __builtin_amdgcn_readlane(wave_incl_scan(a), 63);
    if (lane < C) cc[g * C + lane] = incl - v;
    if (lane == 63) {
      sm.tot[g] = incl;
      cnt[g] = incl;
      acnt[g] = a;
    }
  }
  __syncthreads();
  block_group_offsets(sm.tot, G, sm.goff, sm.wsum);
  for (int g = threadIdx.x; g <= G; g += 1024) off[g] = sm.goff[g];
  for (int t = threadIdx.x; t < N; t += 1024)
    scatter_token(tok_g, tok_w, t, S, G, cc + (t >> 6), C, sm.goff, rows, roww, tokrow);
}

// Window of the single-workgroup plan: narrower windows until the 16 waves
// have work.
inline int plan_small_win(int C, int G) {
  int win = 64;
  while (win > 8 && C * ((G + win - 1) / win) < 16) win >>= 1;
  return win;
}

// Plans of <= 64 tokens over <= 64 groups outside the fused front (fp32
// blocks, the standalone plan entry point): one wave.
__global__ __launch_bounds__(64) void k_plan64(const int32_t* __restrict__ tok_g,
                                               const float* __restrict__ tok_w, int N, int S,
                                               int G, int drop, int32_t* __restrict__ cnt,
                                               int32_t* __restrict__ acnt,
                                               int32_t* __restrict__ off,
                                               int32_t* __restrict__ rows,
                                               float* __restrict__ roww,
                                               int32_t* __restrict__ tokrow) {
  __shared__ uint64_t km[64], am[64];
  __shared__ int soff[64];
  plan64_wave(tok_g, tok_w, N, S, G, drop, cnt, acnt, off, rows, roww, tokrow, km, am, soff);
}

// Small decode steps: every routing stage in one workgroup of 16 waves, the
// phases separated by workgroup barriers; a token is a segment of SEG lanes
// (64 / SEG tokens per wave, 1024 / SEG per pass).  What a later phase reads
// (the tokens' sources and destinations, the plans' token rows) also goes to
// LDS, so only the logits come from memory.  Within a phase a wave issues
// its logit loads (clamped indices, no branch) before its stores: loads and
// stores share one in-order counter, so a load issued after a store would
// wait for it.
constexpr int kFrontMaxSrc = kFrontMaxN * 16;   // N*K
constexpr int kFrontMaxDst = kFrontMaxN * 64;   // N*S
template <int SEG, int KB>
__global__ __launch_bounds__(1024) void k_front_route(
    const float* __restrict__ front, int ldf, int N, int E, int K, int M, int S,
    float* __restrict__ logits, int32_t* __restrict__ top_idx, float* __restrict__ top_w,
    int32_t* __restrict__ tok_e, float* __restrict__ tok_ew, int32_t* __restrict__ e_cnt,
    int32_t* __restrict__ e_acnt, int32_t* __restrict__ e_off, int32_t* __restrict__ e_rows,
    float* __restrict__ e_roww, int32_t* __restrict__ e_tokrow, float* __restrict__ edge_logit,
    int32_t* __restrict__ edge_idx, float* __restrict__ edge_w, int32_t* __restrict__ tok_d,
    float* __restrict__ tok_dc, int32_t* __restrict__ d_cnt, int32_t* __restrict__ d_acnt,
    int32_t* __restrict__ d_off, int32_t* __restrict__ d_rows, float* __restrict__ d_roww,
    int32_t* __restrict__ d_tokrow, const int32_t* __restrict__ active) {
  constexpr int PASS = 1024 / SEG;  // tokens per pass
  __shared__ int32_t s_e[kFrontMaxSrc], s_etr[kFrontMaxSrc], s_d[kFrontMaxDst], s_dtr[kFrontMaxDst];
  __shared__ float s_ew[kFrontMaxSrc], s_dc[kFrontMaxDst];
  __shared__ uint64_t s_km[64], s_am[64];
  __shared__ int s_off[64];
  const int lane = threadIdx.x & 63;
  const int e = lane & (SEG - 1);
  const int le = e < E ? e : E - 1;
  const int tl = threadIdx.x / SEG;  // token of this lane within a pass
  // 1 router top-k (and the logits region)
  for (int t0 = 0; t0 < N; t0 += PASS) {
    const int t = t0 + tl;
    const bool ok = t < N;
    const float v = front[static_cast<int64_t>(ok ? t : N - 1) * ldf + le];
    const bool live = !active || active[ok ? t : N - 1] != 0;
    if (ok && e < E) logits[static_cast<int64_t>(t) * E + e] = v;
    topk_seg<SEG>(v, t, ok, live, E, K, top_idx, top_w, tok_e, tok_ew, s_e, s_ew);
  }
  lds_barrier();
  // 2 expert plan (wave 0)
  if (threadIdx.x < 64)
    plan64_wave(s_e, s_ew, N, K, E, 0, e_cnt, e_acnt, e_off, e_rows, e_roww, s_etr, s_km, s_am,
                s_off);
  lds_barrier();
  // 3 top-m over each token's sources (dense logit rows of the front GEMM)
  const float* dense = front + E;
  for (int t0 = 0; t0 < N; t0 += PASS) {
    const int t = t0 + tl;
    const bool ok = t < N;
    const int tc = ok ? t : N - 1;
    float v[KB];
    int row[KB];
    bool live[KB];
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      const int jj = j < K ? j : K - 1;
      const int sj = s_e[tc * K + jj], rj = s_etr[tc * K + jj];
      live[j] = ok && j < K && sj >= 0;
      row[j] = live[j] ? rj : 0;
      v[j] = dense[static_cast<int64_t>(tc) * ldf + (live[j] ? sj : 0) * E + le];
    }
#pragma unroll
    for (int j = 0; j < KB; ++j)
      if (live[j] && e < E) edge_logit[static_cast<int64_t>(row[j]) * E + e] = v[j];
    topm_seg<SEG, KB>(v, row, live, t, ok, E, M, S, edge_idx, edge_w, tok_d, tok_dc, s_d, s_dc);
  }
  for (int i = threadIdx.x; i < N * K; i += 1024) e_tokrow[i] = s_etr[i];
  lds_barrier();
  // 4 destination plan (wave 0)
  if (threadIdx.x < 64)
    plan64_wave(s_d, s_dc, N, S, E, 1, d_cnt, d_acnt, d_off, d_rows, d_roww, s_dtr, s_km, s_am,
                s_off);
  lds_barrier();
  for (int i = threadIdx.x; i < N * S; i += 1024) d_tokrow[i] = s_dtr[i];
}

int launch_front_route(const float* front, int ldf, int N, int E, int K, int M, int S,
                       float* logits, int32_t* top_idx, float* top_w, int32_t* tok_e,
                       float* tok_ew, int32_t* e_cnt, int32_t* e_acnt, int32_t* e_off,
                       int32_t* e_rows, float* e_roww, int32_t* e_tokrow, float* edge_logit,
                       int32_t* edge_idx, float* edge_w, int32_t* tok_d, float* tok_dc,
                       int32_t* d_cnt, int32_t* d_acnt, int32_t* d_off, int32_t* d_rows,
                       float* d_roww, int32_t* d_tokrow, const int32_t* active, hipStream_t s) {
  if (N < 1 || N > kFrontMaxN || E < 1 || E > 64 || K < 1 || K > 16 || K > E || M < 1 || M > 16 ||
      M > E || S < 1 || S > 64 || ldf < E + E * E)
    return SMOE_EINVAL;
#define SMOE_FRONT(SG, KB)                                                                      \
  hipLaunchKernelGGL((k_front_route<SG, KB>), dim3(1), dim3(1024), 0, s, front, ldf, N, E, K, M, S, \
                     logits, top_idx, top_w, tok_e, tok_ew, e_cnt, e_acnt, e_off, e_rows,          \
                     e_roww, e_tokrow, edge_logit, edge_idx, edge_w, tok_d, tok_dc, d_cnt, d_acnt, \
                     d_off, d_rows, d_roww, d_tokrow, active)
#define SMOE_FRONT_K(SG)           \
  do {                             \
    if (K <= 1) SMOE_FRONT(SG, 1); \
    else if (K <= 2) SMOE_FRONT(SG, 2); \
    else if (K <= 4) SMOE_FRONT(SG, 4); \
    else if (K <= 8) SMOE_FRONT(SG, 8); \
    else SMOE_FRONT(SG, 16);       \
  } while (0)
  const int seg = seg_of(E);
  if (seg == 16) SMOE_FRONT_K(16);
  else if (seg == 32) SMOE_FRONT_K(32);
  else SMOE_FRONT_K(64);
#undef SMOE_FRONT_K
#undef SMOE_FRONT
  return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
}

// ------------------------------------------------------- decode loop ----
#include "smoe_decode.inl"

size_t plan_scratch_bytes(int N, int G) {
  const size_t C = (static_cast<size_t>(N > 0 ? N : 1) + 63) / 64;
  return 2 * C * static_cast<size_t>(G) * sizeof(int32_t);
}

int launch_plan(const int32_t* tok_g, const float* tok_w, int N, int S, int G, int drop,
                int32_t* cnt, int32_t* acnt, int32_t* off, int32_t* rows, float* roww,
                int32_t* tokrow, void* scratch, hipStream_t s) {
  if (G < 1 || G > kPlanMaxG || S < 1 || S > kPlanMaxS || N < 0) return SMOE_EINVAL;
  const int C = (N + 63) / 64;
  // One wave for a single chunk over <= 64 groups; one workgroup while its
  // rank work (C x G ballots) stays small; the three-kernel form spreads
  // larger plans over the chip.
  if (N <= 64 && G <= 64) {
    hipLaunchKernelGGL(k_plan64, dim3(1), dim3(64), 0, s, tok_g, tok_w, N, S, G, drop, cnt, acnt,
                       off, rows, roww, tokrow);
    return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
  }
  if (C * G <= 512) {
    const int win = plan_small_win(C, G);
    hipLaunchKernelGGL(k_plan_small, dim3(1), dim3(1024), 0, s, tok_g, tok_w, N, S, G, drop, win,
                       cnt, acnt, off, rows, roww, tokrow);
    return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
  }
  // group windows per chunk: narrower windows (fewer ballots per wave) until
  // the rank kernel has about 256 waves (C4: 34 chunks x 64 groups -> 8
  // windows of 8)
  int W = (G + 63) / 64;
  while (C * W < 256 && (G + W - 1) / W > 8) W *= 2;
  int32_t* ccnt = reinterpret_cast<int32_t*>(scratch);
  int32_t* cacnt = ccnt + static_cast<int64_t>(C) * G;
  hipLaunchKernelGGL(k_plan_rank, dim3((C * W + 3) / 4), dim3(256), 0, s, tok_g, tok_w, N, S, G,
                     drop, C, W, ccnt, cacnt, tokrow);
  hipLaunchKernelGGL(k_plan_scan, dim3(G), dim3(64), 0, s, C, ccnt, cacnt, cnt, acnt);
  hipLaunchKernelGGL(k_plan_scatter, dim3((N + 255) / 256), dim3(256), 0, s, tok_g, tok_w, N, S,
                     G, C, ccnt, cnt, off, rows, roww, tokrow);
  return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
}

// The scan and scatter of two plans (the expert plan and the destination
// plan of one loop) whose chunk ranks are in place, one launch each: each
// launch's workgroups are split between the plans, which use the same device
// code as launch_plan (so the same results).  The first plan may carry a
// payload: pay_m values per entry (slot order, entry (t, j) at
// (t * S + j) * pay_m) that its scatter copies to the entry's plan row
// (row * pay_m) — the per-source edges.
struct Plan2 {
  const int32_t* tok_g;
  const float* tok_w;
  int S, G, drop;
  int32_t *cnt, *acnt, *off, *rows;
  float* roww;
  int32_t* tokrow;
  int32_t *ccnt, *cacnt;
  const int32_t* pay_idx;
  const float* pay_w;
  int32_t* out_idx;
  float* out_w;
  int pay_m;
};

__global__ __launch_bounds__(64) void k_plan2_scan(const Plan2 a, const Plan2 b, int C) {
  const bool second = static_cast<int>(blockIdx.x) >= a.G;
  const Plan2& p = second ? b : a;
  scan_group(second ? blockIdx.x - a.G : blockIdx.x, C, p.ccnt, p.cacnt, p.cnt, p.acnt);
}

__global__ __launch_bounds__(256) void k_plan2_scatter(const Plan2 a, const Plan2 b, int N, int C) {
  __shared__ int goff[kPlanMaxG + 1], wsum[4];
  const int nb = (N + 255) / 256;
  const bool second = static_cast<int>(blockIdx.x) >= nb;
  const Plan2& p = second ? b : a;
  const int blk = second ? blockIdx.x - nb : blockIdx.x;
  block_group_offsets(p.cnt, p.G, goff, wsum);
  if (blk == 0)
    for (int g = threadIdx.x; g <= p.G; g += 256) p.off[g] = goff[g];
  const int t = blk * 256 + threadIdx.x;
  if (t >= N) return;
  scatter_token(p.tok_g, p.tok_w, t, p.S, p.G, p.ccnt + (t >> 6), C, goff, p.rows, p.roww, p.tokrow);
  if (p.pay_m <= 0) return;
  const int64_t e0 = static_cast<int64_t>(t) * p.S;
  for (int j = 0; j < p.S; ++j) {
    const int row = p.tokrow[e0 + j];  // this thread's own store above: -1 for dropped entries
    if (row < 0) continue;
    for (int i = 0; i < p.pay_m; ++i) {
      p.out_idx[static_cast<int64_t>(row) * p.pay_m + i] = p.pay_idx[(e0 + j) * p.pay_m + i];
      p.out_w[static_cast<int64_t>(row) * p.pay_m + i] = p.pay_w[(e0 + j) * p.pay_m + i];
    }
  }
}

int launch_plan2_finish(const PlanSpec& pa, const PlanSpec& pb, int N, void* scratch,
                        hipStream_t s) {
  for (const PlanSpec* p : {&pa, &pb})
    if (p->G < 1 || p->G > kPlanMaxG || p->S < 1 || p->S > kPlanMaxS) return SMOE_EINVAL;
  if (N < 1 || !scratch || pb.pay_m > 0) return SMOE_EINVAL;  // the payload rides with the first plan
  const int C = (N + 63) / 64;
  Plan2 a, b;
  int32_t* z = reinterpret_cast<int32_t*>(scratch);
  Plan2* dst[2] = {&a, &b};
  const PlanSpec* src[2] = {&pa, &pb};
  for (int i = 0; i < 2; ++i) {
    const PlanSpec& p = *src[i];
    Plan2& q = *dst[i];
    q.tok_g = p.tok_g;
    q.tok_w = p.tok_w;
    q.S = p.S;
    q.G = p.G;
    q.drop = p.drop;
    q.cnt = p.cnt;
    q.acnt = p.acnt;
    q.off = p.off;
    q.rows = p.rows;
    q.roww = p.roww;
    q.tokrow = p.tokrow;
    q.ccnt = z;
    q.cacnt = z + static_cast<int64_t>(C) * p.G;
    z += 2 * static_cast<int64_t>(C) * p.G;
    q.pay_idx = p.pay_idx;
    q.pay_w = p.pay_w;
    q.out_idx = p.out_idx;
    q.out_w = p.out_w;
    q.pay_m = p.pay_m;
  }
  hipLaunchKernelGGL(k_plan2_scan, dim3(a.G + b.G), dim3(64), 0, s, a, b, C);
  hipLaunchKernelGGL(k_plan2_scatter, dim3(2 * ((N + 255) / 256)), dim3(256), 0, s, a, b, N, C);
  return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
}

// ------------------------------------------------------ loop bias ----
__global__ void k_edge_loop_bias(const void* __restrict__ wg, int act_dtype,
                                 const float* __restrict__ bg, const float* __restrict__ emb,
                                 int E2, int H, int L, int R, float* __restrict__ out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= R * E2) return;
  const int r = i / E2, o = i % E2;
  float acc = bg ? bg[o] : 0.f;
  const int64_t rowoff = static_cast<int64_t>(o) * (H + L) + H;
  for (int l = 0; l < L; ++l) {
    const float w = act_dtype == SMOE_F32 ? reinterpret_cast<const float*>(wg)[rowoff + l]
                                          : bf2f(reinterpret_cast<const uint16_t*>(wg)[rowoff + l]);
    acc = fmaf(w, emb[static_cast<int64_t>(r) * L + l], acc);
  }
  out[i] = acc;
}

int launch_edge_loop_bias(const void* wg, int act_dtype, const float* bg, const float* emb, int E,
                          int H, int L, int R, float* out, hipStream_t s) {
  const int n = R * E * E;
  if (n <= 0) return SMOE_OK;
  hipLaunchKernelGGL(k_edge_loop_bias, dim3((n + 255) / 256), dim3(256), 0, s, wg, act_dtype, bg,
                     emb, E * E, H, L, R, out);
  return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
}

}  // namespace smoe
