// Routing of the Spider-MoE block: router top-k, edge generator top-m with
// per-token destination coefficients, and the stable dispatch plan.
//
// Router (model.py:255-258): logits (fp32, loop bias added by the logits
// GEMM) -> softmax -> top-k -> renorm by max(sum, 1e-9).  One wave per token,
// lane e holds expert e (E <= 64); selection is on the logits (softmax is
// monotonic), ties to the lowest index.
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

namespace smoe {

constexpr int kBig = 1 << 20;

// ------------------------------------------------------------ router ----
__global__ __launch_bounds__(256) void k_route_topk(const float* __restrict__ logits, int N, int E,
                                                    int K, int32_t* __restrict__ top_idx,
                                                    float* __restrict__ top_w,
                                                    int32_t* __restrict__ tok_e,
                                                    float* __restrict__ tok_ew) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= N) return;
  const bool in = lane < E;
  const float v = in ? logits[static_cast<int64_t>(t) * E + lane] : -INFINITY;
  const float mx = wave_max(v);
  const float ex = in ? expf(v - mx) : 0.f;
  const float sum = wave_sum(ex);
  const float p = ex / sum;
  bool sel = false;
  float psum = 0.f;
  float slot_p = 0.f;
  int slot_i = 0;
#pragma unroll
  for (int j = 0; j < 16; ++j) {  // K <= 16
    if (j < K) {
      float cv = (in && !sel) ? v : -INFINITY;
      int ci = (in && !sel) ? lane : kBig;
      wave_argmax(cv, ci);
      const float pj = __shfl(p, ci & 63);
      if (lane == ci) sel = true;
      if (lane == j) {
        slot_p = pj;
        slot_i = ci;
      }
      psum += pj;  // slot order, as torch sums the k values
    }
  }
  const float denom = fmaxf(psum, 1e-9f);
  if (lane < K) {
    top_idx[static_cast<int64_t>(t) * K + lane] = slot_i;
    top_w[static_cast<int64_t>(t) * K + lane] = slot_p / denom;
  }
  // distinct experts of the token in ascending order (lane order)
  const uint64_t m = __ballot(sel);
  if (sel) {
    const int rank = __popcll(m & ((1ull << lane) - 1));
    tok_e[static_cast<int64_t>(t) * K + rank] = lane;
    tok_ew[static_cast<int64_t>(t) * K + rank] = p / denom;
  }
}

int launch_route_topk(const float* logits, int N, int E, int K, int32_t* top_idx, float* top_w,
                      int32_t* tok_e, float* tok_ew, hipStream_t s) {
  if (E < 1 || E > 64 || K < 1 || K > E || K > 16) return SMOE_EINVAL;
  if (N <= 0) return SMOE_OK;
  hipLaunchKernelGGL(k_route_topk, dim3((N + 3) / 4), dim3(256), 0, s, logits, N, E, K, top_idx,
                     top_w, tok_e, tok_ew);
  return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
}

// --------------------------------------------------------- slot merge ----
// Arbitrary (idx, w) [N,K] -> distinct groups ascending with merged weights
// (sum over the token's slots of that group, in slot order, from 0 — the
// accumulation of sparse_experts.py:52-55).  Ids outside [0, E) never match
// an expert and are dropped, as in the reference; drop_nonpos also drops
// merged weights <= 0 (sparse_experts.py:56).
__global__ __launch_bounds__(256) void k_merge_slots(const int32_t* __restrict__ idx,
                                                     const float* __restrict__ w, int N, int K,
                                                     int E, int drop_nonpos,
                                                     int32_t* __restrict__ tok_g,
                                                     float* __restrict__ tok_w) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= N) return;
  const int32_t* ti = idx + static_cast<int64_t>(t) * K;
  const float* tw = w + static_cast<int64_t>(t) * K;
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
      if (ti[s] == best) acc = acc + tw[s];
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
__global__ __launch_bounds__(256) void k_edge_topm(const float* __restrict__ edge_logit,
                                                   const int32_t* __restrict__ tok_e,
                                                   const int32_t* __restrict__ e_tokrow, int N,
                                                   int E, int K, int M, int S,
                                                   int32_t* __restrict__ edge_idx,
                                                   float* __restrict__ edge_w,
                                                   int32_t* __restrict__ tok_d,
                                                   float* __restrict__ tok_dc) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= N) return;
  const bool in = lane < E;
  float c = 0.f;
  for (int j = 0; j < K; ++j) {
    const int src = tok_e[static_cast<int64_t>(t) * K + j];
    if (src < 0) break;
    const int row = e_tokrow[static_cast<int64_t>(t) * K + j];
    const float v = in ? edge_logit[static_cast<int64_t>(row) * E + lane] : -INFINITY;
    bool sel = false;
    float vmax = 0.f, den = 0.f, rec_v = 0.f;
    int rec_i = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {  // M <= 16
      if (i < M) {
        float cv = (in && !sel) ? v : -INFINITY;
        int ci = (in && !sel) ? lane : kBig;
        wave_argmax(cv, ci);
        if (lane == ci) sel = true;
        if (i == 0) vmax = cv;
        if (lane == i) {
          rec_v = cv;
          rec_i = ci;
        }
        den += expf(cv - vmax);  // softmax over the m values, slot order
      }
    }
    if (sel) c += expf(v - vmax) / den;
    if (lane < M) {
      edge_idx[static_cast<int64_t>(row) * M + lane] = rec_i;
      edge_w[static_cast<int64_t>(row) * M + lane] = expf(rec_v - vmax) / den;
    }
  }
  const bool nz = in && c != 0.f;
  const uint64_t m = __ballot(nz);
  const int cnt = __popcll(m);
  if (nz) {
    const int rank = __popcll(m & ((1ull << lane) - 1));
    tok_d[static_cast<int64_t>(t) * S + rank] = lane;
    tok_dc[static_cast<int64_t>(t) * S + rank] = c;
  }
  if (lane >= cnt && lane < S) {
    tok_d[static_cast<int64_t>(t) * S + lane] = -1;
    tok_dc[static_cast<int64_t>(t) * S + lane] = 0.f;
  }
}

int launch_edge_topm(const float* edge_logit, const int32_t* tok_e, const int32_t* e_tokrow,
                     int N, int E, int K, int M, int S, int32_t* edge_idx, float* edge_w,
                     int32_t* tok_d, float* tok_dc, hipStream_t s) {
  if (E < 1 || E > 64 || M < 1 || M > E || M > 16 || S < 1 || S > 64) return SMOE_EINVAL;
  if (N <= 0) return SMOE_OK;
  hipLaunchKernelGGL(k_edge_topm, dim3((N + 3) / 4), dim3(256), 0, s, edge_logit, tok_e, e_tokrow,
                     N, E, K, M, S, edge_idx, edge_w, tok_d, tok_dc);
  return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
}

// -------------------------------------------------------------- plan ----
// Entries: tok_g [N,S] groups ascending per token (-1 pad), tok_w [N,S].
// An entry is kept when 0 <= g < G and (!drop_nonpos || w > 0).
constexpr int kPlanThreads = 256;
constexpr int kPlanMaxG = 256;

__device__ __forceinline__ bool keep_entry(int g, float w, int G, int drop) {
  return g >= 0 && g < G && (!drop || w > 0.f);
}

// Rank the kept entries of tokens [t0, t0+256) within the block and scatter
// them to rows base[g] + rank.  base[] (LDS) advances by the chunk's counts.
__device__ void plan_scatter_chunk(const int32_t* __restrict__ tok_g,
                                   const float* __restrict__ tok_w, int N, int S, int G, int drop,
                                   int t0, int* base, int (*wcnt)[kPlanMaxG],
                                   int32_t* __restrict__ rows, float* __restrict__ roww,
                                   int32_t* __restrict__ tokrow) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int t = t0 + tid;
  const bool valid = t < N;
  const int32_t* tg = tok_g + static_cast<int64_t>(t) * S;
  const float* tw = tok_w + static_cast<int64_t>(t) * S;
  // phase A: within-wave rank of each kept entry, stored in tokrow
  int j = 0;  // entries are sorted by group, so matches arrive in slot order
  int gj = valid && S > 0 ? tg[0] : -1;
  for (int g = 0; g < G; ++g) {
    while (valid && j < S && gj >= 0 && gj < g) {  // skip out-of-order / dropped
      tokrow[static_cast<int64_t>(t) * S + j] = -1;
      ++j;
      gj = j < S ? tg[j] : -1;
    }
    const bool has = valid && j < S && gj == g && keep_entry(g, tw[j], G, drop);
    const uint64_t m = __ballot(has);
    if (lane == 0) wcnt[wave][g] = __popcll(m);
    if (valid && j < S && gj == g) {
      tokrow[static_cast<int64_t>(t) * S + j] = has ? __popcll(m & ((1ull << lane) - 1)) : -1;
      ++j;
      gj = j < S ? tg[j] : -1;
    }
  }
  for (; valid && j < S; ++j) tokrow[static_cast<int64_t>(t) * S + j] = -1;
  __syncthreads();
  // phase B: per-group wave prefixes -> wcnt[w][g] becomes the wave's row base
  for (int g = tid; g < G; g += kPlanThreads) {
    int run = base[g];
    for (int w = 0; w < kPlanThreads / 64; ++w) {
      const int c = wcnt[w][g];
      wcnt[w][g] = run;
      run += c;
    }
    base[g] = run;
  }
  __syncthreads();
  // phase C: final rows
  if (valid) {
    for (int jj = 0; jj < S; ++jj) {
      const int g = tg[jj];
      const int64_t o = static_cast<int64_t>(t) * S + jj;
      const int r = tokrow[o];
      if (r < 0 || g < 0 || g >= G) continue;
      const int row = wcnt[wave][g] + r;
      tokrow[o] = row;
      rows[row] = t;
      roww[row] = tw[jj];
    }
  }
  __syncthreads();
}

// Single-workgroup plan (small N): count, scan and scatter in one launch.
__global__ __launch_bounds__(kPlanThreads) void k_plan_fused(
    const int32_t* __restrict__ tok_g, const float* __restrict__ tok_w, int N, int S, int G,
    int drop, int32_t* __restrict__ cnt, int32_t* __restrict__ acnt, int32_t* __restrict__ off,
    int32_t* __restrict__ rows, float* __restrict__ roww, int32_t* __restrict__ tokrow) {
  __shared__ int hist[kPlanMaxG], ahist[kPlanMaxG], base[kPlanMaxG];
  __shared__ int wcnt[kPlanThreads / 64][kPlanMaxG];
  const int tid = threadIdx.x;
  for (int g = tid; g < G; g += kPlanThreads) hist[g] = ahist[g] = 0;
  __syncthreads();
  for (int t = tid; t < N; t += kPlanThreads)
    for (int j = 0; j < S; ++j) {
      const int g = tok_g[static_cast<int64_t>(t) * S + j];
      const float w = tok_w[static_cast<int64_t>(t) * S + j];
      if (keep_entry(g, w, G, drop)) {
        atomicAdd(&hist[g], 1);
        if (w > 0.f) atomicAdd(&ahist[g], 1);
      }
    }
  __syncthreads();
  if (tid == 0) {
    int run = 0;
    for (int g = 0; g < G; ++g) {
      base[g] = run;
      off[g] = run;
      cnt[g] = hist[g];
      acnt[g] = ahist[g];
      run += hist[g];
    }
    off[G] = run;
  }
  __syncthreads();
  for (int t0 = 0; t0 < N; t0 += kPlanThreads)
    plan_scatter_chunk(tok_g, tok_w, N, S, G, drop, t0, base, wcnt, rows, roww, tokrow);
}

__global__ __launch_bounds__(kPlanThreads) void k_plan_count(const int32_t* __restrict__ tok_g,
                                                             const float* __restrict__ tok_w,
                                                             int N, int S, int G, int drop,
                                                             int chunk, int32_t* __restrict__ bc,
                                                             int32_t* __restrict__ bac) {
  __shared__ int hist[kPlanMaxG], ahist[kPlanMaxG];
  const int tid = threadIdx.x;
  for (int g = tid; g < G; g += kPlanThreads) hist[g] = ahist[g] = 0;
  __syncthreads();
  const int t_end = min(N, (blockIdx.x + 1) * chunk);
  for (int t = blockIdx.x * chunk + tid; t < t_end; t += kPlanThreads)
    for (int j = 0; j < S; ++j) {
      const int g = tok_g[static_cast<int64_t>(t) * S + j];
      const float w = tok_w[static_cast<int64_t>(t) * S + j];
      if (keep_entry(g, w, G, drop)) {
        atomicAdd(&hist[g], 1);
        if (w > 0.f) atomicAdd(&ahist[g], 1);
      }
    }
  __syncthreads();
  for (int g = tid; g < G; g += kPlanThreads) {
    bc[static_cast<int64_t>(blockIdx.x) * G + g] = hist[g];
    bac[static_cast<int64_t>(blockIdx.x) * G + g] = ahist[g];
  }
}

// One workgroup: totals per group, exclusive scan over groups, and each
// block's base row per group (bc is overwritten with the bases).
__global__ __launch_bounds__(kPlanThreads) void k_plan_scan(int nblk, int G,
                                                            int32_t* __restrict__ bc,
                                                            const int32_t* __restrict__ bac,
                                                            int32_t* __restrict__ cnt,
                                                            int32_t* __restrict__ acnt,
                                                            int32_t* __restrict__ off) {
  __shared__ int tot[kPlanMaxG], goff[kPlanMaxG + 1];
  const int tid = threadIdx.x;
  for (int g = tid; g < G; g += kPlanThreads) {
    int s = 0, a = 0;
    for (int b = 0; b < nblk; ++b) {
      s += bc[static_cast<int64_t>(b) * G + g];
      a += bac[static_cast<int64_t>(b) * G + g];
    }
    tot[g] = s;
    cnt[g] = s;
    acnt[g] = a;
  }
  __syncthreads();
  if (tid == 0) {
    int run = 0;
    for (int g = 0; g < G; ++g) {
      goff[g] = run;
      run += tot[g];
    }
    goff[G] = run;
  }
  __syncthreads();
  for (int g = tid; g <= G; g += kPlanThreads) off[g] = goff[g];
  for (int g = tid; g < G; g += kPlanThreads) {
    int run = goff[g];
    for (int b = 0; b < nblk; ++b) {
      const int64_t i = static_cast<int64_t>(b) * G + g;
      const int c = bc[i];
      bc[i] = run;
      run += c;
    }
  }
}

__global__ __launch_bounds__(kPlanThreads) void k_plan_scatter(
    const int32_t* __restrict__ tok_g, const float* __restrict__ tok_w, int N, int S, int G,
    int drop, int chunk, const int32_t* __restrict__ bbase, int32_t* __restrict__ rows,
    float* __restrict__ roww, int32_t* __restrict__ tokrow) {
  __shared__ int base[kPlanMaxG];
  __shared__ int wcnt[kPlanThreads / 64][kPlanMaxG];
  const int tid = threadIdx.x;
  for (int g = tid; g < G; g += kPlanThreads)
    base[g] = bbase[static_cast<int64_t>(blockIdx.x) * G + g];
  __syncthreads();
  const int t_beg = blockIdx.x * chunk;
  const int t_end = min(N, t_beg + chunk);
  for (int t0 = t_beg; t0 < t_end; t0 += kPlanThreads)
    plan_scatter_chunk(tok_g, tok_w, t_end, S, G, drop, t0, base, wcnt, rows, roww, tokrow);
}

namespace {
constexpr int kFusedMaxN = 4096;
constexpr int kMaxBlocks = 256;
int plan_blocks(int N, int* chunk) {
  int nblk = (N + kPlanThreads - 1) / kPlanThreads;
  if (nblk > kMaxBlocks) nblk = kMaxBlocks;
  int c = (N + nblk - 1) / nblk;
  c = (c + kPlanThreads - 1) / kPlanThreads * kPlanThreads;
  *chunk = c;
  return (N + c - 1) / c;
}
}  // namespace

size_t plan_scratch_bytes(int N, int G) {
  int chunk;
  const int nblk = plan_blocks(N > 0 ? N : 1, &chunk);
  return static_cast<size_t>(2) * nblk * G * sizeof(int32_t);
}

int launch_plan(const int32_t* tok_g, const float* tok_w, int N, int S, int G, int drop,
                int32_t* cnt, int32_t* acnt, int32_t* off, int32_t* rows, float* roww,
                int32_t* tokrow, void* scratch, hipStream_t s) {
  if (G < 1 || G > kPlanMaxG || S < 1) return SMOE_EINVAL;
  if (N <= kFusedMaxN) {
    hipLaunchKernelGGL(k_plan_fused, dim3(1), dim3(kPlanThreads), 0, s, tok_g, tok_w, N, S, G,
                       drop, cnt, acnt, off, rows, roww, tokrow);
    return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
  }
  int chunk;
  const int nblk = plan_blocks(N, &chunk);
  int32_t* bc = reinterpret_cast<int32_t*>(scratch);
  int32_t* bac = bc + static_cast<int64_t>(nblk) * G;
  hipLaunchKernelGGL(k_plan_count, dim3(nblk), dim3(kPlanThreads), 0, s, tok_g, tok_w, N, S, G,
                     drop, chunk, bc, bac);
  hipLaunchKernelGGL(k_plan_scan, dim3(1), dim3(kPlanThreads), 0, s, nblk, G, bc, bac, cnt, acnt,
                     off);
  hipLaunchKernelGGL(k_plan_scatter, dim3(nblk), dim3(kPlanThreads), 0, s, tok_g, tok_w, N, S, G,
                     drop, chunk, bc, rows, roww, tokrow);
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
