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
// One wave per token, lane d = destination.  The token's KB source slots
// (KB >= K, a compile-time bucket) are fetched one lane per slot, then all
// their logit rows at once (slots past K or empty read row 0 and are
// dropped), so the kernel waits on memory twice.
template <int KB>
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
  const int64_t e = static_cast<int64_t>(t) * K + (lane < K ? lane : K - 1);
  const int src_l = tok_e[e];
  const int row_l = e_tokrow[e];
  int row[KB];
  bool live[KB];
  float v[KB];
#pragma unroll
  for (int j = 0; j < KB; ++j) {
    const int sj = __shfl(src_l, j);
    const int rj = __shfl(row_l, j);
    live[j] = j < K && sj >= 0;  // sources are packed first (ascending expert)
    row[j] = live[j] ? rj : 0;
    v[j] = edge_logit[static_cast<int64_t>(row[j]) * E + (in ? lane : 0)];
  }
  float c = 0.f;
#pragma unroll
  for (int j = 0; j < KB; ++j) {
    if (!live[j]) continue;  // uniform
    const float vj = in ? v[j] : -INFINITY;
    bool sel = false;
    float vmax = 0.f, den = 0.f, rec_v = 0.f;
    int rec_i = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {  // M <= 16
      if (i < M) {
        float cv = (in && !sel) ? vj : -INFINITY;
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
    if (sel) c += expf(vj - vmax) / den;
    if (lane < M) {
      edge_idx[static_cast<int64_t>(row[j]) * M + lane] = rec_i;
      edge_w[static_cast<int64_t>(row[j]) * M + lane] = expf(rec_v - vmax) / den;
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
  if (E < 1 || E > 64 || M < 1 || M > E || M > 16 || S < 1 || S > 64 || K < 1 || K > 16)
    return SMOE_EINVAL;
  if (N <= 0) return SMOE_OK;
  const dim3 grid((N + 3) / 4), block(256);
#define SMOE_EDGE_TOPM(KB)                                                                     \
  hipLaunchKernelGGL(k_edge_topm<KB>, grid, block, 0, s, edge_logit, tok_e, e_tokrow, N, E, K, M, \
                     S, edge_idx, edge_w, tok_d, tok_dc)
  if (K <= 1) SMOE_EDGE_TOPM(1);
  else if (K <= 2) SMOE_EDGE_TOPM(2);
  else if (K <= 4) SMOE_EDGE_TOPM(4);
  else if (K <= 8) SMOE_EDGE_TOPM(8);
  else SMOE_EDGE_TOPM(16);
#undef SMOE_EDGE_TOPM
  return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
}

// -------------------------------------------------------------- plan ----
// Entries: tok_g [N,S] and tok_w [N,S], S <= 256.  A token's valid entries
// are the prefix of strictly ascending groups in [0, G); from the first
// entry that is not greater than the previous one or not in [0, G) on, the
// row is padding (the producers write the token's groups ascending followed
// by -1 pads).  A valid entry is kept when !drop_nonpos || w > 0.
//
// Tokens are cut into chunks of 64 (one wave, one token per lane) and groups
// into windows of at most 64.
//   rank:    one wave per (chunk, window): each lane turns its token's
//            entries into bit masks over the window (present / kept /
//            positive weight); one ballot per group gives the chunk's count
//            (kept in the lane of that group) and each kept entry's rank
//            among the chunk's earlier tokens
//   scan:    one wave per group: exclusive scan of the chunk counts
//   scatter: group offsets by a workgroup scan of the group totals, then
//            row = off[g] + chunk prefix + rank -> rows / row_w / tok_row
// Token order inside a group is preserved (stable) and no atomics are used,
// so the plan is bit-exact run to run.
constexpr int kPlanMaxG = 256;
constexpr int kPlanMaxS = 256;

// One wave ranks tokens [t0, t0 + 64) for groups [g0, g0 + win) (win <= 64):
// cnt[g * cs] / acnt[g * cs] get the chunk's kept / positive-weight counts,
// tokrow the rank of each kept entry among the chunk's earlier tokens and -1
// for every other entry (the g0 == 0 wave writes the padding entries).
// acnt is only counted when drop == 0 (otherwise it equals cnt).
template <typename P>
__device__ __forceinline__ void rank_chunk(const int32_t* __restrict__ tok_g,
                                           const float* __restrict__ tok_w, int N, int S, int G,
                                           int drop, int t0, int g0, int win, P cnt, P acnt,
                                           int cs, int32_t* __restrict__ tokrow) {
  const int lane = threadIdx.x & 63;
  const int t = t0 + lane;
  const bool valid = t < N;
  const int nb = G - g0 < win ? G - g0 : win;
  const int64_t e0 = static_cast<int64_t>(t) * S;
  uint64_t gm = 0, km = 0, am = 0;
  int below = 0;  // valid entries with a group < g0
  if (valid) {
    int prev = -1;
    bool open = true;
    for (int j0 = 0; j0 < S; j0 += 8) {
      int gv[8];
      float wv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {  // unconditional (clamped) loads: issued together
        const int jj = j0 + u < S ? j0 + u : S - 1;
        gv[u] = tok_g[e0 + jj];
        wv[u] = tok_w[e0 + jj];
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) gv[u] = j0 + u < S ? gv[u] : -1;
#pragma unroll
      for (int u = 0; u < 8; ++u) {  // branch-free, so no load is sunk behind a branch
        const int g = gv[u];
        open = open && g > prev && g < G;  // g > prev >= -1, so g >= 0
        prev = open ? g : prev;
        below += (open && g < g0) ? 1 : 0;
        const int b = g - g0;
        const uint64_t bit = (open && b >= 0 && b < nb) ? (1ull << (b & 63)) : 0ull;
        const bool pos = wv[u] > 0.f;
        gm |= bit;
        km |= (!drop || pos) ? bit : 0ull;
        am |= pos ? bit : 0ull;
        if (!open && g0 == 0 && j0 + u < S) tokrow[e0 + j0 + u] = -1;
      }
    }
  }
  int mycnt = 0, myacnt = 0;
  for (int b = 0; b < nb; ++b) {
    const uint64_t bit = 1ull << b;
    const uint64_t m = __ballot((km & bit) != 0);
    mycnt = lane == b ? static_cast<int>(__popcll(m)) : mycnt;
    if (!drop) {
      const uint64_t ma = __ballot((am & bit) != 0);
      myacnt = lane == b ? static_cast<int>(__popcll(ma)) : myacnt;
    }
    if (gm & bit) {
      const int j = below + static_cast<int>(__popcll(gm & (bit - 1)));
      const int r = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                              __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0));
      tokrow[e0 + j] = (km & bit) ? r : -1;
    }
  }
  if (lane < nb) {
    cnt[(g0 + lane) * cs] = mycnt;
    acnt[(g0 + lane) * cs] = drop ? mycnt : myacnt;
  }
}

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
  int incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int u = __shfl_up(incl, o);
    if (lane >= o) incl += u;
  }
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
  const int chunk = item / W, g0 = (item % W) * 64;
  rank_chunk(tok_g, tok_w, N, S, G, drop, chunk * 64, g0, 64, ccnt + chunk, cacnt + chunk, C,
             tokrow);
}

// One wave per group: chunk counts -> exclusive chunk prefixes (in place),
// group totals -> cnt, positive-weight totals -> acnt.
__global__ __launch_bounds__(64) void k_plan_scan(int C, int32_t* __restrict__ ccnt,
                                                  const int32_t* __restrict__ cacnt,
                                                  int32_t* __restrict__ cnt,
                                                  int32_t* __restrict__ acnt) {
  const int g = blockIdx.x, lane = threadIdx.x;
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
    int incl = s;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int u = __shfl_up(incl, o);
      if (lane >= o) incl += u;
    }
    int p = run + incl - s;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int c = c0 + lane * 4 + k;
      if (c < C) row[c] = p;
      p += v[k];
    }
    run += __shfl(incl, 63);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) a += __shfl_xor(a, o);
  if (lane == 0) {
    cnt[g] = run;
    acnt[g] = a;
  }
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
__global__ __launch_bounds__(1024) void k_plan_small(const int32_t* __restrict__ tok_g,
                                                     const float* __restrict__ tok_w, int N,
                                                     int S, int G, int drop, int win,
                                                     int32_t* __restrict__ cnt,
                                                     int32_t* __restrict__ acnt,
                                                     int32_t* __restrict__ off,
                                                     int32_t* __restrict__ rows,
                                                     float* __restrict__ roww,
                                                     int32_t* __restrict__ tokrow) {
  __shared__ int cc[kSmallMaxCells], ca[kSmallMaxCells];
  __shared__ int tot[kPlanMaxG], goff[kPlanMaxG + 1], wsum[4];
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
    int incl = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int u = __shfl_up(incl, o);
      if (lane >= o) incl += u;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) a += __shfl_xor(a, o);
    if (lane < C) cc[g * C + lane] = incl - v;
    if (lane == 63) {
      tot[g] = incl;
      cnt[g] = incl;
      acnt[g] = a;
    }
  }
  __syncthreads();
  block_group_offsets(tot, G, goff, wsum);
  for (int g = threadIdx.x; g <= G; g += 1024) off[g] = goff[g];
  for (int t = threadIdx.x; t < N; t += 1024)
    scatter_token(tok_g, tok_w, t, S, G, cc + (t >> 6), C, goff, rows, roww, tokrow);
}

size_t plan_scratch_bytes(int N, int G) {
  const size_t C = (static_cast<size_t>(N > 0 ? N : 1) + 63) / 64;
  return 2 * C * static_cast<size_t>(G) * sizeof(int32_t);
}

int launch_plan(const int32_t* tok_g, const float* tok_w, int N, int S, int G, int drop,
                int32_t* cnt, int32_t* acnt, int32_t* off, int32_t* rows, float* roww,
                int32_t* tokrow, void* scratch, hipStream_t s) {
  if (G < 1 || G > kPlanMaxG || S < 1 || S > kPlanMaxS || N < 0) return SMOE_EINVAL;
  const int C = (N + 63) / 64;
  // One workgroup while its rank work (C x G ballots) stays small; the
  // three-kernel form spreads larger plans over the chip.
  if (C * G <= 512) {
    int win = 64;  // narrower windows until the 16 waves have work
    while (win > 8 && C * ((G + win - 1) / win) < 16) win >>= 1;
    hipLaunchKernelGGL(k_plan_small, dim3(1), dim3(1024), 0, s, tok_g, tok_w, N, S, G, drop, win,
                       cnt, acnt, off, rows, roww, tokrow);
    return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
  }
  const int W = (G + 63) / 64;
  int32_t* ccnt = reinterpret_cast<int32_t*>(scratch);
  int32_t* cacnt = ccnt + static_cast<int64_t>(C) * G;
  hipLaunchKernelGGL(k_plan_rank, dim3((C * W + 3) / 4), dim3(256), 0, s, tok_g, tok_w, N, S, G,
                     drop, C, W, ccnt, cacnt, tokrow);
  hipLaunchKernelGGL(k_plan_scan, dim3(G), dim3(64), 0, s, C, ccnt, cacnt, cnt, acnt);
  hipLaunchKernelGGL(k_plan_scatter, dim3((N + 255) / 256), dim3(256), 0, s, tok_g, tok_w, N, S,
                     G, C, ccnt, cnt, off, rows, roww, tokrow);
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
