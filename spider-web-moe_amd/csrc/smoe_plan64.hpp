// One-wave dispatch plans of decode steps (<= 64 tokens, <= 64 groups),
// shared by the routing kernels and the decode edge projection, which runs
// a decode loop's plans in one of its workgroups.
#pragma once
#include "smoe_common.hpp"
#include "smoe_internal.hpp"

namespace smoe {

// Plan of <= 64 tokens over <= 64 groups by one wave, lane t = token t
// (tok_g, tok_w and tokrow in LDS or global memory): each valid entry sets bit t of its
// group's token masks (kept, positive weight) by an LDS atomic OR; lane g
// counts group g by popcount and a wave scan gives the offsets; a kept
// entry's row is off[g] + the number of earlier tokens in its group's mask.
// The plan the multi-wave forms write (stable token order, tokrow -1 for
// every entry not kept), in one wave and without a workgroup barrier: the
// wave's LDS operations complete in order.  km / am: 64 words of LDS each;
// soff: 64.
__device__ __forceinline__ void plan64_wave(const int32_t* tok_g, const float* tok_w, int N, int S,
                                            int G, int drop, int32_t* __restrict__ cnt,
                                            int32_t* __restrict__ acnt, int32_t* __restrict__ off,
                                            int32_t* __restrict__ rows, float* __restrict__ roww,
                                            int32_t* tokrow, uint64_t* km, uint64_t* am,
                                            int* soff) {
  const int t = threadIdx.x & 63;
  const bool tv = t < N;
  km[t] = 0ull;
  am[t] = 0ull;
  const uint64_t bit = 1ull << t, below = bit - 1ull;
  int prev = -1;
  bool open = tv;
  for (int j = 0; j < S; ++j) {
    const int g = tv ? tok_g[t * S + j] : -1;
    const float w = tv ? tok_w[t * S + j] : 0.f;
    open = open && g > prev && g < G;  // g > prev >= -1, so g >= 0
    prev = open ? g : prev;
    if (open && (!drop || w > 0.f)) atomicOr(&km[g], bit);
    if (open && !drop && w > 0.f) atomicOr(&am[g], bit);
  }
  const int gl = t < G ? t : 0;
  const int c = t < G ? __popcll(km[gl]) : 0;
  const int a = t < G ? (drop ? c : __popcll(am[gl])) : 0;
  const int incl = wave_incl_scan(c);
  if (t < G) {
    cnt[t] = c;
    acnt[t] = a;
    off[t] = incl - c;
    soff[t] = incl - c;
  }
  if (t == 0) off[G] = __builtin_amdgcn_readlane(incl, 63);
  prev = -1;
  open = tv;
  for (int j = 0; j < S; ++j) {
    const int g = tv ? tok_g[t * S + j] : -1;
    const float w = tv ? tok_w[t * S + j] : 0.f;
    open = open && g > prev && g < G;
    prev = open ? g : prev;
    const bool kept = open && (!drop || w > 0.f);
    const int gc = kept ? g : 0;
    const int row = soff[gc] + __popcll(km[gc] & below);
    if (tv) tokrow[t * S + j] = kept ? row : -1;
    if (kept) {
      rows[row] = t;
      roww[row] = w;
    }
  }
}

// The plans of a decode loop (N <= 64 tokens, S <= 16 destinations per
// token), from the front's top-k and per-source top-m; KB >= K and KMB >=
// K * M (compile-time bounds).  Two waves that share no data, lane t = token
// t: wave 0 sorts each token's top-k by expert (tok_e / tok_ew), builds the
// expert plan (plan64_wave) and puts each source's edges at its plan row;
// wave 1 sums each token's destination coefficients over its sources in
// ascending order (the order topm_seg adds them), lists them ascending
// (tok_d / tok_dc) and builds the destination plan.  Threads past the first
// 128 return at once; no workgroup barrier.  lds: decode_plan_lds_bytes<KB>().
constexpr int kDecMaxS = 16;
template <int KB>
constexpr int decode_plan_lds_bytes() {
  return 2 * 64 * 8 * 2 + 2 * 64 * 4 + 3 * kFrontMaxN * KB * 4 + kFrontMaxN * 65 * 4 +
         3 * kFrontMaxN * kDecMaxS * 4;
}
template <int KB, int KMB>
__device__ __forceinline__ void decode_plan_body(const DecPlan& q, uint8_t* lds) {
  uint64_t* s_km = reinterpret_cast<uint64_t*>(lds);        // [2][64]
  uint64_t* s_am = s_km + 2 * 64;                            // [2][64]
  int* s_off = reinterpret_cast<int*>(s_am + 2 * 64);        // [2][64]
  int32_t* s_te = s_off + 2 * 64;                            // [64 * KB]
  int32_t* s_etr = s_te + kFrontMaxN * KB;
  float* s_tw = reinterpret_cast<float*>(s_etr + kFrontMaxN * KB);
  float* s_c = s_tw + kFrontMaxN * KB;                       // [64][65]
  int32_t* s_td = reinterpret_cast<int32_t*>(s_c + kFrontMaxN * 65);  // [64 * 16]
  int32_t* s_dtr = s_td + kFrontMaxN * kDecMaxS;
  float* s_tc = reinterpret_cast<float*>(s_dtr + kFrontMaxN * kDecMaxS);
  if (threadIdx.x >= 128) return;
  const int t = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int N = q.N, E = q.E, K = q.K, M = q.M, S = q.S;
  const bool tv = t < N;
  const int tc = tv ? t : 0;
  const int km = K * M;
  const bool live = !q.active || q.active[tc] != 0;  // a token out of orbit: no sources
  if (wave == 0) {
    // the token's top-k sorted by expert (ids are distinct: rank = # smaller),
    // its sources' edges (in that order already) loaded alongside
    int ti[KB], ei[KMB];
    float tw[KB], ew[KMB];
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      const int jj = j < K ? j : K - 1;
      ti[j] = q.top_idx[tc * K + jj];
      tw[j] = q.top_w[tc * K + jj];
    }
#pragma unroll
    for (int u = 0; u < KMB; ++u) {
      const int uu = u < km ? u : km - 1;
      ei[u] = q.sel_idx[tc * km + uu];
      ew[u] = q.sel_w[tc * km + uu];
    }
    if (tv && live)
#pragma unroll
      for (int j = 0; j < KB; ++j) {
        if (j >= K) break;
        int rank = 0;
#pragma unroll
        for (int i = 0; i < KB; ++i) rank += (i < K && ti[i] < ti[j]) ? 1 : 0;
        s_te[t * K + rank] = ti[j];
        s_tw[t * K + rank] = tw[j];
        q.tok_e[t * K + rank] = ti[j];
        q.tok_ew[t * K + rank] = tw[j];
      }
    else if (tv)
      for (int j = 0; j < K; ++j) {
        s_te[t * K + j] = -1;
        s_tw[t * K + j] = 0.f;
        q.tok_e[t * K + j] = -1;
        q.tok_ew[t * K + j] = 0.f;
      }
    plan64_wave(s_te, s_tw, N, K, E, 0, q.e_cnt, q.e_acnt, q.e_off, q.e_rows, q.e_roww, s_etr,
                s_km, s_am, s_off);
    if (tv)
#pragma unroll
      for (int u = 0; u < KMB; ++u) {
        if (u >= km) break;
        const int j = u / M, i = u - j * M;
        const int row = s_etr[t * K + j];
        if (i == 0) q.e_tokrow[t * K + j] = row;
        if (row >= 0) {
          q.edge_idx[static_cast<int64_t>(row) * M + i] = ei[u];
          q.edge_w[static_cast<int64_t>(row) * M + i] = ew[u];
        }
      }
  } else {
    // destination coefficients: sum over the sources in ascending order
    int ei[KMB];
    float ew[KMB];
#pragma unroll
    for (int u = 0; u < KMB; ++u) {
      const int uu = u < km ? u : km - 1;
      ei[u] = q.sel_idx[tc * km + uu];
      ew[u] = q.sel_w[tc * km + uu];
    }
    float* crow = s_c + tc * 65;
    if (tv) {
      for (int d = 0; d < E; ++d) crow[d] = 0.f;
#pragma unroll
      for (int u = 0; u < KMB; ++u)
        if (u < km && live) crow[ei[u]] += ew[u];
      int cnt = 0;
      for (int d = 0; d < E; ++d) {
        const float c = crow[d];
        if (c != 0.f) {
          s_td[t * S + cnt] = d;
          s_tc[t * S + cnt] = c;
          ++cnt;
        }
      }
      for (int j = cnt; j < S; ++j) {
        s_td[t * S + j] = -1;
        s_tc[t * S + j] = 0.f;
      }
      for (int j = 0; j < S; ++j) {
        q.tok_d[t * S + j] = s_td[t * S + j];
        q.tok_dc[t * S + j] = s_tc[t * S + j];
      }
    }
    plan64_wave(s_td, s_tc, N, S, E, 1, q.d_cnt, q.d_acnt, q.d_off, q.d_rows, q.d_roww, s_dtr,
                s_km + 64, s_am + 64, s_off + 64);
    if (tv)
      for (int j = 0; j < S; ++j) q.d_tokrow[t * S + j] = s_dtr[t * S + j];
  }
}

}  // namespace smoe
