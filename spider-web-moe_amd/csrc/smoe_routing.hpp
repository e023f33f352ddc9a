// Per-token routing and the plan's per-chunk ranks as device functions:
// the routing kernels (smoe_route.hip) and the one-pass prefill front
// (smoe_front.hip) share them, so every path selects and ranks with the same
// operations.
#pragma once

#include "smoe_common.hpp"
#include "smoe_internal.hpp"

namespace smoe {

constexpr int kBig = 1 << 20;

// ------------------------------------------------------------ router ----
// Segment of token t (lane e of the segment: expert e, logit v, -inf past
// E); tokens with !ok compute but store nothing.  tok_e2 / tok_ew2 (may be
// null) receive a second copy of tok_e / tok_ew (indexed t2 * K + slot; t2
// defaults to t).
// The K loop stays rolled: unrolled copies overflow the instruction cache of
// the single-workgroup front, which runs each instruction a few times only.
// p of the selected expert is recomputed from its logit (the same ops on the
// same value as p itself).
// live == false (a token that has left the orbit under an exit gate): the
// token's tok_e / tok_ew slots are all -1 / 0, so every plan, the edge
// stages and the expert GEMMs skip it; top_idx / top_w are still written.
// Returns the segment's mask of selected experts (bit e = expert e).
template <int SEG>
__device__ __forceinline__ uint64_t topk_seg(float v, int t, bool ok, bool live, int E, int K,
                                         int32_t* __restrict__ top_idx, float* __restrict__ top_w,
                                         int32_t* __restrict__ tok_e, float* __restrict__ tok_ew,
                                         int32_t* tok_e2, float* tok_ew2, int t2 = -1) {
  const int u2 = t2 >= 0 ? t2 : t;  // the token's index in the second copy
  const int lane = threadIdx.x & 63;
  const int e = lane & (SEG - 1), sbase = lane - e;
  const bool in = e < E;
  v = in ? v : -INFINITY;
  const float mx = seg_max<SEG>(v);
  const float ex = in ? expf(v - mx) : 0.f;
  const float sum = seg_sum<SEG>(ex);
  const float p = ex / sum;
  bool sel = false;
  float psum = 0.f, slot_p = 0.f;
  int slot_i = 0;
#pragma unroll 1
  for (int j = 0; j < K; ++j) {
    float cv = (in && !sel) ? v : -INFINITY;
    int ci = (in && !sel) ? e : kBig;
    seg_argmax<SEG>(cv, ci);
    const float pj = expf(cv - mx) / sum;
    sel = sel || e == ci;
    slot_p = e == j ? pj : slot_p;
    slot_i = e == j ? ci : slot_i;
    psum += pj;  // slot order, as torch sums the k values
  }
  const float denom = fmaxf(psum, 1e-9f);
  if (ok && e < K) {
    top_idx[static_cast<int64_t>(t) * K + e] = slot_i;
    top_w[static_cast<int64_t>(t) * K + e] = slot_p / denom;
  }
  // distinct experts of the token in ascending order (lane order)
  const uint64_t segm = SEG == 64 ? ~0ull : ((1ull << SEG) - 1);
  const uint64_t m = (__ballot(sel) >> sbase) & segm;
  if (!tok_e) return m;  // top-k only (the decode front: its plan kernel sorts the sources)
  if (ok && live && sel) {
    const int rank = __popcll(m & ((1ull << e) - 1));
    tok_e[static_cast<int64_t>(t) * K + rank] = e;
    tok_ew[static_cast<int64_t>(t) * K + rank] = p / denom;
    if (tok_e2) {
      tok_e2[u2 * K + rank] = e;
      tok_ew2[u2 * K + rank] = p / denom;
    }
  }
  if (ok && !live && e < K) {
    tok_e[static_cast<int64_t>(t) * K + e] = -1;
    tok_ew[static_cast<int64_t>(t) * K + e] = 0.f;
    if (tok_e2) {
      tok_e2[u2 * K + e] = -1;
      tok_ew2[u2 * K + e] = 0.f;
    }
  }
  return m;
}

// ------------------------------------------------------------- edges ----
// Segment of token t, lane d of the segment = destination d.  Source slot j
// of the token has logit v[j] (lane d: the logit of edge s_j -> d), plan
// row row[j] and is live when j < K and the slot holds a source (dead slots
// compute on garbage and store nothing; tokens with !ok store nothing).
// Writes top-m and softmax weights per source row (edge_idx / edge_w at the
// plan row) and the token's destination coefficients (tok_d / tok_dc, and a
// second copy in tok_d2 / tok_dc2 when not null, indexed t2 * S + slot; t2
// defaults to t).
template <int SEG, int KB>
__device__ __forceinline__ void topm_seg(const float (&v)[KB], const int (&row)[KB],
                                         const bool (&live)[KB], int t, bool ok, int E, int M,
                                         int S, int32_t* __restrict__ edge_idx,
                                         float* __restrict__ edge_w, int32_t* __restrict__ tok_d,
                                         float* __restrict__ tok_dc, int32_t* tok_d2,
                                         float* tok_dc2, int t2 = -1) {
  const int u2 = t2 >= 0 ? t2 : t;  // the token's index in the second copy
  const int lane = threadIdx.x & 63;
  const int d = lane & (SEG - 1), sbase = lane - d;
  const bool in = d < E;
  float c = 0.f;
#pragma unroll
  for (int j = 0; j < KB; ++j) {
    if (!__ballot(live[j])) continue;  // uniform (sources are packed first)
    const float vj = (in && live[j]) ? v[j] : -INFINITY;
    bool sel = false;
    float vmax = 0.f, den = 0.f, rec_v = 0.f;
    int rec_i = 0;
#pragma unroll 1
    for (int i = 0; i < M; ++i) {  // rolled, as the top-k loop
      float cv = (in && !sel) ? vj : -INFINITY;
      int ci = (in && !sel) ? d : kBig;
      seg_argmax<SEG>(cv, ci);
      sel = sel || d == ci;
      vmax = i == 0 ? cv : vmax;
      rec_v = d == i ? cv : rec_v;
      rec_i = d == i ? ci : rec_i;
      den += expf(cv - vmax);  // softmax over the m values, slot order
    }
    if (live[j]) {
      if (sel) c += expf(vj - vmax) / den;
      if (ok && d < M) {
        edge_idx[static_cast<int64_t>(row[j]) * M + d] = rec_i;
        edge_w[static_cast<int64_t>(row[j]) * M + d] = expf(rec_v - vmax) / den;
      }
    }
  }
  const bool nz = in && c != 0.f;
  const uint64_t segm = SEG == 64 ? ~0ull : ((1ull << SEG) - 1);
  const uint64_t m = (__ballot(nz) >> sbase) & segm;
  const int cnt = __popcll(m);
  if (ok && nz) {
    const int rank = __popcll(m & ((1ull << d) - 1));
    tok_d[static_cast<int64_t>(t) * S + rank] = d;
    tok_dc[static_cast<int64_t>(t) * S + rank] = c;
    if (tok_d2) {
      tok_d2[u2 * S + rank] = d;
      tok_dc2[u2 * S + rank] = c;
    }
  }
  if (ok && d >= cnt && d < S) {
    tok_d[static_cast<int64_t>(t) * S + d] = -1;
    tok_dc[static_cast<int64_t>(t) * S + d] = 0.f;
    if (tok_d2) {
      tok_d2[u2 * S + d] = -1;
      tok_dc2[u2 * S + d] = 0.f;
    }
  }
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
// acnt is only counted when drop == 0 (otherwise it equals cnt).  tsrc:
// token tsrc's entries sit at the start of tok_g / tok_w (a chunk's copy in
// LDS: tsrc = t0), tokrow is indexed by the token itself.
template <typename P>
__device__ __forceinline__ void rank_chunk(const int32_t* __restrict__ tok_g,
                                           const float* __restrict__ tok_w, int N, int S, int G,
                                           int drop, int t0, int g0, int win, P cnt, P acnt,
                                           int cs, int32_t* __restrict__ tokrow, int tsrc = 0) {
  const int lane = threadIdx.x & 63;
  const int t = t0 + lane;
  const bool valid = t < N;
  const int nb = G - g0 < win ? G - g0 : win;
  const int64_t e0 = static_cast<int64_t>(t) * S;
  const int64_t src0 = static_cast<int64_t>(tsrc) * S;
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
        gv[u] = tok_g[e0 - src0 + jj];
        wv[u] = tok_w[e0 - src0 + jj];
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

}  // namespace smoe
