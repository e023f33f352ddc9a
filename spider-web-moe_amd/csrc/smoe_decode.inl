// Decode loop kernels (bf16, N <= 64 tokens).  Included by smoe_route.hip,
// inside namespace smoe, after the routing device functions it uses
// (topk_seg, plan64_wave, seg_argmax).
//
// Decode steps spend most of a loop's time outside the weight streams when
// every routing stage is its own launch.  Here a loop takes one launch
// before its edge projection:
//
//  k_decode_front (strip, 8-token tile; 16 waves): the tile's input rows go
//   to LDS as bf16 — for loops after the first, as the previous loop's
//   LayerNorm (ln_row over h_{r-1}, x0 and the previous loop's expert rows,
//   the operations of k_epilogue in its order, so the rows are the bits that
//   kernel writes; the router strip stores them as the loop's input).  Wave
//   w < 8 normalises token w, so the latency chains overlap; the
//   LayerNorm's operands are requested first and the router rows and the
//   strip's own weights after them.  8-token tiles put twice the
//   workgroups of 16-token ones on the chip, each moving half the rows
//   (C2: 0.297 -> 0.290 ms per step; 4-token tiles 0.308).  One 16 x 16 x
//   32 MFMA per 32-k step and 16-channel tile (rows past the tile's tokens
//   are zeros), K split over the waves and added in wave order, + bias.  Every
//   strip then runs the router top-k of its tokens (topk_seg; the same bits
//   in every strip, since the logits are computed the same way); strip 0
//   writes it, strip s + 1 runs top-m over source s's logits (topm_row, the
//   operations of topm_seg) and, for each token that selected s, writes its
//   destinations and softmax weights at s's rank among the token's sources.
//
//  the plans (decode_plan_body: two waves that share no data): wave 0 sorts
//   each token's top-k by expert (tok_e / tok_ew), builds the expert plan
//   (plan64_wave) and puts each source's edges at its plan row; wave 1 sums
//   each token's destination coefficients over its sources in ascending
//   order (the order topm_seg adds them), lists them ascending (tok_d /
//   tok_dc) and builds the destination plan.  They run in one workgroup of
//   the edge projection (k_decode_edge), beside its weight streams, which
//   read the front's selections directly; k_decode_plan runs them alone
//   for the shapes k_decode_edge does not take.
//
// The previous loop's epilogue is folded into the next front, so a call
// ends with one k_epilogue after its last loop.

// Top-m of one source row over the E lanes of a segment (lane d: the logit
// of the edge to destination d): the operations of topm_seg for one live
// source; written, when `sel`, to sel_idx / sel_w [N, K, M] at (t, rank).
template <int SEG>
__device__ __forceinline__ void topm_row(float v, int t, bool ok, bool sel_src, int rank, int E,
                                         int K, int M, int32_t* __restrict__ sel_idx,
                                         float* __restrict__ sel_w) {
  const int lane = threadIdx.x & 63;
  const int d = lane & (SEG - 1);
  const bool in = d < E;
  const float vj = in ? v : -INFINITY;
  bool sel = false;
  float vmax = 0.f, den = 0.f, rec_v = 0.f;
  int rec_i = 0;
#pragma unroll 1
  for (int i = 0; i < M; ++i) {
    float cv = (in && !sel) ? vj : -INFINITY;
    int ci = (in && !sel) ? d : kBig;
    seg_argmax<SEG>(cv, ci);
    sel = sel || d == ci;
    vmax = i == 0 ? cv : vmax;
    rec_v = d == i ? cv : rec_v;
    rec_i = d == i ? ci : rec_i;
    den += expf(cv - vmax);
  }
  if (ok && sel_src && d < M) {
    const int64_t o = (static_cast<int64_t>(t) * K + rank) * M + d;
    sel_idx[o] = rec_i;
    sel_w[o] = expf(rec_v - vmax) / den;
  }
}

constexpr int kFrontTile = 8;  // tokens per workgroup of k_decode_front
// CPL: row chunks per lane (H); SEG: lanes per token (E); ET: 16-channel
// tiles of E; NS: H / 128; PRO: the input rows are the previous loop's
// LayerNorm.
template <int CPL, int SEG, int ET, int NS, bool PRO>
__global__ __launch_bounds__(1024) void k_decode_front(const DecFront a) {
  constexpr int TT = kFrontTile;            // tokens per tile (one per wave of the first TT)
  constexpr int TR = 16;                    // MFMA rows (tokens past TT: zero rows)
  constexpr int NW = 16;                    // waves
  constexpr int H = NS * 128;
  constexpr int KST = H / 32;               // 32-k steps
  constexpr int NSW = (KST + NW - 1) / NW;  // steps per wave (the last may be short)
  constexpr int LDX = H + 8;                // LDS row pitch (bf16): 16-byte reads conflict-free
  constexpr int LTW = ET * 16 + 1;
  constexpr int XA_BYTES = TR * LDX * 2, RED_BYTES = NW * 2 * ET * 64 * 16;
  // the input rows, then (once every wave's MFMAs are done) the waves' partials
  __shared__ __attribute__((aligned(16))) uint8_t smem[XA_BYTES > RED_BYTES ? XA_BYTES : RED_BYTES];
  __shared__ float lt[2][TR][LTW];          // [router | the strip's source] logits
  uint16_t* xa = reinterpret_cast<uint16_t*>(smem);
  f32x4* red = reinterpret_cast<f32x4*>(smem);  // [NW][2 ET][64]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = lane >> 4, l16 = lane & 15;
  const int strip = blockIdx.x, t0 = blockIdx.y * TT;
  const bool src = strip > 0;
  const int E = a.E, N = a.N;
  // 1 what the LayerNorm of token `wave` waits on goes out first: the
  // token's expert rows' indices, its h and x0 rows, and this thread's share
  // of the LayerNorm parameters (one element per thread, shared through LDS:
  // every wave normalises with the same ones).  The weight fragments follow,
  // so a wait for the token's operands does not wait for them (vmcnt counts
  // in issue order).
  __shared__ float lnp[PRO ? 2 * H : 1];
  __shared__ int s_live[TT];  // the tile's tokens in orbit for this loop (the gate's)
  const int j = wave;
  const int t = t0 + j;
  const bool tv = j < TT && t < N;  // wave-uniform
  // the gate: whether the token is in orbit on entry, its loop count, and
  // (PRO with exit_wb) the exit head weights, all requested first
  const bool gate = a.active != nullptr;
  const bool gate_here = PRO && gate && a.exit_wb != nullptr;
  int live_in = 1, loops_in = 0;
  if (gate && tv) {
    live_in = a.active[t];
    if (gate_here && a.loops) loops_in = a.loops[t];
  }
  float ewv[PRO ? CPL : 1][8];
  float hv[CPL][8], xv[CPL][8];
  int te = -1, tr = 0;
  float tw = 0.f, pw = 1.f, pb = 0.f;
  if constexpr (PRO) {
    const int pi = threadIdx.x < H ? threadIdx.x : 0;
    if (a.ln_w) pw = a.ln_w[pi];
    if (a.ln_b) pb = a.ln_b[pi];
    const int tc = tv ? t : 0;  // rows past N: token 0's (never stored)
    const int64_t e = static_cast<int64_t>(tc) * a.K + (lane < a.K ? lane : a.K - 1);
    te = a.tok_e[e];
    tw = a.tok_ew[e];
    tr = a.e_tokrow[e];
#pragma unroll
    for (int c = 0; c < CPL; ++c) {  // columns past H load column 0 (not stored)
      const int col = (lane + 64 * c) * 8;
      const int64_t o = static_cast<int64_t>(tc) * H + (col < H ? col : 0);
      load8<SMOE_BF16>(a.h, o, hv[c]);
      load8<SMOE_BF16>(a.x0, o, xv[c]);
    }
    if (gate_here)
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const int col = (lane + 64 * c) * 8;
        load8<SMOE_F32>(a.exit_wb, col < H ? col : 0, ewv[c]);
      }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  }
  // 2 weight fragments (lane: row l16 of tile ct, k 8q.. of step wave +
  // 16 st): the router's, and (strips > 0) the source's E edge rows; rows
  // past E read row E - 1 (never stored), steps past the last read step 0
  // (not multiplied)
  const uint16_t* rw = reinterpret_cast<const uint16_t*>(a.router_w);
  const uint16_t* sw = reinterpret_cast<const uint16_t*>(a.edge_w) +
                       static_cast<int64_t>(src ? strip - 1 : 0) * E * a.ldw;
  u32x4 wr[NSW][ET], ws[NSW][ET];
#pragma unroll
  for (int ct = 0; ct < ET; ++ct) {
    const int row = min(16 * ct + l16, E - 1);
#pragma unroll
    for (int st = 0; st < NSW; ++st) {
      const int k = wave + NW * st;
      const int kk = 32 * (k < KST ? k : 0) + 8 * q;
      wr[st][ct] = *reinterpret_cast<const u32x4*>(rw + static_cast<int64_t>(row) * H + kk);
      if (src)
        ws[st][ct] = *reinterpret_cast<const u32x4*>(sw + static_cast<int64_t>(row) * a.ldw + kk);
      else
        ws[st][ct] = u32x4{0u, 0u, 0u, 0u};
    }
  }
  // 3 token `wave` of the tile -> LDS (bf16); rows past N are zeros
  int live = live_in;  // in orbit for this loop's routing (after the gate)
  {
    float o[CPL][8];
#pragma unroll
    for (int c = 0; c < CPL; ++c)
#pragma unroll
      for (int i = 0; i < 8; ++i) o[c][i] = 0.f;
    if constexpr (PRO) {
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      if (threadIdx.x < H) {
        lnp[threadIdx.x] = pw;
        lnp[H + threadIdx.x] = pb;
      }
      if (tv && live_in) {  // the previous loop's expert rows, then its epilogue's LayerNorm
        const int my_row = (lane < a.K && te >= 0 && tw > 0.f) ? tr : -1;
        gather_add<CPL, SMOE_BF16>(a.y, H, my_row, __ballot(my_row >= 0), o);
      }
      __syncthreads();  // the LayerNorm parameters are in LDS
      if (tv && !live_in) {  // out of orbit: h passes through (k_epilogue's gate)
#pragma unroll
        for (int c = 0; c < CPL; ++c)
#pragma unroll
          for (int i = 0; i < 8; ++i) o[c][i] = hv[c][i];
      } else if (tv) {
        float gw[CPL][8], gb[CPL][8];
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
          const int col = (lane + 64 * c) * 8;
          const int cc = col < H ? col : 0;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            gw[c][i] = lnp[cc + i];
            gb[c][i] = lnp[H + cc + i];
          }
        }
        ln_row<CPL>(hv, xv, gw, gb, o, H, a.alpha, a.beta, a.eps, o);  // in place
        if (gate_here) {  // k_epilogue's exit decision on the stored (bf16) row
          float g = 0.f;
#pragma unroll
          for (int c = 0; c < CPL; ++c) {
            const int col = (lane + 64 * c) * 8;
            if (col < H)
#pragma unroll
              for (int i = 0; i < 8; ++i) g += bf2f(f2bf(o[c][i])) * ewv[c][i];
          }
          // a bf16 model's exit_head is a bf16 Linear: its output (the logit)
          // is rounded to bf16 before the fp32 sigmoid (model.py:467)
          const float z = bf2f(f2bf(wave_sum(g) + a.exit_wb[H]));
          const bool out = 1.0f / (1.0f + expf(-z)) > a.threshold;
          live = out ? 0 : 1;
          if (strip == 0 && lane == 0) {
            if (out) a.active[t] = 0;
            if (a.loops) a.loops[t] = loops_in + 1;
          }
        }
      }
    } else if (tv) {
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const int col = (lane + 64 * c) * 8;
        load8<SMOE_BF16>(a.h, static_cast<int64_t>(t) * H + (col < H ? col : 0), o[c]);
      }
    }
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int col = (lane + 64 * c) * 8;
      if (col < H) {
        u32x4 pk;
#pragma unroll
        for (int i = 0; i < 4; ++i) pk[i] = pack_bf2(o[c][2 * i], o[c][2 * i + 1]);
        *reinterpret_cast<u32x4*>(xa + j * LDX + col) = pk;
        if (PRO && strip == 0 && tv)
          *reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(a.h_out) +
                                    static_cast<int64_t>(t) * H + col) = pk;
      }
    }
  }
  if (j < TT && lane == 0) s_live[j] = live;
  lds_barrier();
  // 3 logits: this wave's k steps, then the waves' partials in wave order
  f32x4 acc[2 * ET];
#pragma unroll
  for (int c = 0; c < 2 * ET; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int st = 0; st < NSW; ++st) {
    const int k = wave + NW * st;
    if (k < KST) {  // wave-uniform
      const u32x4 b = *reinterpret_cast<const u32x4*>(xa + l16 * LDX + 32 * k + 8 * q);
#pragma unroll
      for (int ct = 0; ct < ET; ++ct) {
        acc[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wr[st][ct]),
                                                          __builtin_bit_cast(bf16x8, b), acc[ct],
                                                          0, 0, 0);
        if (src)
          acc[ET + ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8, ws[st][ct]), __builtin_bit_cast(bf16x8, b), acc[ET + ct],
              0, 0, 0);
      }
    }
  }
  lds_barrier();  // every wave's reads of the rows are done: `red` reuses them
#pragma unroll
  for (int c = 0; c < 2 * ET; ++c) red[(wave * 2 * ET + c) * 64 + lane] = acc[c];
  lds_barrier();
  if (wave < 2 * ET && (src || wave < ET)) {  // tile `wave`: channels 4q.. of token l16
    const int seg = wave / ET, ct = wave % ET;  // seg 0 router, 1 the source
    f32x4 s = red[wave * 64 + lane];
#pragma unroll
    for (int w = 1; w < NW; ++w) s += red[(w * 2 * ET + wave) * 64 + lane];
    const float* bias = seg == 0 ? a.router_bias : a.edge_bias + (strip - 1) * E;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ch = 16 * ct + 4 * q + i;
      if (ch < E) lt[seg][l16][ch] = s[i] + bias[ch];
    }
  }
  lds_barrier();
  // 4 per token: a segment of SEG lanes, lane e = channel e
  constexpr int TPW = 64 / SEG;
  const int e = lane & (SEG - 1);
  if (wave * TPW < TT) {  // wave-uniform: waves past the tile's tokens are done
    const int j = wave * TPW + lane / SEG;
    const int t = t0 + j;
    const bool ok = t < N;
    const int ec = e < E ? e : 0;
    const float v = lt[0][j][ec];
    const bool live_t = s_live[j] != 0;
    uint64_t m = topk_seg<SEG>(v, t, ok && !src, live_t, E, a.K, a.top_idx, a.top_w, nullptr,
                               nullptr, nullptr, nullptr);
    if (!live_t) m = 0;  // out of orbit: no sources, so no strip writes its edges
    if (!src) {
      if (ok && e < E) a.logits[static_cast<int64_t>(t) * E + e] = v;
      if (ok && !live_t)  // its selections select nothing (c[t, g] = 0 for every g)
        for (int u = e; u < a.K * a.M; u += SEG) {
          a.sel_idx[static_cast<int64_t>(t) * a.K * a.M + u] = 0;
          a.sel_w[static_cast<int64_t>(t) * a.K * a.M + u] = 0.f;
        }
    } else {
      const int s = strip - 1;
      const bool sel_src = (m >> s) & 1ull;
      const int rank = __popcll(m & ((1ull << s) - 1ull));
      topm_row<SEG>(lt[1][j][ec], t, ok, sel_src, rank, E, a.K, a.M, a.sel_idx, a.sel_w);
    }
  }
}

bool decode_front_fits(int N, int H, int E, int K, int M, int S, int ldw) {
  return N >= 1 && N <= kFrontMaxN && E >= 1 && E <= 64 && K >= 1 && K <= 16 && K <= E &&
         M >= 1 && M <= 16 && M <= E && K * M <= 64 && S >= 1 && S <= 16 && H >= 128 &&
         H <= 1024 && H % 128 == 0 && ldw >= H && ldw % 8 == 0;  // H > 1024: the rows spill
}

namespace {
template <int CPL, int NS, bool PRO>
int decode_front_e(const DecFront& a, hipStream_t s) {
  const dim3 grid(a.E + 1, (a.N + kFrontTile - 1) / kFrontTile), block(1024);
  const int et = (a.E + 15) / 16;
#define SMOE_DFRONT(SG, ET_)                                                              \
  do {                                                                                    \
    SMOE_LAUNCH((k_decode_front<CPL, SG, ET_, NS, PRO>), grid, block, 0, s, a);           \
    return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;                         \
  } while (0)
  switch (et) {
    case 1: SMOE_DFRONT(16, 1);
    case 2: SMOE_DFRONT(32, 2);
    case 3: SMOE_DFRONT(64, 3);
    case 4: SMOE_DFRONT(64, 4);
    default: return SMOE_EINVAL;
  }
#undef SMOE_DFRONT
}
template <bool PRO>
int decode_front_h(const DecFront& a, hipStream_t s) {
  switch (a.H) {
    case 128: return decode_front_e<1, 1, PRO>(a, s);
    case 256: return decode_front_e<1, 2, PRO>(a, s);
    case 384: return decode_front_e<1, 3, PRO>(a, s);
    case 512: return decode_front_e<1, 4, PRO>(a, s);
    case 640: return decode_front_e<2, 5, PRO>(a, s);
    case 768: return decode_front_e<2, 6, PRO>(a, s);
    case 896: return decode_front_e<2, 7, PRO>(a, s);
    case 1024: return decode_front_e<2, 8, PRO>(a, s);
    default: return SMOE_EINVAL;
  }
}
}  // namespace

int launch_decode_front(const DecFront& a, hipStream_t s) {
  const int S = a.E < a.K * a.M ? a.E : a.K * a.M;
  if (!decode_front_fits(a.N, a.H, a.E, a.K, a.M, S, a.ldw)) return SMOE_EINVAL;
  if (!a.h || !a.router_w || !a.edge_w || !a.router_bias || !a.edge_bias || !a.logits ||
      !a.top_idx || !a.top_w || !a.sel_idx || !a.sel_w)
    return SMOE_EINVAL;
  if (a.y) {
    if (!a.x0 || !a.tok_e || !a.tok_ew || !a.e_tokrow || !a.h_out) return SMOE_EINVAL;
    return decode_front_h<true>(a, s);
  }
  return decode_front_h<false>(a, s);
}

// Plans of a decode loop in one workgroup of their own (decode_plan_body).
template <int KB, int KMB>
__global__ __launch_bounds__(128) void k_decode_plan(const DecPlan q) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[decode_plan_lds_bytes<KB>()];
  decode_plan_body<KB, KMB>(q, lds);
}

bool decode_plan_fits(const DecPlan& q) {
  const int N = q.N, E = q.E, K = q.K, M = q.M, S = q.S;
  return N >= 1 && N <= kFrontMaxN && E >= 1 && E <= 64 && K >= 1 && K <= 16 && K <= E &&
         M >= 1 && M <= E && M <= 16 && S >= 1 && S <= kDecMaxS &&
         S == (E < K * M ? E : K * M) && K * M <= 64;
}

int launch_decode_plan(const DecPlan& q, hipStream_t s) {
  if (!decode_plan_fits(q)) return SMOE_EINVAL;
  const int K = q.K, km = q.K * q.M;
#define SMOE_DPLAN(KB_, KMB_) \
  hipLaunchKernelGGL((k_decode_plan<KB_, KMB_>), dim3(1), dim3(128), 0, s, q)
  if (K <= 2 && km <= 4) SMOE_DPLAN(2, 4);
  else if (K <= 2 && km <= 8) SMOE_DPLAN(2, 8);
  else if (K <= 4 && km <= 8) SMOE_DPLAN(4, 8);
  else if (K <= 4 && km <= 16) SMOE_DPLAN(4, 16);
  else if (K <= 8 && km <= 32) SMOE_DPLAN(8, 32);
  else SMOE_DPLAN(16, 64);
#undef SMOE_DPLAN
  return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
}
