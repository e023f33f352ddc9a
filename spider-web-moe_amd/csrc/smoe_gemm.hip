// Grouped GEMMs of the Spider-MoE block on gfx950.
//
//   C[row, n] = sum_k A[a_row(row), k] * W_g[n, k]      (row in group g)
//
// Rows are the entries of a dispatch plan (tokens sorted by expert or by
// edge destination; group g owns rows [grp_off[g], grp_off[g+1])).  A rows
// are gathered through a_rows, W_g is group g's [N_out, K] nn.Linear weight
// (K contiguous), so both MFMA operands load as 16-byte K-runs.
//
// bf16 / fp8 / int4 weights: bf16 MFMA (v_mfma_f32_16x16x32_bf16), fp32
// accumulate.  fp8-e4m3 codes are widened to bf16 exactly on the way into
// LDS and their per-output-channel scale is applied in the epilogue; int4
// nibbles are dequantized (q * group scale, fp32, rounded once to bf16) on
// the way into LDS.  fp32 weights (fp32 models) use a VALU fp32 tile kernel.
//
// Tiles: one workgroup computes BM plan rows x BN output channels; the grid
// is sized for the worst case (sum of ceil(rows_g / BM) <= ceil(R / BM) + G)
// and workgroups past the real tile count exit at once, so no host ever
// reads the routing.  Operands stream through double-buffered LDS with a
// register prefetch of the next K slice.
#include <type_traits>

#include "smoe_common.hpp"
#include "smoe_internal.hpp"
#include "smoe_plan64.hpp"

namespace smoe {

// Tile lookups over the plan's groups, wave-parallel: lane i holds group
// b + i of a 64-group chunk (offsets by one clamped load per lane), the
// per-group tile counts are prefix-summed by DPP, and the group holding a
// tile is the first lane whose inclusive count exceeds it (a ballot).  A
// serial loop over the groups would wait on one scalar load per group at the
// start of every workgroup.  Every lane of the wave must be active; the
// results are wave-uniform.
__device__ __forceinline__ void group_chunk(const GemmArgs& p, int BM, int b, int& lo, int& hi,
                                            int& t) {
  const int i = b + static_cast<int>(threadIdx.x & 63);
  const int ic = i < p.G ? i : p.G - 1;
  lo = p.grp_off[ic];
  hi = p.grp_off[ic + 1];
  t = i < p.G ? (hi - lo + BM - 1) / BM : 0;
}

// Number of BM-row tiles over all groups.
__device__ __forceinline__ int count_tiles(const GemmArgs& p, int BM) {
  if (p.G == 0) return (p.single_rows + BM - 1) / BM;
  int total = 0;
  for (int b = 0; b < p.G; b += 64) {
    int lo, hi, t;
    group_chunk(p, BM, b, lo, hi, t);
    total += __builtin_amdgcn_readlane(wave_incl_scan(t), 63);
  }
  return total;
}

// The tile-th BM-row tile in group order: group, first row, rows.  skip:
// the first `skip` tiles of every group are left out of the count (their
// workgroups find them directly).
__device__ __forceinline__ bool find_tile(const GemmArgs& p, int BM, int tile, int& g, int& m0,
                                          int& mrows, int skip = 0) {
  if (p.G == 0) {
    const int t = (p.single_rows + BM - 1) / BM;
    if (tile >= t) return false;
    g = 0;
    m0 = tile * BM;
    mrows = min(BM, p.single_rows - m0);
    return true;
  }
  int acc = 0;
  for (int b = 0; b < p.G; b += 64) {
    int lo, hi, t;
    group_chunk(p, BM, b, lo, hi, t);
    t = max(t - skip, 0);
    const int incl = wave_incl_scan(t) + acc;
    const uint64_t m = __ballot(tile < incl);  // empty groups never come first
    if (m) {
      const int f = __builtin_ctzll(m);
      g = b + f;
      const int excl = __builtin_amdgcn_readlane(incl - t, f);
      const int glo = __builtin_amdgcn_readlane(lo, f), ghi = __builtin_amdgcn_readlane(hi, f);
      m0 = glo + (tile - excl + skip) * BM;
      mrows = min(BM, ghi - m0);
      return true;
    }
    acc = __builtin_amdgcn_readlane(incl, 63);
  }
  return false;
}

__device__ __forceinline__ void store_out(void* out, int dtype, int64_t idx, float v) {
  if (dtype == SMOE_F32)
    reinterpret_cast<float*>(out)[idx] = v;
  else
    reinterpret_cast<uint16_t*>(out)[idx] = f2bf(v);
}

__device__ __forceinline__ float col_scale(const GemmArgs& p, int fmt, int g, int n) {
  if (fmt == SMOE_FP8_E4M3) return reinterpret_cast<const float*>(p.S)[g * p.s_gstride + n];
  return 1.0f;
}

__device__ __forceinline__ float bias_at(const GemmArgs& p, int g, int n) {
  return p.bias ? p.bias[g * p.bias_gstride + n] : 0.0f;
}

// Single-element epilogue (all but SwiGLU).
template <int EPI>
__device__ __forceinline__ void epi_one(const GemmArgs& p, int fmt, int g, int row, int n,
                                        float acc) {
  const int64_t o = static_cast<int64_t>(row) * p.ldo + n;
  if constexpr (EPI == EPI_F32_BIAS) {
    reinterpret_cast<float*>(p.out)[o] = acc * col_scale(p, fmt, g, n) + bias_at(p, g, n);
  } else if constexpr (EPI == EPI_ROWSCALE) {
    store_out(p.out, p.out_dtype, o, acc * p.row_scale[row]);
  } else if constexpr (EPI == EPI_GELU) {
    store_out(p.out, p.out_dtype, o, gelu_erf(acc * col_scale(p, fmt, g, n) + bias_at(p, g, n)));
  } else if constexpr (EPI == EPI_DOWN) {
    store_out(p.out, p.out_dtype, o,
              (acc * col_scale(p, fmt, g, n) + bias_at(p, g, n)) * p.row_scale[row]);
  }
}

// SwiGLU pair: interleaved column c (gate, c % 64 < 32) and c + 32 (up).
__device__ __forceinline__ void epi_swiglu(const GemmArgs& p, int fmt, int g, int row, int c,
                                           float gate, float up) {
  const int u = (c >> 6) * 32 + (c & 31);
  const float gs = gate * col_scale(p, fmt, g, c);
  const float us = up * col_scale(p, fmt, g, c + 32) + bias_at(p, g, u);
  store_out(p.out, p.out_dtype, static_cast<int64_t>(row) * p.ldo + u, silu(gs) * us);
}

// ------------------------------------------------------------------ MFMA ----
template <int FMT>
__device__ __forceinline__ u32x4 load_w8(const GemmArgs& p, const void* wrow, int k, int g, int n) {
  if constexpr (FMT == SMOE_BF16) {
    return *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(wrow) + k);
  } else if constexpr (FMT == SMOE_FP8_E4M3) {
    const u32x2 v = *reinterpret_cast<const u32x2*>(reinterpret_cast<const uint8_t*>(wrow) + k);
    const u32x2 lo = fp8x4_to_bf16x4(v.x);
    const u32x2 hi = fp8x4_to_bf16x4(v.y);
    return u32x4{lo.x, lo.y, hi.x, hi.y};
  } else {  // INT4
    const uint32_t v = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint8_t*>(wrow) + (k >> 1));
    const int ng = p.K / p.group_size;
    const float s = load_scale(p.S, g * p.s_gstride + static_cast<int64_t>(n) * ng + k / p.group_size,
                               p.s_f16);
    return int4x8_to_bf16x8(v, s);
  }
}

template <int FMT>
__device__ __forceinline__ const void* w_row_ptr(const GemmArgs& p, int g, int n) {
  const int64_t e = g * p.w_gstride + static_cast<int64_t>(n) * p.ldw;
  if constexpr (FMT == SMOE_BF16) return reinterpret_cast<const uint16_t*>(p.W) + e;
  else if constexpr (FMT == SMOE_FP8_E4M3) return reinterpret_cast<const uint8_t*>(p.W) + e;
  else return reinterpret_cast<const uint8_t*>(p.W) + (e >> 1);
}

template <int BM, int BN, int BK, int WM, int WN, int FMT, int EPI>
__global__ __launch_bounds__(WM* WN * 64) void k_gemm_mfma(const GemmArgs p) {
  constexpr int NT = WM * WN * 64;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 16, FN = TN / 16;
  constexpr int LDK = BK + 8;  // +16 B per row against bank conflicts
  constexpr int CPR = BK / 8;  // 8-element chunks per row
  constexpr int A_CH = (BM * CPR + NT - 1) / NT;
  constexpr int B_CH = (BN * CPR + NT - 1) / NT;
  static_assert(TM % 16 == 0 && TN % 16 == 0 && BK % 32 == 0, "tile shape");
  static_assert(EPI != EPI_SWIGLU || TN % 64 == 0, "SwiGLU pairs 32-column blocks");

  __shared__ __attribute__((aligned(16))) uint16_t sA[2][BM * LDK];
  __shared__ __attribute__((aligned(16))) uint16_t sB[2][BN * LDK];

  int g, m0, mrows;
  if (!find_tile(p, BM, blockIdx.x, g, m0, mrows)) return;
  const int n0 = blockIdx.y * BN;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  const uint16_t* A = reinterpret_cast<const uint16_t*>(p.A);
  const uint16_t* arow[A_CH];
  int a_lds[A_CH];
#pragma unroll
  for (int i = 0; i < A_CH; ++i) {
    const int c = tid + i * NT;
    const int r = c / CPR, kc = (c % CPR) * 8;
    a_lds[i] = (c < BM * CPR) ? r * LDK + kc : -1;
    arow[i] = nullptr;
    if (c < BM * CPR && r < mrows) {
      const int ar = p.a_rows ? p.a_rows[m0 + r] : (m0 + r);
      arow[i] = A + static_cast<int64_t>(ar) * p.lda + kc;
    }
  }
  const void* wrow[B_CH];
  int b_lds[B_CH], b_kc[B_CH], b_n[B_CH];
#pragma unroll
  for (int i = 0; i < B_CH; ++i) {
    const int c = tid + i * NT;
    const int r = c / CPR, kc = (c % CPR) * 8;
    b_lds[i] = (c < BN * CPR) ? r * LDK + kc : -1;
    b_kc[i] = kc;
    b_n[i] = n0 + r;
    // rows past N_out (a partial last N tile) load zeros and are not stored
    wrow[i] = (c < BN * CPR && n0 + r < p.N_out) ? w_row_ptr<FMT>(p, g, n0 + r) : nullptr;
  }

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  u32x4 ra[A_CH], rb[B_CH];
  auto gload = [&](int kt) {
    const int k0 = kt * BK;
#pragma unroll
    for (int i = 0; i < A_CH; ++i)
      ra[i] = arow[i] ? *reinterpret_cast<const u32x4*>(arow[i] + k0) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < B_CH; ++i)
      rb[i] = wrow[i] ? load_w8<FMT>(p, wrow[i], k0 + b_kc[i], g, b_n[i]) : u32x4{0u, 0u, 0u, 0u};
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_CH; ++i)
      if (a_lds[i] >= 0) *reinterpret_cast<u32x4*>(&sA[buf][a_lds[i]]) = ra[i];
#pragma unroll
    for (int i = 0; i < B_CH; ++i)
      if (b_lds[i] >= 0) *reinterpret_cast<u32x4*>(&sB[buf][b_lds[i]]) = rb[i];
  };

  const int KT = p.K / BK;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < KT) gload(kt + 1);
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      bf16x8 af[FM], bfr[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[i] = *reinterpret_cast<const bf16x8*>(
            &sA[buf][(wm * TM + i * 16 + (lane & 15)) * LDK + ks * 32 + (lane >> 4) * 8]);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bfr[j] = *reinterpret_cast<const bf16x8*>(
            &sB[buf][(wn * TN + j * 16 + (lane & 15)) * LDK + ks * 32 + (lane >> 4) * 8]);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < KT) sstore(buf ^ 1);
    __syncthreads();
  }

  // C layout of 16x16 MFMA: lane holds rows 4*(lane/16)+r, column lane%16.
#pragma unroll
  for (int i = 0; i < FM; ++i) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int lr = wm * TM + i * 16 + (lane >> 4) * 4 + r;
      if (lr >= mrows) continue;
      const int row = m0 + lr;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int c = n0 + wn * TN + j * 16 + (lane & 15);
        if (c >= p.N_out) continue;
        if constexpr (EPI == EPI_SWIGLU) {
          if ((j & 3) < 2) epi_swiglu(p, FMT, g, row, c, acc[i][j][r], acc[i][j + 2][r]);
        } else {
          epi_one<EPI>(p, FMT, g, row, c, acc[i][j][r]);
        }
      }
    }
  }
}

// ------------------------------------------------ tile order, 4-wide out ----
// Tile order of the large-tile kernels: the tile grid (real count, from the
// plan) is split into 8 contiguous ranges, one per XCD (workgroup ids are
// dealt to XCDs round robin), and each range is walked in super-rows of GM
// m-tiles x all n-tiles so the super-row's A tiles stay in that XCD's L2
// while weight tiles stream.
template <int BM>
__device__ __forceinline__ int count_m_tiles(const GemmArgs& p) {
  return count_tiles(p, BM);
}

// Row tiles on 16-row bands (an operand or the output in the row-tile
// layout): group g's tiles start at its first row rounded down to a multiple
// of 16, BM rows apart; a tile's live rows are the group's, [rlo, rhi) in
// tile rows.  A band shared by two groups is computed by a tile of each, and
// each stores only its own rows.
__device__ __forceinline__ void band_chunk(const GemmArgs& p, int BM, int b, int& lo, int& hi,
                                           int& t) {
  const int i = b + static_cast<int>(threadIdx.x & 63);
  const int ic = i < p.G ? i : p.G - 1;
  lo = p.grp_off[ic];
  hi = p.grp_off[ic + 1];
  t = (i < p.G && hi > lo) ? (hi - (lo & ~15) + BM - 1) / BM : 0;
}

__device__ __forceinline__ int count_band_tiles(const GemmArgs& p, int BM) {
  if (p.G == 0) return (p.single_rows + BM - 1) / BM;
  int total = 0;
  for (int b = 0; b < p.G; b += 64) {
    int lo, hi, t;
    band_chunk(p, BM, b, lo, hi, t);
    total += __builtin_amdgcn_readlane(wave_incl_scan(t), 63);
  }
  return total;
}

__device__ __forceinline__ bool find_band_tile(const GemmArgs& p, int BM, int tile, int& g, int& m0,
                                               int& rlo, int& rhi) {
  if (p.G == 0) {
    int mrows;
    if (!find_tile(p, BM, tile, g, m0, mrows)) return false;
    rlo = 0;
    rhi = mrows;
    return true;
  }
  int acc = 0;
  for (int b = 0; b < p.G; b += 64) {
    int lo, hi, t;
    band_chunk(p, BM, b, lo, hi, t);
    const int incl = wave_incl_scan(t) + acc;
    const uint64_t m = __ballot(tile < incl);
    if (m) {
      const int f = __builtin_ctzll(m);
      g = b + f;
      const int excl = __builtin_amdgcn_readlane(incl - t, f);
      const int glo = __builtin_amdgcn_readlane(lo, f), ghi = __builtin_amdgcn_readlane(hi, f);
      m0 = (glo & ~15) + (tile - excl) * BM;
      rlo = max(glo - m0, 0);
      rhi = min(ghi - m0, BM);
      return true;
    }
    acc = __builtin_amdgcn_readlane(incl, 63);
  }
  return false;
}

__device__ __forceinline__ bool row_tiles(const GemmArgs& p) { return p.At != nullptr || p.out_tiles; }

// The tile of workgroup bid: group, first row m0, live rows
// [rlo, rhi) in tile rows (rlo > 0 only for band-aligned tiles), first
// output channel.  Workgroup ids are dealt to the 8 XCDs round robin
// (bid & 7 is the XCD).
template <int BM, int BN, int GM>
__device__ __forceinline__ bool big_tile(const GemmArgs& p, int bid, int& g, int& m0, int& rlo,
                                         int& rhi, int& n0) {
  const bool bands = row_tiles(p);
  const int tn_count = (p.N_out + BN - 1) / BN;
  const int tm_count = bands ? count_band_tiles(p, BM) : count_m_tiles<BM>(p);
  const int T = tm_count * tn_count;
  if (bid >= T) return false;
  const int x = bid & 7, local = bid >> 3;
  const int base = T >> 3, rem = T & 7;
  const int logical = x * base + min(x, rem) + local;
  const int grp = logical / (GM * tn_count);
  const int first_m = grp * GM;
  const int gsize = min(GM, tm_count - first_m);
  const int in = logical - grp * GM * tn_count;
  const int tm = first_m + in % gsize;
  n0 = (in / gsize) * BN;
  if (bands) return find_band_tile(p, BM, tm, g, m0, rlo, rhi);
  int mrows;
  if (!find_tile(p, BM, tm, g, m0, mrows)) return false;
  rlo = 0;
  rhi = mrows;
  return true;
}

template <int EPI>
__device__ __forceinline__ void store4(const GemmArgs& p, int fmt, int g, int row, int n, f32x4 v) {
  // 4 consecutive channels n..n+3 of one row
  const int64_t o = static_cast<int64_t>(row) * p.ldo + n;
  float r[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float a = v[i] * col_scale(p, fmt, g, n + i);
    if constexpr (EPI == EPI_F32_BIAS)
      r[i] = a + ((p.W2 && n >= p.n_split) ? (p.bias2 ? p.bias2[n - p.n_split + i] : 0.f)
                                            : bias_at(p, g, n + i));
    else if constexpr (EPI == EPI_ROWSCALE) r[i] = v[i] * p.row_scale[row];
    else if constexpr (EPI == EPI_GELU) r[i] = gelu_erf(a + bias_at(p, g, n + i));
    else r[i] = (a + bias_at(p, g, n + i)) * p.row_scale[row];  // EPI_DOWN
  }
  if (EPI == EPI_F32_BIAS || p.out_dtype == SMOE_F32) {
    *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(p.out) + o) = f32x4{r[0], r[1], r[2], r[3]};
  } else {
    *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(p.out) + o) =
        u32x2{pack_bf2(r[0], r[1]), pack_bf2(r[2], r[3])};
  }
}

// Epilogue of an LDS-staged tile: math in registers, the bf16 tile staged
// in the (idle) LDS ring, then coalesced 16-byte stores.  Staging layout:
// row r, 16-byte chunk c at chunk c ^ (r & 15) (rows of OW bf16, no padding;
// r & 7 for 8-chunk rows).  Only the live rows [rlo, rhi) are stored, and
// 16-row strips without any are skipped.  With p.out_tiles the stores follow
// the row-tile layout (m0 a multiple of 16): 64 consecutive threads write
// one 1 KB block (16 rows x 32 columns).
//
// The lane's bias values (4 channels of each fragment column; SwiGLU: of its
// up columns) and the row scales of its strips are loaded before any math
// (one memory round trip for the whole epilogue).  The costly activations
// (SwiGLU; GELU of small wave tiles) are computed into packed registers
// before the workgroup barrier that frees the ring (the caller need not
// synchronise), so one wave row's math overlaps the other's last MFMAs; the
// others are computed as they are staged (a packed tile of 4 channels per
// fragment column would not fit beside the accumulators).
// Without a bias (the SwiGLU experts) its loads and adds are compiled out.
// fp8 weights (WF): each channel's scale multiplies its accumulator first.
template <int BM, int BN, int TM, int TN, int NT, int EPI, int WF = SMOE_BF16>
__device__ __forceinline__ void tile_epilogue(const GemmArgs& p, const f32x4 (&acc)[TN / 16][TM / 16],
                                              int g, int m0, int rlo, int rhi, int n0, int wm,
                                              int wn, uint8_t* ring) {
  constexpr int FM = TM / 16, FN = TN / 16;
  constexpr int OW = (EPI == EPI_SWIGLU) ? BN / 2 : BN;  // output columns of the tile
  constexpr int SWM = (OW / 8 >= 16 ? 16 : OW / 8) - 1;  // chunk swizzle mask
  constexpr bool HAS_BIAS = EPI != EPI_ROWSCALE;
  constexpr bool HAS_RS = EPI == EPI_ROWSCALE || EPI == EPI_DOWN;
  constexpr int NJ = (EPI == EPI_SWIGLU) ? FN / 2 : FN;  // output fragment columns
  constexpr bool EARLY = EPI == EPI_SWIGLU || (EPI == EPI_GELU && FM * NJ <= 16);
  const int tid = threadIdx.x, lane = tid & 63;
  const int fr = lane & 15, fc = lane >> 4;
  uint16_t* stg = reinterpret_cast<uint16_t*>(ring);
  auto stg_at = [&](int r, int col) {  // staging row r, col: multiple of 4
    return stg + r * OW + ((((col >> 3) ^ (r & SWM)) << 3) | (col & 7));
  };
  const int ncol0 = (EPI == EPI_SWIGLU) ? (n0 >> 1) : n0;
  const int ncols = (EPI == EPI_SWIGLU) ? (p.N_out >> 1) : p.N_out;  // a last tile may be partial
  auto live = [&](int i) {  // strip i holds a live row (wave-uniform)
    const int tr0 = wm * TM + i * 16;
    return tr0 < rhi && tr0 + 16 > rlo;
  };
  constexpr bool F8 = WF == SMOE_FP8_E4M3;
  auto body = [&](auto with_bias) {
    constexpr bool WB = HAS_BIAS && decltype(with_bias)::value;
    float bq[WB ? NJ : 1][4];
    float rsv[HAS_RS ? FM : 1];
    // fp8 channel scales: [fragment column][channel] (SwiGLU: gate, then up 32 on)
    float sc[F8 ? FN : 1][4];
    if constexpr (F8) {
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int c = n0 + wn * TN + j * 16 + fc * 4;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          sc[j][q] = c + q < p.N_out
                         ? reinterpret_cast<const float*>(p.S)[g * p.s_gstride + c + q]
                         : 0.f;
      }
    }
    if constexpr (WB) {
#pragma unroll
      for (int j = 0, b = 0; j < FN; ++j) {
        if (EPI == EPI_SWIGLU && (j & 3) >= 2) continue;
        const int cl = wn * TN + j * 16 + fc * 4;
        const int c = (EPI == EPI_SWIGLU) ? (n0 >> 1) + (cl >> 6) * 32 + (cl & 31) : n0 + cl;
#pragma unroll
        for (int q = 0; q < 4; ++q) bq[b][q] = c + q < ncols ? bias_at(p, g, c + q) : 0.f;
        ++b;
      }
    }
    if constexpr (HAS_RS) {
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int lr = wm * TM + i * 16 + fr;
        rsv[i] = lr >= rlo && lr < rhi ? p.row_scale[m0 + lr] : 0.f;
      }
    }
    // the packed outputs of strip i, fragment column j (bias slot b)
    auto value = [&](int i, int j, int b) {
      float r[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if constexpr (EPI == EPI_SWIGLU) {
          const float gate = F8 ? acc[j][i][q] * sc[F8 ? j : 0][q] : acc[j][i][q];
          const float up = F8 ? acc[j + 2][i][q] * sc[F8 ? j + 2 : 0][q] : acc[j + 2][i][q];
          r[q] = silu(gate) * (WB ? up + bq[WB ? b : 0][q] : up);
        } else {
          const float v = F8 ? acc[j][i][q] * sc[F8 ? j : 0][q] : acc[j][i][q];
          const float a = WB ? v + bq[WB ? b : 0][q] : v;
          if constexpr (HAS_RS) r[q] = a * rsv[HAS_RS ? i : 0];
          else if constexpr (EPI == EPI_GELU) r[q] = gelu_erf(a);
          else r[q] = a;
        }
      }
      return u32x2{pack_bf2(r[0], r[1]), pack_bf2(r[2], r[3])};
    };
    u32x2 pk[EARLY ? FM : 1][NJ];
    if constexpr (EARLY) {
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        if (!live(i)) continue;
#pragma unroll
        for (int j = 0, b = 0; j < FN; ++j) {
          if (EPI == EPI_SWIGLU && (j & 3) >= 2) continue;
          pk[i][b] = value(i, j, b);
          ++b;
        }
      }
    }
    __syncthreads();  // every wave is done with the ring: it becomes the staging buffer
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      if (!live(i)) continue;
      const int sr = wm * TM + i * 16 + fr;  // staging row = tile row
#pragma unroll
      for (int j = 0, b = 0; j < FN; ++j) {
        if (EPI == EPI_SWIGLU && (j & 3) >= 2) continue;
        const int cl = wn * TN + j * 16 + fc * 4;  // channel within the tile
        const int col = (EPI == EPI_SWIGLU) ? (cl >> 6) * 32 + (cl & 31) : cl;
        *reinterpret_cast<u32x2*>(stg_at(sr, col)) = EARLY ? pk[EARLY ? i : 0][b] : value(i, j, b);
        ++b;
      }
    }
  };
  if (!HAS_BIAS || p.bias) body(std::true_type{});
  else body(std::false_type{});
  __syncthreads();
  uint16_t* out = reinterpret_cast<uint16_t*>(p.out);
  if (p.out_tiles) {
    constexpr int KB = OW / 32;  // 32-column blocks per tile row band
    const int ldb = p.ldo >> 5;  // blocks per band of the whole output
    for (int q = tid; q < BM / 16 * KB * 64; q += NT) {
      const int blk = q >> 6, l = q & 63;
      const int r = (blk / KB) * 16 + (l & 15), cc = (blk % KB) * 32 + (l >> 4) * 8;
      if (r >= rlo && r < rhi && ncol0 + cc < ncols)
        __builtin_nontemporal_store(
            *reinterpret_cast<const u32x4*>(stg_at(r, cc)),
            reinterpret_cast<u32x4*>(out + ((static_cast<int64_t>((m0 + r) >> 4) * ldb +
                                             ((ncol0 + cc) >> 5)) << 9) + 8 * l));
    }
    return;
  }
  constexpr int CPR_OUT = OW / 8;  // 16-byte chunks per output row
  for (int q = tid; q < BM * CPR_OUT; q += NT) {
    const int r = q / CPR_OUT, cc = (q % CPR_OUT) * 8;
    // non-temporal: every CU stores its tile at about the same time, and
    // the burst streams past the caches (the next kernel reads it once).
    // With the epilogue loads hoisted: C1's up GEMM 2.20 -> 2.15 ms per
    // step, C3's step 3.66 -> 3.49 ms.
    if (r >= rlo && r < rhi && ncol0 + cc < ncols)
      __builtin_nontemporal_store(
          *reinterpret_cast<const u32x4*>(stg_at(r, cc)),
          reinterpret_cast<u32x4*>(out + static_cast<int64_t>(m0 + r) * p.ldo + ncol0 + cc));
  }
}

// ------------------------------------------------- MFMA, LDS-DMA ring ----
// 256 x BN block tile (BN = 256 or 128), 4 waves in a 2 x 2 grid, wave tile
// 128 x BN/2.  K advances 32 per stage; operands go global -> LDS directly
// with global_load_lds_dwordx4 (no VGPR staging) into an NS-stage LDS ring,
// loads for stage s+NS-1 are issued while stage s computes, and each
// iteration waits only for the loads of the stage it needs next (explicit
// vmcnt — the in-order VMEM counter — then one s_barrier).  The fragments of
// stage s+1 are read into a second register set while stage s's MFMAs run.
//
// LDS rows are 64 B (32 bf16 = 4 chunks of 16 B), chunk c of row r stored at
// chunk c ^ ((r >> 1) & 3).  Measured on gfx950, fragment reads (16 rows x one
// chunk per ds_read_b128) run at ~226 B/clk/CU with this swizzle against
// ~118 with c ^ ((r >> 2) & 3) or no swizzle.  A DMA instruction writes 1 KB
// lane-linearly (16 rows x 64 B): lane i covers row i/4, physical chunk i%4,
// and loads the logical chunk that the swizzle places there.
__device__ __forceinline__ int swz32(int row, int chunk) {
  return row * 64 + ((chunk ^ ((row >> 1) & 3)) << 4);
}

template <int BN, int NS, int GM, int EPI, bool PK = false>
// A ring of 3 stages (72 KB of LDS at BN = 128) lets two workgroups share a
// CU (registers are held to 256 per lane by the launch bound), so one's
// epilogue math and DMA waits overlap the other's MFMAs.
__global__ __launch_bounds__(256, NS <= 3 ? 2 : 1) void k_gemm_ring(const GemmArgs p) {
  constexpr int BM = 256;
  constexpr int TM = BM / 2, TN = BN / 2;
  constexpr int FM = TM / 16, FN = TN / 16;
  constexpr int A_BYTES = BM * 64, B_BYTES = BN * 64, STAGE = A_BYTES + B_BYTES;
  constexpr int A_LD = BM / 16 / 4, B_LD = BN / 16 / 4;  // DMA instructions per wave per stage
  constexpr int LD = A_LD + B_LD;
  static_assert(EPI != EPI_SWIGLU || TN % 64 == 0, "SwiGLU pairs 32-channel blocks");
  static_assert(BM * ((EPI == EPI_SWIGLU) ? BN / 2 : BN) * 2 <= NS * STAGE,
                "output staging fits in the ring");
  __shared__ __attribute__((aligned(1024))) uint8_t ring[NS * STAGE];

  int g, m0, rlo, mrows, n0;  // never given row tiles: rlo = 0
  if (!big_tile<BM, BN, GM>(p, blockIdx.x, g, m0, rlo, mrows, n0)) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // DMA sources: instruction j of this wave covers rows 16 (4 j + wave) ..
  const uint16_t* A = reinterpret_cast<const uint16_t*>(p.A);
  const uint16_t* W = reinterpret_cast<const uint16_t*>(p.W) + g * p.w_gstride;
  const uint16_t* asrc[A_LD];
  const uint16_t* bsrc[B_LD];
  {
    const int pr = lane >> 2, pc = lane & 3;
#pragma unroll
    for (int j = 0; j < A_LD; ++j) {
      const int r = (4 * j + wave) * 16 + pr;
      const int rr = r < mrows ? r : 0;  // rows past the group end: valid data, never stored
      const int ar = p.a_rows ? p.a_rows[m0 + rr] : (m0 + rr);
      asrc[j] = A + static_cast<int64_t>(ar) * p.lda + ((pc ^ ((r >> 1) & 3)) << 3);
    }
#pragma unroll
    for (int j = 0; j < B_LD; ++j) {
      const int r = (4 * j + wave) * 16 + pr;
      if constexpr (PK) {  // weight tile layout: 16 rows x 32 k = 1 KB of lane-ordered fragments
        const int r0 = n0 + (4 * j + wave) * 16;
        const int tile = (r0 < p.N_out ? r0 : n0) >> 4;
        bsrc[j] = reinterpret_cast<const uint16_t*>(p.Wt) +
                  ((static_cast<int64_t>(g) * (p.N_out >> 4) + tile) * (p.K >> 5)) * 512 + 8 * lane;
      } else {
        const int n = n0 + r < p.N_out ? n0 + r : n0;
        bsrc[j] = W + static_cast<int64_t>(n) * p.ldw + ((pc ^ ((r >> 1) & 3)) << 3);
      }
    }
  }
  auto issue = [&](int stage) {  // DMA of K slice `stage` into ring slot stage % NS
    uint8_t* base = ring + (stage % NS) * STAGE;
    const int k0 = stage * 32;
#pragma unroll
    for (int j = 0; j < A_LD; ++j)
      __builtin_amdgcn_global_load_lds((gbl_vptr)(asrc[j] + k0),
                                       (lds_vptr)(base + (4 * j + wave) * 1024), 16, 0, 0);
#pragma unroll
    for (int j = 0; j < B_LD; ++j)  // tile layout: each stage's block is the next 1 KB
      __builtin_amdgcn_global_load_lds((gbl_vptr)(bsrc[j] + (PK ? stage * 512 : k0)),
                                       (lds_vptr)(base + A_BYTES + (4 * j + wave) * 1024), 16, 0, 0);
  };

  const int fr = lane & 15, fc = lane >> 4;
  // two fragment sets, addressed statically (the stage loop is unrolled by 2)
  bf16x8 wf0[FN], af0[FM], wf1[FN], af1[FM];
  auto read_frags = [&](int stage, bf16x8 (&wf)[FN], bf16x8 (&af)[FM]) {
    const uint8_t* sa = ring + (stage % NS) * STAGE;
    const uint8_t* sb = sa + A_BYTES;
#pragma unroll
    for (int j = 0; j < FN; ++j)
      wf[j] = *reinterpret_cast<const bf16x8*>(
          sb + (PK ? (wn * TN / 16 + j) * 1024 + 16 * lane : swz32(wn * TN + j * 16 + fr, fc)));
#pragma unroll
    for (int i = 0; i < FM; ++i)
      af[i] = *reinterpret_cast<const bf16x8*>(sa + swz32(wm * TM + i * 16 + fr, fc));
  };

  f32x4 acc[FN][FM];
#pragma unroll
  for (int j = 0; j < FN; ++j)
#pragma unroll
    for (int i = 0; i < FM; ++i) acc[j][i] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int KT = p.K / 32;
  // one stage: make stage s+1 resident and read its fragments into the
  // other set, then the MFMAs of stage s.  Stage s's fragments are in
  // registers by the barrier (lgkmcnt(0)), so its slot takes stage s+NS:
  // NS slots keep NS-1 stages in flight while the registers hold the NS-th.
  auto step = [&](int s, bf16x8 (&wc)[FN], bf16x8 (&ac)[FM], bf16x8 (&wn_)[FN],
                  bf16x8 (&an)[FM]) {
    if (s + 1 < KT) {
      // stage s+1 landed (stages s+2 .. s+NS-1 may still be in flight)
      if (s + NS - 1 < KT) wait_vmcnt<(NS - 2) * LD>();
      else wait_vmcnt<0>();
      wait_lgkm0();
      __builtin_amdgcn_s_barrier();
      if (s + NS < KT) issue(s + NS);  // into the slot stage s used
      read_frags(s + 1, wn_, an);
    }
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int i = 0; i < FM; ++i)
        acc[j][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wc[j], ac[i], acc[j][i], 0, 0, 0);
  };

  // prologue: stages 0 .. NS-1 in flight, stage 0 landed everywhere
#pragma unroll
  for (int st = 0; st < NS; ++st)
    if (st < KT) issue(st);
  if (KT >= NS) wait_vmcnt<(NS - 1) * LD>();
  else wait_vmcnt<0>();
  __builtin_amdgcn_s_barrier();
  read_frags(0, wf0, af0);
  // KT is even (K % 64 == 0, checked by the launcher): no conditional step,
  // so the accumulators stay in AGPRs across the loop
  for (int s = 0; s < KT; s += 2) {
    step(s, wf0, af0, wf1, af1);
    step(s + 1, wf1, af1, wf0, af0);
  }

  // (no DMA is outstanding here; the epilogue synchronises before it reuses the ring)
  tile_epilogue<BM, BN, TM, TN, 256, EPI>(p, acc, g, m0, 0, mrows, n0, wm, wn, ring);
}

// --------------------------------------------- MFMA, ping-pong 8 waves ----
// 256 x 256 block tile, 8 waves: wave w and w + 4 share SIMD w % 4, wave tile
// 128 x 64 (rows 128 (w >> 2), channels 64 (w & 3)).  The two wave groups
// (w < 4, w >= 4) run half a K step apart and alternate between a memory
// phase (DMA issue for a later stage, fragment reads of the next stage) and
// an MFMA phase, so on every SIMD one wave feeds the matrix core while its
// partner moves data.  Two workgroup barriers per K step keep them in
// lock-step:
//
//   group 0:  MEM(0) | MFMA(0) | MEM(1)  | MFMA(1) | ...           | MFMA(KT-1)
//   group 1:  ------ | MEM(0)  | MFMA(0) | MEM(1)  | ... | MFMA(KT-1)
//
// MEM(k) issues stage k+NS-1 into the slot of stage k-1 (read by both groups'
// MEM(k-1), which end with lgkmcnt(0) before their barriers), reads stage k's
// fragments, then waits for its own part of stage k+1 (vmcnt) so the next
// barrier certifies stage k+1 for both groups.  LDS layout and DMA scheme as
// in the ring kernel (32-bf16 rows, chunk c of row r at c ^ ((r >> 1) & 3)).
// BM = 256 (wave tile 128 x 64) for many rows per group; BM = 128 (wave tile
// 64 x 64, two workgroups per CU) when groups hold a few hundred rows and a
// 256-row tile would be mostly padding.
constexpr int kPpScaleMax = 8192;  // int4 scale-table entries per 256-channel tile (K / gs <= 32)

template <int NS, int GM, int EPI, int BM, bool PK = false, int WF = SMOE_BF16>
__global__ __launch_bounds__(512, BM == 128 ? 2 : 1) void k_gemm_pp(const GemmArgs p) {
  // WF: the weight format.  fp8-e4m3 weights come from their weight tile
  // copy (16 rows x 64 k per 1 KB block): a 32-k stage of a 16-row tile is
  // half a block, a DMA instruction moves the halves of two tiles, and the
  // fragment reads widen the codes to bf16 (exact) in registers; the
  // per-channel scale is applied in the epilogue.  Half the W bytes of bf16
  // through the DMA and LDS.
  // int4 weights come from their int4 tile copy (smoe_pack_int4_qtiles: a
  // stage of a 64-row quad is one 1 KB block of lane-ordered 4-byte
  // fragments): waves 0-3 each DMA one quad, a quarter of the W bytes of
  // bf16, and a fragment read is one 4-byte LDS load whose 8 nibbles are
  // widened to bf16 in registers as q * s (the row's group scale, from a
  // table of the tile's 256 channels x K / group_size scales loaded into LDS
  // before the main loop, kept in the part of the ring that only the
  // output staging uses), rounded once to bf16 — the values every int4
  // kernel here multiplies.  The widening of stage k + 1 runs in the wave's
  // MFMA phase of stage k, not in its memory phase.
  static_assert(WF == SMOE_BF16 || ((WF == SMOE_FP8_E4M3 || WF == SMOE_INT4) && PK),
                "fp8 / int4 weights need their tile copy");
  constexpr bool F8 = WF == SMOE_FP8_E4M3;
  constexpr bool I4 = WF == SMOE_INT4;
  constexpr int BN = 256, TM = BM / 2, TN = 64;
  constexpr int FM = TM / 16, FN = TN / 16;
  constexpr int A_BYTES = BM * 64, B_BYTES = BN * (I4 ? 16 : F8 ? 32 : 64), STAGE = A_BYTES + B_BYTES;
  // DMA instructions (16 rows each; fp8 W: 32 rows) per stage: A_INS of A,
  // B_LD per wave of W.  With BM = 320 the 20 A instructions do not split
  // evenly over the 8 waves: waves 0-3 issue 3, waves 4-7 issue 2, and each
  // wave's vmcnt waits count its own.  int4 W: one quad per wave 0-3.
  constexpr int A_INS = BM / 16, B_LD = I4 ? 1 : BN / (F8 ? 32 : 16) / 8;
  constexpr int A_LD = (A_INS + 7) / 8;                  // most per wave
  constexpr int A_HI = A_INS % 8 == 0 ? 8 : A_INS % 8;   // waves issuing A_LD of them
  // int4: waves 0-3 issue the W DMA, and (A_HI = 4) the extra A one, so
  // waves 0-3 and 4-7 are the two counts
  static_assert(!I4 || A_HI == 4 || A_HI == 8, "int4: waves 0-3 issue the most DMAs");
  constexpr int LD = A_LD + B_LD;
  constexpr int LD_LO = I4 ? (A_HI == 8 ? A_LD : A_INS / 8) : (A_INS / 8) + B_LD;
  constexpr int OUT_BYTES = BM * ((EPI == EPI_SWIGLU) ? BN / 2 : BN) * 2;
  // the ring also stages the output tile, in one pass: it grows to the tile
  // when that is larger (320 x 256 bf16 is exactly 160 KB; two passes
  // through the 144 KB ring cost a barrier and a half-idle store phase).
  // int4: the scale table follows the stages, inside that allocation.
  constexpr int SC_BYTES = I4 ? kPpScaleMax * 4 : 0;
  constexpr int RING = NS * STAGE + SC_BYTES > OUT_BYTES ? NS * STAGE + SC_BYTES : OUT_BYTES;
  static_assert(RING <= 163840, "LDS of one workgroup");
  static_assert(NS >= 2, "ring depth");
  static_assert(BM == 128 || BM == 256 || BM == 320, "block rows");
  __shared__ __attribute__((aligned(1024))) uint8_t ring[RING];

  int g, m0, rlo, rhi, n0;
  if (!big_tile<BM, BN, GM>(p, blockIdx.x, g, m0, rlo, rhi, n0)) return;  // workgroup-uniform
  uint64_t clk0 = 0, wall0 = 0;
  if (p.clk) {  // diagnostics (uniform): the tile's clock cycles and wall ticks
    clk0 = __builtin_amdgcn_s_memtime();
    wall0 = __builtin_amdgcn_s_memrealtime();
  }
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int grp = wave >> 2;
  const int wm = grp, wn = wave & 3;
  const bool a_hi = wave < A_HI;  // issues A_LD A instructions (else A_LD - 1)
  const bool w_hi = !I4 || wave < 4;  // issues the stage's W DMA (int4: waves 0-3)
  // s_waitcnt vmcnt(n stages of this wave's DMA in flight)
  auto wait_stages = [&](auto n_stages) {
    constexpr int n = decltype(n_stages)::value;
    if constexpr (LD == LD_LO) {
      wait_vmcnt<n * LD>();
    } else {
      if (I4 ? w_hi : a_hi) wait_vmcnt<n * LD>();
      else wait_vmcnt<n * LD_LO>();
    }
  };
  // int4: the tile's group scales, channel-major [256][ng], into LDS.  The
  // loads are unconditional (indices clamped; channels past N_out read the
  // last one's) and go out before the DMA prologue, so the wait for the
  // first stage covers them too.
  float* stab = reinterpret_cast<float*>(ring + NS * STAGE);
  int ng = 1, gshift = 0;
  float scv[I4 ? kPpScaleMax / 512 : 1];
  if constexpr (I4) {
    ng = p.K / p.group_size;
    gshift = __builtin_ctz(p.group_size);
    const int64_t sb = g * p.s_gstride + static_cast<int64_t>(n0) * ng;
    const int last = (min(p.N_out, n0 + BN) - n0) * ng - 1;
    if (p.s_f16) {
      const _Float16* s16 = reinterpret_cast<const _Float16*>(p.S) + sb;
      _Float16 hv[kPpScaleMax / 512];
#pragma unroll
      for (int j = 0; j < kPpScaleMax / 512; ++j) hv[j] = s16[min(tid + 512 * j, last)];
#pragma unroll
      for (int j = 0; j < kPpScaleMax / 512; ++j) scv[j] = static_cast<float>(hv[j]);
    } else {
      const float* s32 = reinterpret_cast<const float*>(p.S) + sb;
#pragma unroll
      for (int j = 0; j < kPpScaleMax / 512; ++j) scv[j] = s32[min(tid + 512 * j, last)];
    }
  }

  // DMA sources: instruction j of wave w covers rows 16 (8 j + w) ..; with
  // At, the 1 KB row-tile block of that band (bands past the buffer's last
  // read its last band: never stored), the next one each K step
  const uint16_t* A = reinterpret_cast<const uint16_t*>(p.A);
  const int a_step = p.At ? 512 : 32;  // elements per K step
  const uint16_t* W = reinterpret_cast<const uint16_t*>(p.W) + g * p.w_gstride;
  const uint16_t* asrc[A_LD];
  const uint8_t* bsrc[B_LD];  // bytes
  {
    const int pr = lane >> 2, pc = lane & 3;
#pragma unroll
    for (int j = 0; j < A_LD; ++j) {
      const int r = min(8 * j + wave, A_INS - 1) * 16 + pr;  // past A_INS: never issued
      if (p.At) {
        const int band = min((m0 >> 4) + min(8 * j + wave, A_INS - 1), ((p.max_rows + 15) >> 4) - 1);
        asrc[j] = reinterpret_cast<const uint16_t*>(p.At) +
                  (static_cast<int64_t>(band) * (p.K >> 5)) * 512 + 8 * lane;
      } else {
        const int rr = r < rhi ? r : rlo;  // rows past the group end: valid data, never stored
        const int ar = p.a_rows ? p.a_rows[m0 + rr] : (m0 + rr);
        asrc[j] = A + static_cast<int64_t>(ar) * p.lda + ((pc ^ ((r >> 1) & 3)) << 3);
      }
    }
#pragma unroll
    for (int j = 0; j < B_LD; ++j) {
      const int r = (8 * j + wave) * 16 + pr;
      if constexpr (I4) {  // quad n0 / 64 + wave (waves 4-7: never issued)
        const int quads = p.N_out >> 6;
        const int qd = min((n0 >> 6) + (wave & 3), quads - 1);
        bsrc[j] = reinterpret_cast<const uint8_t*>(p.Wt) +
                  (static_cast<int64_t>(g) * quads + qd) * (p.K >> 5) * 1024 + 16 * lane;
      } else if constexpr (F8) {  // lanes 0-31: tile 2 (8 j + w), 32-63: the next; 512 B of each per stage
        const int t = n0 + (2 * (8 * j + wave) + (lane >> 5)) * 16;
        const int tile = (t < p.N_out ? t : n0) >> 4;
        bsrc[j] = reinterpret_cast<const uint8_t*>(p.Wt) +
                  ((static_cast<int64_t>(g) * (p.N_out >> 4) + tile) * (p.K >> 6)) * 1024 +
                  16 * (lane & 31);
      } else if constexpr (PK) {  // weight tile layout: 16 rows x 32 k = 1 KB of lane-ordered fragments
        const int tile = (n0 + (8 * j + wave) * 16 < p.N_out ? n0 + (8 * j + wave) * 16 : n0) >> 4;
        bsrc[j] = reinterpret_cast<const uint8_t*>(
            reinterpret_cast<const uint16_t*>(p.Wt) +
            ((static_cast<int64_t>(g) * (p.N_out >> 4) + tile) * (p.K >> 5)) * 512 + 8 * lane);
      } else {
        const int n = n0 + r < p.N_out ? n0 + r : n0;
        bsrc[j] = reinterpret_cast<const uint8_t*>(W + static_cast<int64_t>(n) * p.ldw +
                                                   ((pc ^ ((r >> 1) & 3)) << 3));
      }
    }
  }
  auto issue = [&](int stage) {  // DMA of K slice `stage` into ring slot stage % NS
    uint8_t* base = ring + (stage % NS) * STAGE;
    const int k0 = stage * 32;
#pragma unroll
    for (int j = 0; j < A_LD; ++j)
      if (j + 1 < A_LD || a_hi)  // wave-uniform
        __builtin_amdgcn_global_load_lds((gbl_vptr)(asrc[j] + stage * a_step),
                                         (lds_vptr)(base + (8 * j + wave) * 1024), 16, 0, 0);
#pragma unroll
    for (int j = 0; j < B_LD; ++j)  // tile layout: each stage's (half) block is the next 1 KB (512 B)
      if (w_hi)  // wave-uniform
        __builtin_amdgcn_global_load_lds(
            (gbl_vptr)(bsrc[j] + stage * (I4 ? 1024 : F8 ? 512 : PK ? 1024 : 64)),
            (lds_vptr)(base + A_BYTES + (8 * j + wave) * 1024), 16, 0, 0);
  };
  const int fr = lane & 15, fc = lane >> 4;
  // the lane's A fragment of strip i at a_lds + 1024 i: the swizzled 64-byte
  // rows, or the row-tile block's lane-ordered fragments
  const int a_lds = p.At ? wm * TM * 64 + 16 * lane : swz32(wm * TM + fr, fc);
  bf16x8 wf[FN], af[FM];
  float sj[I4 ? FN : 1];  // int4: the lane's rows' scales of the current group
  int kg_cur = -1;
  // int4: the lane's raw nibbles of `stage` (quad wn, tile j: 8 nibbles at
  // 4 lane), and the scales of its group.  The widening runs one stage ahead,
  // beside the MFMAs of the stage before (tile j once its MFMAs have read
  // it), so the memory phase only reads the activation fragments.
  uint32_t w4[I4 ? FN : 1];
  auto load_w4 = [&](int stage) {
    const int kg = (stage * 32) >> gshift;
    if (kg != kg_cur) {  // uniform: a new scale group every group_size / 32 stages
      kg_cur = kg;
#pragma unroll
      for (int j = 0; j < FN; ++j) sj[j] = stab[(wn * TN + j * 16 + fr) * ng + kg];
    }
    const uint8_t* sb = ring + (stage % NS) * STAGE + A_BYTES;
#pragma unroll
    for (int j = 0; j < FN; ++j)
      w4[j] = *reinterpret_cast<const uint32_t*>(sb + wn * 1024 + j * 256 + 4 * lane);
  };
  auto read_frags = [&](int stage) {
    const uint8_t* sa = ring + (stage % NS) * STAGE;
    const uint8_t* sb = sa + A_BYTES;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      if constexpr (I4) {  // widened during the previous stage's MFMAs
      } else if constexpr (F8) {  // tile tt's half block: row fr, k 8 fc.. at 16 fr + 256 (fc >> 1) + 8 (fc & 1)
        const int tt = wn * TN / 16 + j;
        const u32x2 c = *reinterpret_cast<const u32x2*>(
            sb + (tt >> 1) * 1024 + (tt & 1) * 512 + 16 * fr + 256 * (fc >> 1) + 8 * (fc & 1));
        const u32x2 lo = fp8x4_to_bf16x4(c.x), hi = fp8x4_to_bf16x4(c.y);
        wf[j] = __builtin_bit_cast(bf16x8, u32x4{lo.x, lo.y, hi.x, hi.y});
      } else {  // tile layout: block (wn * TN + 16 j) / 16 holds lane l's fragment at 16 l
        wf[j] = *reinterpret_cast<const bf16x8*>(
            sb + (PK ? (wn * TN / 16 + j) * 1024 + 16 * lane : swz32(wn * TN + j * 16 + fr, fc)));
      }
    }
#pragma unroll
    for (int i = 0; i < FM; ++i)
      af[i] = *reinterpret_cast<const bf16x8*>(sa + a_lds + 1024 * i);
  };

  f32x4 acc[FN][FM];
#pragma unroll
  for (int j = 0; j < FN; ++j)
#pragma unroll
    for (int i = 0; i < FM; ++i) acc[j][i] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int KT = p.K / 32;
  // prologue: stages 0 .. NS-2 in flight, stage 0 landed everywhere
#pragma unroll
  for (int st = 0; st < NS - 1; ++st)
    if (st < KT) issue(st);
  if constexpr (I4) {
#pragma unroll
    for (int j = 0; j < kPpScaleMax / 512; ++j)
      if (tid + 512 * j < BN * ng) stab[tid + 512 * j] = scv[j];
  }
  if (KT >= NS - 1) wait_stages(std::integral_constant<int, NS - 2>{});
  else wait_vmcnt<0>();
  if constexpr (I4) wait_lgkm0();  // the scale table is written
  __builtin_amdgcn_s_barrier();
  if constexpr (I4) {  // stage 0's weights, before the first memory phase
    load_w4(0);
#pragma unroll
    for (int j = 0; j < FN; ++j) wf[j] = __builtin_bit_cast(bf16x8, int4x8_to_bf16x8(w4[j], sj[j]));
  }
  if (grp == 1) __builtin_amdgcn_s_barrier();  // group 1 starts half a step behind
  for (int k = 0; k < KT; ++k) {
    // MEM(k)
    if (k + NS - 1 < KT) issue(k + NS - 1);
    read_frags(k);
    if (k + 1 < KT) {  // own part of stage k+1 landed (stages k+2 .. k+NS-1 may fly)
      if (k + NS - 1 < KT) wait_stages(std::integral_constant<int, NS - 2>{});
      else wait_vmcnt<0>();
    }
    wait_lgkm0();
    __builtin_amdgcn_s_barrier();
    // MFMA(k); int4: stage k + 1's weights (the last stage re-reads itself).
    // Only waves 0-3 (group 0) DMA int4 weights, and they waited for stage
    // k + 1 before the barrier that ended group 0's memory phase of k, which
    // precedes both groups' MFMA phase of k.  (fp8 weights are DMA'd by all
    // eight waves, so group 0 could read group 1's part early: not here.)
    if constexpr (I4) load_w4(min(k + 1, KT - 1));
#pragma unroll
    for (int j = 0; j < FN; ++j) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
        acc[j][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[j], af[i], acc[j][i], 0, 0, 0);
      if constexpr (I4) {
        // the empty asm pins the widening before the barrier: left free, the
        // compiler sinks it to its use, the next memory phase
        u32x4 u = int4x8_to_bf16x8(w4[j], sj[j]);
        asm volatile("" : "+v"(u));
        wf[j] = __builtin_bit_cast(bf16x8, u);
      }
    }
    if (grp == 0 || k + 1 < KT) __builtin_amdgcn_s_barrier();
  }
  // (no DMA is outstanding here; the epilogue synchronises before it reuses the ring)
  tile_epilogue<BM, BN, TM, TN, 512, EPI, WF>(p, acc, g, m0, rlo, rhi, n0, wm, wn, ring);
  if (p.clk && tid == 0) {
    const uint64_t dc = __builtin_amdgcn_s_memtime() - clk0;
    const uint64_t dw = __builtin_amdgcn_s_memrealtime() - wall0;
    atomicAdd(p.clk, static_cast<unsigned long long>(dc));
    atomicAdd(p.clk + 1, static_cast<unsigned long long>(dw));
  }
}

// --------------------------------------------------------------- skinny ----
// Few rows per group (decode): the weights are nearly all of the traffic, so
// a workgroup streams one strip of 16*TN weight rows (output channels) of one
// group from HBM straight into registers and its NW waves split K.  In each
// 64-wide K step a lane loads the 16 consecutive k at k0 + 16*(lane/16) of
// its weight row (fp8 16 B, bf16 32 B, int4 8 B) and of its activation row;
// the step's two MFMAs take the low and the high 8 of them (the order of k
// inside a step is free as long as both operands follow it).  The loads of U
// steps are issued before the first MFMA of the batch.  The waves' partial
// sums meet in LDS and are added in wave order, so results are bit-identical
// run to run; the epilogue writes 4 consecutive channels per lane.
// A workgroup takes one tile of at most 16*RT rows of one group; the tiles
// of all groups form one flat list (grid.y), so at many rows (router / edge
// logits at prefill: narrow outputs, the activations are the stream) and
// skewed groups the work still spreads evenly.
// A lane's raw 16 consecutive k of one weight row, in its storage format
// (only what the format needs stays in registers).
template <int FMT> struct WRaw;
template <> struct WRaw<SMOE_BF16> { u32x4 a, b; };
template <> struct WRaw<SMOE_FP8_E4M3> { u32x4 a; };
template <> struct WRaw<SMOE_INT4> { u32x2 a; float s; };  // 16 nibbles + their group scale

template <int FMT>
__device__ __forceinline__ WRaw<FMT> skinny_wload(const GemmArgs& p, const uint8_t* wrow, int k,
                                                  int g, int n) {
  WRaw<FMT> r;
  if constexpr (FMT == SMOE_BF16) {
    const u32x4* q = reinterpret_cast<const u32x4*>(wrow + 2 * static_cast<int64_t>(k));
    r.a = q[0];
    r.b = q[1];
  } else if constexpr (FMT == SMOE_FP8_E4M3) {
    r.a = *reinterpret_cast<const u32x4*>(wrow + k);
  } else {  // INT4: inside one scale group (group_size % 16 == 0)
    r.a = *reinterpret_cast<const u32x2*>(wrow + (k >> 1));
    r.s = load_scale(p.S,
                     g * p.s_gstride + static_cast<int64_t>(n) * (p.K / p.group_size) +
                         k / p.group_size,
                     p.s_f16);
  }
  return r;
}

// The raw 16 k of a lane -> the bf16 A operands of the step's two MFMAs.
template <int FMT>
__device__ __forceinline__ void skinny_wconv(const WRaw<FMT>& r, bf16x8& lo, bf16x8& hi) {
  u32x4 l, h;
  if constexpr (FMT == SMOE_BF16) {
    l = r.a;
    h = r.b;
  } else if constexpr (FMT == SMOE_FP8_E4M3) {
    const u32x2 a0 = fp8x4_to_bf16x4(r.a.x), a1 = fp8x4_to_bf16x4(r.a.y);
    const u32x2 b0 = fp8x4_to_bf16x4(r.a.z), b1 = fp8x4_to_bf16x4(r.a.w);
    l = u32x4{a0.x, a0.y, a1.x, a1.y};
    h = u32x4{b0.x, b0.y, b1.x, b1.y};
  } else {
    l = int4x8_to_bf16x8(r.a.x, r.s);
    h = int4x8_to_bf16x8(r.a.y, r.s);
  }
  lo = __builtin_bit_cast(bf16x8, l);
  hi = __builtin_bit_cast(bf16x8, h);
}

template <int FMT, int EPI, int TN, int RT, int NW, int U>
__global__ __launch_bounds__(NW * 64) void k_gemm_skinny(const GemmArgs p) {
  constexpr int BN = 16 * TN;
  constexpr int ESZ2 = FMT == SMOE_BF16 ? 4 : (FMT == SMOE_FP8_E4M3 ? 2 : 1);  // 2 x bytes/elt
  static_assert(EPI != EPI_SWIGLU || TN == 4, "SwiGLU pairs channel c with c + 32");
  static_assert(NW >= TN, "one wave per channel tile in the epilogue");
  __shared__ f32x4 red[NW][TN * RT][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = lane >> 4, l16 = lane & 15;
  const int n0 = blockIdx.x * BN;
  // one tile of <= 16*RT rows of one group: the tiles of all groups form one
  // flat list over grid.y, so skewed groups spread over many workgroups
  int g, r_lo, r_hi;
  {
    int m0, mrows;
    if (!find_tile(p, 16 * RT, blockIdx.y, g, m0, mrows)) return;  // uniform, before any barrier
    r_lo = m0;
    r_hi = m0 + mrows;
  }
  const uint8_t* wrow[TN];
  int wn[TN];
#pragma unroll
  for (int t = 0; t < TN; ++t) {
    const int n = min(n0 + 16 * t + l16, p.N_out - 1);  // rows past N_out: loaded, never stored
    wn[t] = n;
    wrow[t] = (p.W2 && n >= p.n_split)
                  ? reinterpret_cast<const uint8_t*>(p.W2) +
                        static_cast<int64_t>(n - p.n_split) * p.ldw2 * ESZ2 / 2
                  : reinterpret_cast<const uint8_t*>(p.W) +
                        (g * p.w_gstride + static_cast<int64_t>(n) * p.ldw) * ESZ2 / 2;
  }
  // the epilogue operands of this wave's channel tile (waves < ET), requested
  // before the weight stream: they are in registers when the partial sums
  // meet instead of costing a round trip after them
  constexpr int ET = EPI == EPI_SWIGLU ? TN / 2 : TN;
  float esc[4], esc2[4], ebi[4], ers[RT];
  {
    const int ce = min(n0 + 16 * (wave < ET ? wave : 0) + 4 * q, p.N_out - 4);
    const bool seg2 = p.W2 && ce >= p.n_split;  // second weight segment (front GEMM)
    const int bc = EPI == EPI_SWIGLU ? (ce >> 6) * 32 + (ce & 31) : ce;
    const int64_t s0 = g * p.s_gstride + ce;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      constexpr bool fp8 = FMT == SMOE_FP8_E4M3 && EPI != EPI_ROWSCALE;
      esc[i] = fp8 ? reinterpret_cast<const float*>(p.S)[s0 + i] : 1.0f;
      esc2[i] = (fp8 && EPI == EPI_SWIGLU) ? reinterpret_cast<const float*>(p.S)[s0 + 32 + i] : 1.0f;
      ebi[i] = EPI == EPI_ROWSCALE ? 0.0f
               : seg2              ? (p.bias2 ? p.bias2[ce - p.n_split + i] : 0.0f)
                                   : bias_at(p, g, bc + i);
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
      ers[rt] = (EPI == EPI_ROWSCALE || EPI == EPI_DOWN)
                    ? p.row_scale[min(r_lo + 16 * rt + l16, r_hi - 1)]
                    : 1.0f;
  }
  const int KS = p.K / 64;
  const int s_begin = wave * KS / NW, s_end = (wave + 1) * KS / NW;
  const uint16_t* A = reinterpret_cast<const uint16_t*>(p.A);
  for (int m0 = r_lo; m0 < r_hi; m0 += 16 * RT) {  // one pass (the tile)
    const uint16_t* arow[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      int r = m0 + 16 * rt + l16;
      r = r < r_hi ? r : r_lo;  // rows past the group: a valid row, never stored
      const int ar = p.a_rows ? p.a_rows[r] : r;
      arow[rt] = A + static_cast<int64_t>(ar) * p.lda + 16 * q;
    }
    f32x4 acc[TN][RT];
#pragma unroll
    for (int t = 0; t < TN; ++t)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) acc[t][rt] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int s0 = s_begin; s0 < s_end; s0 += U) {
      WRaw<FMT> wr[U][TN];
      u32x4 av[U][RT][2];
#pragma unroll
      for (int u = 0; u < U; ++u) {  // steps past s_end reload the last one (not used)
        const int st = min(s0 + u, s_end - 1);
        const int k = st * 64 + 16 * q;
#pragma unroll
        for (int t = 0; t < TN; ++t) wr[u][t] = skinny_wload<FMT>(p, wrow[t], k, g, wn[t]);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          const u32x4* ap = reinterpret_cast<const u32x4*>(arow[rt] + st * 64);
          av[u][rt][0] = ap[0];
          av[u][rt][1] = ap[1];
        }
      }
      // steps past s_end multiply zeros (both operands, so 0 * 0): no branch
      // for the compiler to sink the batch's loads into
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool live = s0 + u < s_end;
        const u32x4 z = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int t = 0; t < TN; ++t) {
          bf16x8 lo, hi;
          skinny_wconv<FMT>(wr[u][t], lo, hi);
          if (u > 0) {  // step s0 is always live
            lo = live ? lo : __builtin_bit_cast(bf16x8, z);
            hi = live ? hi : __builtin_bit_cast(bf16x8, z);
          }
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) {
            const u32x4 b0 = (u == 0 || live) ? av[u][rt][0] : z;
            const u32x4 b1 = (u == 0 || live) ? av[u][rt][1] : z;
            acc[t][rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                lo, __builtin_bit_cast(bf16x8, b0), acc[t][rt], 0, 0, 0);
            acc[t][rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                hi, __builtin_bit_cast(bf16x8, b1), acc[t][rt], 0, 0, 0);
          }
        }
      }
    }
#pragma unroll
    for (int t = 0; t < TN; ++t)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) red[wave][t * RT + rt][lane] = acc[t][rt];
    __syncthreads();
    // lane: channels n0 + 16 t + 4 q + (0..3) of row m0 + 16 rt + l16
    if (wave < ET) {
      const int t = wave;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const int row = m0 + 16 * rt + l16;
        f32x4 v = red[0][t * RT + rt][lane];
#pragma unroll
        for (int w = 1; w < NW; ++w) v += red[w][t * RT + rt][lane];
        const int c = n0 + 16 * t + 4 * q;
        if (row >= r_hi || c >= p.N_out) continue;
        float o[4];
        int col = c;
        if constexpr (EPI == EPI_SWIGLU) {
          f32x4 up = red[0][(t + TN / 2) * RT + rt][lane];
#pragma unroll
          for (int w = 1; w < NW; ++w) up += red[w][(t + TN / 2) * RT + rt][lane];
          col = (c >> 6) * 32 + (c & 31);
#pragma unroll
          for (int i = 0; i < 4; ++i) o[i] = silu(v[i] * esc[i]) * (up[i] * esc2[i] + ebi[i]);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if constexpr (EPI == EPI_ROWSCALE) o[i] = v[i] * ers[rt];
            else if constexpr (EPI == EPI_GELU) o[i] = gelu_erf(v[i] * esc[i] + ebi[i]);
            else if constexpr (EPI == EPI_DOWN) o[i] = (v[i] * esc[i] + ebi[i]) * ers[rt];
            else o[i] = v[i] * esc[i] + ebi[i];  // EPI_F32_BIAS
          }
        }
        const int64_t off = static_cast<int64_t>(row) * p.ldo + col;
        if (EPI == EPI_F32_BIAS || p.out_dtype == SMOE_F32)
          *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(p.out) + off) =
              f32x4{o[0], o[1], o[2], o[3]};
        else
          *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(p.out) + off) =
              u32x2{pack_bf2(o[0], o[1]), pack_bf2(o[2], o[3])};
      }
    }
    __syncthreads();  // red is rewritten by the next pass
  }
}

// ------------------------------------------------------ decode stream ----
// Weight streams of decode steps (a few rows per group, wide outputs): the
// weights are nearly all of the traffic.  Each wave streams its own slice,
// TNW 16-channel tiles of one group (SwiGLU: TNW / 2 gate tiles and the up
// tiles 32 channels on) over one KSPLIT-th of K, for one tile of <= 16*RT rows,
// through a D-step register ring: step s + D is requested as step s is
// widened and multiplied, so every wave keeps D steps in flight and its MFMAs
// run while the rest of its stream arrives (a wave that requested its whole
// slice at once would wait for the last byte before its first MFMA, and all
// waves of the grid would do their arithmetic at the end).  The KSPLIT waves
// of a slice add their partial sums through LDS in wave order (bit-identical
// run to run); with KSPLIT 1 no wave waits for another.  k order inside a
// 64-wide step, the same for both operands: bf16 weights take k 8q..8q+7
// (first MFMA) and 32+8q.. (second), so each of their two 16-byte loads
// covers 64 contiguous bytes of 16 rows; fp8 / int4 take the 16 consecutive
// k at 16q.  Only the last 2D - 1 steps' refills sit under a branch, so the
// main loop's waits count the loads in flight exactly.
template <int FMT>
struct DRaw;
template <> struct DRaw<SMOE_BF16> { u32x4 a, b; };
template <> struct DRaw<SMOE_FP8_E4M3> { u32x4 a; };
template <> struct DRaw<SMOE_INT4> { u32x2 a; float s; };

// The position of the j-th set bit (0-based) of m; j < popcount(m).
__device__ __forceinline__ int nth_set_bit(uint64_t m, int j) {
  int pos = 0;
#pragma unroll
  for (int w = 32; w >= 1; w >>= 1) {
    const uint64_t lo = m & ((1ull << w) - 1ull);
    const int c = __popcll(lo);
    const bool up = j >= c;
    j = up ? j - c : j;
    m = up ? (m >> w) : lo;
    pos += up ? w : 0;
  }
  return pos;
}

// SEL: the decode edge projection's row selection (GemmArgs::sel_*): row
// tile gy is tile gy % sel_tpg of destination gy / sel_tpg, whose rows are
// found from the front's selections by a ballot over the tokens (lane t);
// its weights are known before any load.  red: LDS of
// (KSPLIT > 1 ? 4 : 1) * TNW * RT * 64 f32x4.
template <int FMT, int EPI, int TNW, int RT, int KSPLIT, int D, bool PK, bool SEL>
__device__ __forceinline__ void decode_gemm(const GemmArgs& p, int gy, f32x4* red) {
  constexpr int ESZ2 = FMT == SMOE_BF16 ? 4 : (FMT == SMOE_FP8_E4M3 ? 2 : 1);  // 2 x bytes/elt
  constexpr int CS = 4 / KSPLIT;  // channel slices per workgroup
  static_assert(4 % KSPLIT == 0, "KSPLIT divides the 4 waves");
  static_assert(EPI != EPI_SWIGLU || TNW == 2 || TNW == 4, "SwiGLU slices pair gate and up tiles");
  static_assert(!PK || FMT != SMOE_INT4, "the weight tile layout holds bf16 or fp8 weights");
  static_assert(!SEL || EPI == EPI_ROWSCALE, "row selection: the edge projection");
  constexpr int BLK = 512 * ESZ2;  // bytes of one 64-k step of a 16-row tile
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = lane >> 4, l16 = lane & 15;
  const int kp = wave % KSPLIT, slice = blockIdx.x * CS + wave / KSPLIT;
  int g, r_lo, r_hi;
  int stok[RT];     // SEL: the token of the lane's row in each 16-row tile, -1 past the tile's rows
  int atok[RT];     // SEL: the token whose A row the lane loads (past the rows: the tile's first)
  float scoef[RT];  // SEL: its coefficient (the row scale)
  if constexpr (SEL) {
    g = gy / p.sel_tpg;
    const int tile = gy - g * p.sel_tpg;
    // lane t: c[t, g], token t's selected edges to g summed in order (the
    // destination plan's coefficient, the same operations); sel_km is a
    // multiple of 4 and at most 16
    const int km = p.sel_km, kv = km >> 2;
    const int tt = lane < p.sel_n ? lane : 0;
    const int32_t* si = p.sel_idx + static_cast<int64_t>(tt) * km;
    const float* sw = p.sel_w + static_cast<int64_t>(tt) * km;
    i32x4 iv[4];
    f32x4 wv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {  // unconditional loads at clamped indices
      const int jj = j < kv ? j : kv - 1;
      iv[j] = reinterpret_cast<const i32x4*>(si)[jj];
      wv[j] = reinterpret_cast<const f32x4*>(sw)[jj];
    }
    float c = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (j < kv && iv[j][i] == g) c += wv[j][i];
    const uint64_t mask = __ballot(lane < p.sel_n && c != 0.f);
    const int cnt = __popcll(mask);
    r_lo = 16 * RT * tile;
    if (r_lo >= cnt) return;  // uniform, before any barrier
    r_hi = min(cnt, r_lo + 16 * RT);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int j = r_lo + 16 * rt + l16;
      const int tok = nth_set_bit(mask, j < r_hi ? j : r_lo);  // past the rows: a valid token, never stored
      atok[rt] = tok;
      stok[rt] = j < r_hi ? tok : -1;
      scoef[rt] = __shfl(c, tok);
    }
  } else if (p.G > 0 && gy < p.G) {
    // the first tile of group gy: the weights are requested before its rows
    // are looked up (below)
    g = gy;
    r_lo = r_hi = 0;
  } else {
    // a group's later tiles (rows past its first 16 * RT), in group order
    int m0, mrows;
    if (!find_tile(p, 16 * RT, p.G > 0 ? gy - p.G : gy, g, m0, mrows, p.G > 0 ? 1 : 0))
      return;  // uniform, before any barrier
    r_lo = m0;
    r_hi = m0 + mrows;
  }
  const bool early = !SEL && p.G > 0 && gy < p.G;  // uniform
  int c0[TNW];  // first channel of each tile (slices past N_out: clamped rows, never stored)
#pragma unroll
  for (int t = 0; t < TNW; ++t)
    c0[t] = EPI == EPI_SWIGLU ? 64 * (slice / (4 / TNW)) + 8 * TNW * (slice % (4 / TNW)) +
                                    16 * (t % (TNW / 2)) + 32 * (t / (TNW / 2))
                              : 16 * (TNW * slice + t);
  const uint8_t* wrow[TNW];
  int wn[TNW];
#pragma unroll
  for (int t = 0; t < TNW; ++t) {
    const int n = min(c0[t] + l16, p.N_out - 1);
    wn[t] = n;
    wrow[t] = reinterpret_cast<const uint8_t*>(p.W) +
              (g * p.w_gstride + static_cast<int64_t>(n) * p.ldw) * ESZ2 / 2;
  }
  // weight tile layout: tile t's 64-k step st is block (g * N_out/16 + t) *
  // K/64 + st of BLK bytes, lane l's fragments at 16 l (fp8: 64 k) or at
  // 16 l and 1 KB + 16 l (bf16: k 8q.. and 32 + 8q..)
  const uint8_t* wtile[TNW];
  if constexpr (PK) {
#pragma unroll
    for (int t = 0; t < TNW; ++t) {
      const int tile = min(c0[t], p.N_out - 16) >> 4;
      wtile[t] = reinterpret_cast<const uint8_t*>(p.Wt) +
                 (static_cast<int64_t>(g) * (p.N_out >> 4) + tile) * (p.K >> 6) * BLK + 16 * lane;
    }
  }
  const int steps = p.K / 64;
  const int s_begin = kp * steps / KSPLIT, nst = (kp + 1) * steps / KSPLIT - s_begin;
  const int last = min(s_begin + max(nst - 1, 0), steps - 1);
  DRaw<FMT> wr[D][TNW];
  u32x4 av[D][RT][2];
  const uint16_t* arow[RT];
  auto fetch_w = [&](int d, int i) {  // ring slot d <- step s_begin + i (clamped): weights
    const int k0 = 64 * min(s_begin + i, last);
#pragma unroll
    for (int t = 0; t < TNW; ++t) {
      if constexpr (PK) {
        const uint8_t* blk = wtile[t] + static_cast<int64_t>(k0 >> 6) * BLK;
        wr[d][t].a = *reinterpret_cast<const u32x4*>(blk);
        if constexpr (FMT == SMOE_BF16) wr[d][t].b = *reinterpret_cast<const u32x4*>(blk + 1024);
      } else if constexpr (FMT == SMOE_BF16) {
        wr[d][t].a = *reinterpret_cast<const u32x4*>(wrow[t] + 2 * (k0 + 8 * q));
        wr[d][t].b = *reinterpret_cast<const u32x4*>(wrow[t] + 2 * (k0 + 32 + 8 * q));
      } else if constexpr (FMT == SMOE_FP8_E4M3) {
        wr[d][t].a = *reinterpret_cast<const u32x4*>(wrow[t] + k0 + 16 * q);
      } else {
        const int k = k0 + 16 * q;
        wr[d][t].a = *reinterpret_cast<const u32x2*>(wrow[t] + (k >> 1));
        wr[d][t].s = load_scale(p.S,
                                g * p.s_gstride + static_cast<int64_t>(wn[t]) * (p.K / p.group_size) +
                                    k / p.group_size,
                                p.s_f16);
      }
    }
  };
  auto fetch_a = [&](int d, int i) {  // ... and activations
    const int k0 = 64 * min(s_begin + i, last);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      if constexpr (FMT == SMOE_BF16) {
        av[d][rt][0] = *reinterpret_cast<const u32x4*>(arow[rt] + k0 + 8 * q);
        av[d][rt][1] = *reinterpret_cast<const u32x4*>(arow[rt] + k0 + 32 + 8 * q);
      } else {
        const u32x4* ap = reinterpret_cast<const u32x4*>(arow[rt] + k0 + 16 * q);
        av[d][rt][0] = ap[0];
        av[d][rt][1] = ap[1];
      }
    }
  };
  auto fetch = [&](int d, int i) {
    fetch_w(d, i);
    fetch_a(d, i);
  };
  if (early) {  // the first steps' weights go out before the group's rows are read
#pragma unroll
    for (int d = 0; d < D; ++d) fetch_w(d, d);
    r_lo = p.grp_off[g];
    r_hi = min(p.grp_off[g + 1], r_lo + 16 * RT);
    if (r_hi <= r_lo) return;  // uniform (an empty group), before any barrier
  }
  const uint16_t* A = reinterpret_cast<const uint16_t*>(p.A);
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    int ar;
    if constexpr (SEL) {
      ar = atok[rt];
    } else {
      int r = r_lo + 16 * rt + l16;
      r = r < r_hi ? r : r_lo;  // rows past the tile: a valid row, never stored
      ar = p.a_rows ? p.a_rows[r] : r;
    }
    arow[rt] = A + static_cast<int64_t>(ar) * p.lda;
  }
  f32x4 acc[TNW][RT];
#pragma unroll
  for (int t = 0; t < TNW; ++t)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[t][rt] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto step = [&](int d) {  // widen ring slot d and multiply it into acc
#pragma unroll
    for (int t = 0; t < TNW; ++t) {
      u32x4 l, h;
      if constexpr (FMT == SMOE_BF16) {
        l = wr[d][t].a;
        h = wr[d][t].b;
      } else if constexpr (FMT == SMOE_FP8_E4M3) {
        const u32x2 a0 = fp8x4_to_bf16x4(wr[d][t].a.x), a1 = fp8x4_to_bf16x4(wr[d][t].a.y);
        const u32x2 b0 = fp8x4_to_bf16x4(wr[d][t].a.z), b1 = fp8x4_to_bf16x4(wr[d][t].a.w);
        l = u32x4{a0.x, a0.y, a1.x, a1.y};
        h = u32x4{b0.x, b0.y, b1.x, b1.y};
      } else {
        l = int4x8_to_bf16x8(wr[d][t].a.x, wr[d][t].s);
        h = int4x8_to_bf16x8(wr[d][t].a.y, wr[d][t].s);
      }
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        acc[t][rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8, l), __builtin_bit_cast(bf16x8, av[d][rt][0]), acc[t][rt],
            0, 0, 0);
        acc[t][rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8, h), __builtin_bit_cast(bf16x8, av[d][rt][1]), acc[t][rt],
            0, 0, 0);
      }
    }
  };
  if (early) {
#pragma unroll
    for (int d = 0; d < D; ++d) fetch_a(d, d);
  } else {
#pragma unroll
    for (int d = 0; d < D; ++d) fetch(d, d);  // a slice of < D steps: its last step again (unused)
  }
  int s = 0;
  for (; s + 2 * D <= nst; s += D) {  // slot d holds step s + d; every refill is a real step
#pragma unroll
    for (int d = 0; d < D; ++d) {
      step(d);
      fetch(d, s + d + D);
    }
  }
  // the epilogue's per-channel scales / biases and row weights go out now,
  // behind the slice's last loads, so they land while the last steps run
  float esc[TNW][4], ebi[TNW][4], ers[RT];
#pragma unroll
  for (int t = 0; t < TNW; ++t) {
    const int c = min(c0[t] + 4 * q, p.N_out - 4);
    const bool sw_gate = EPI == EPI_SWIGLU && t < TNW / 2;
    const int bc = EPI == EPI_SWIGLU ? (c >> 6) * 32 + (c & 31) : c;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      esc[t][i] = (FMT == SMOE_FP8_E4M3 && EPI != EPI_ROWSCALE)
                      ? reinterpret_cast<const float*>(p.S)[g * p.s_gstride + c + i]
                      : 1.0f;
      ebi[t][i] = (p.bias && (EPI == EPI_SWIGLU ? sw_gate : EPI != EPI_ROWSCALE))
                      ? p.bias[g * p.bias_gstride + bc + i]
                      : 0.0f;
    }
  }
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int r = min(r_lo + 16 * rt + l16, r_hi - 1);
    if constexpr (SEL) ers[rt] = scoef[rt];
    else ers[rt] = (EPI == EPI_ROWSCALE || EPI == EPI_DOWN) ? p.row_scale[r] : 1.0f;
  }
  // the last 2D - 1 steps at most: refills only where a step is left
#pragma unroll
  for (int d = 0; d < D; ++d) {
    if (s + d < nst) step(d);
    if (s + d + D < nst) fetch(d, s + d + D);
  }
#pragma unroll
  for (int d = 0; d < D - 1; ++d)
    if (s + D + d < nst) step(d);
  if constexpr (KSPLIT > 1) {
    if (kp > 0)
#pragma unroll
      for (int t = 0; t < TNW; ++t)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) red[(wave * TNW * RT + t * RT + rt) * 64 + lane] = acc[t][rt];
    __syncthreads();
    if (kp > 0) return;
#pragma unroll
    for (int j = 1; j < KSPLIT; ++j)
#pragma unroll
      for (int t = 0; t < TNW; ++t)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
          acc[t][rt] += red[((wave + j) * TNW * RT + t * RT + rt) * 64 + lane];
  }
  // lane: channels c0[t] + 4 q + (0..3) of row r_lo + 16 rt + l16.
  // Stores count in vmcnt too: one explicit wait for the epilogue operands
  // here, and the output type resolved outside the loops, keep the compiler
  // from draining each store before the next.
  wait_vmcnt<0>();
  auto emit = [&](auto f32_out) {
    auto put4 = [&](int row, int col, const float (&o)[4]) {
      const int64_t off = static_cast<int64_t>(row) * p.ldo + col;
      if constexpr (decltype(f32_out)::value)
        *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(p.out) + off) = f32x4{o[0], o[1], o[2], o[3]};
      else
        *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(p.out) + off) =
            u32x2{pack_bf2(o[0], o[1]), pack_bf2(o[2], o[3])};
    };
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      int row = r_lo + 16 * rt + l16;
      if constexpr (SEL) {
        if (stok[rt] < 0) continue;
        row = g * p.sel_n + stok[rt];
      } else if (row >= r_hi) {
        continue;
      }
      if constexpr (EPI == EPI_SWIGLU) {
#pragma unroll
        for (int t = 0; t < TNW / 2; ++t) {  // gate tile t, up tile t + TNW / 2
          const int c = c0[t] + 4 * q;
          if (c >= p.N_out) continue;
          float o[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float gs = acc[t][rt][i] * esc[t][i];
            const float us = acc[t + TNW / 2][rt][i] * esc[t + TNW / 2][i] + ebi[t][i];
            o[i] = silu(gs) * us;
          }
          put4(row, (c >> 6) * 32 + (c & 31), o);
        }
      } else {
#pragma unroll
        for (int t = 0; t < TNW; ++t) {
          const int c = c0[t] + 4 * q;
          if (c >= p.N_out) continue;
          float o[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float a = acc[t][rt][i];
            if constexpr (EPI == EPI_ROWSCALE) o[i] = a * ers[rt];
            else if constexpr (EPI == EPI_GELU) o[i] = gelu_erf(a * esc[t][i] + ebi[t][i]);
            else if constexpr (EPI == EPI_DOWN) o[i] = (a * esc[t][i] + ebi[t][i]) * ers[rt];
            else o[i] = a * esc[t][i] + ebi[t][i];  // EPI_F32_BIAS
          }
          put4(row, c, o);
        }
      }
    }
  };
  if (EPI == EPI_F32_BIAS || p.out_dtype == SMOE_F32) emit(std::true_type{});
  else emit(std::false_type{});
}

template <int FMT, int EPI, int TNW, int RT, int KSPLIT, int D, bool PK = false>
__global__ __launch_bounds__(256) void k_gemm_decode(const GemmArgs p) {
  __shared__ f32x4 red[(KSPLIT > 1 ? 4 : 1) * TNW * RT * 64];
  decode_gemm<FMT, EPI, TNW, RT, KSPLIT, D, PK, false>(p, blockIdx.y, red);
}

// The decode edge projection (bf16 weight tiles, row selection from the
// front's top-m) and, in the first workgroup, the loop's plans
// (decode_plan_body; the rest of grid row 0 exits at once).  Row 0 is
// dispatched first, so the plans start with the weight streams even when
// the grid exceeds one round of workgroup slots.  One LDS allocation serves
// either role.
template <int RT, int KSPLIT>
__global__ __launch_bounds__(256) void k_decode_edge(const GemmArgs p, const DecPlan q) {
  constexpr int RED = (KSPLIT > 1 ? 4 : 1) * 4 * RT * 64 * 16;
  constexpr int PLAN = decode_plan_lds_bytes<4>();
  __shared__ __attribute__((aligned(16))) uint8_t lds[RED > PLAN ? RED : PLAN];
  if (blockIdx.y == 0) {  // uniform
    if (blockIdx.x == 0) decode_plan_body<4, 16>(q, lds);
    return;
  }
  decode_gemm<SMOE_BF16, EPI_ROWSCALE, 4, RT, KSPLIT, 3, true, true>(
      p, blockIdx.y - 1, reinterpret_cast<f32x4*>(lds));
}

// ------------------------------------------------------- weight stream ----
// Medium rows per group (a few dozen to ~128: mixed decode + prefill steps),
// bf16 and fp8 weights (int4: k_gemm_stream4 below, the same work split).
// The weights dominate the traffic and every weight is
// used by all rows of its group, so a workgroup owns one group, a strip of
// 256 output channels (wave w: channels 64 w .. 64 w + 63, four 16-channel
// MFMA tiles) and the group's rows in passes of RT*16.  Both operands stream
// global -> LDS by DMA (global_load_lds_dwordx4) through an NS-stage ring of
// 64-wide K chunks, so the main loop's only vector-memory operations are the
// DMAs and the explicit vmcnt waits stay exact:
//   weights:     256 channel rows x 64 k in storage format (fp8 64 B, bf16
//                128 B per row); a lane reads the 16 k at 16*(lane/16) of
//                its channel and widens them to bf16
//   activations: RT*16 rows x 64 k bf16 (128 B rows)
//   MFMAs:       the step's two MFMAs take the low and the high 8 of the 16 k
//                (the same permutation for both operands).
// Every LDS row's 16-byte chunk c is stored at c ^ ((r / R) % C), C chunks
// per row, R rows per 256 bytes: the 16 rows a ds_read phase touches then
// cover all 64 banks once.  One barrier per chunk; chunk k+NS-1 is in flight
// while chunk k computes.  Results go from registers to memory, 4
// consecutive channels per lane.
template <int FMT>
constexpr int stream_wb() {  // bytes of one channel's 64-k slice
  return FMT == SMOE_BF16 ? 128 : (FMT == SMOE_FP8_E4M3 ? 64 : 32);
}
constexpr int kStreamScaleMax = 4096;  // int4 scale-table entries per strip

template <int FMT, int EPI, int RT, int NS, int WGS>
__global__ __launch_bounds__(256, WGS) void k_gemm_stream(const GemmArgs p) {
  constexpr int TN = 4;
  constexpr int WB = stream_wb<FMT>();
  constexpr int CPR = WB / 16;  // 16-byte chunks per weight row
  constexpr int ROWS = RT * 16;
  constexpr int W_BYTES = 256 * WB, A_BYTES = ROWS * 128, STAGE = W_BYTES + A_BYTES;
  constexpr int W_LD = W_BYTES / 4096, A_LD = A_BYTES / 4096;  // DMA instructions per wave per stage
  constexpr int LD = W_LD + A_LD;
  constexpr int ESZ2 = FMT == SMOE_BF16 ? 4 : (FMT == SMOE_FP8_E4M3 ? 2 : 1);  // 2 x bytes/elt
  static_assert(W_BYTES % 4096 == 0 && A_BYTES % 4096 == 0, "whole DMA instructions per wave");
  static_assert(NS >= 3, "ring depth");
  static_assert(EPI != EPI_SWIGLU || TN == 4, "SwiGLU pairs channel c with c + 32");
  static_assert(FMT == SMOE_BF16 || FMT == SMOE_FP8_E4M3, "int4: k_gemm_stream4");
  __shared__ __attribute__((aligned(1024))) uint8_t ring[NS * STAGE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int q = lane >> 4, l16 = lane & 15;
  // (group, strip) of this workgroup: workgroup ids are dealt to the 8 XCDs
  // round robin, so the linear id is split into 8 contiguous ranges of
  // (group, strip) pairs, one per XCD, and a group's strips share one L2
  // (its activation rows come from HBM once instead of once per strip)
  int g, nb;
  {
    const int S = gridDim.x, T = S * gridDim.y;
    const int bid = blockIdx.x + S * blockIdx.y;
    const int x = bid & 7, local = bid >> 3, base = T >> 3, rem = T & 7;
    const int logical = x * base + min(x, rem) + local;
    g = logical / S;
    nb = (logical - g * S) * 256;
  }
  int r_lo, r_hi;
  if (p.G == 0) {
    r_lo = 0;
    r_hi = p.single_rows;
  } else {
    r_lo = p.grp_off[g];
    r_hi = p.grp_off[g + 1];
  }
  if (r_hi <= r_lo) return;  // workgroup-uniform, before any barrier
  const int KC = p.K / 64;
  // weight DMA: instruction j of wave w fills bytes [(4 j + w) KB, +1 KB) of
  // the stage's weight region; lane l writes byte b = that + 16 l, i.e. row
  // b / WB, physical chunk (b % WB) / 16 (which holds the logical chunk the
  // swizzle maps there)
  const uint8_t* wsrc[W_LD];
#pragma unroll
  for (int j = 0; j < W_LD; ++j) {
    const int b = (4 * j + wave) * 1024 + 16 * lane;
    const int row = b / WB, pc = (b % WB) >> 4;
    const int lc = sw_chunk<CPR>(row, pc);  // the map is an involution
    const int n = min(nb + row, p.N_out - 1);  // channels past N_out: loaded, never stored
    wsrc[j] = reinterpret_cast<const uint8_t*>(p.W) +
              (g * p.w_gstride + static_cast<int64_t>(n) * p.ldw) * ESZ2 / 2 + lc * 16;
  }
  const uint16_t* A = reinterpret_cast<const uint16_t*>(p.A);
  for (int m0 = r_lo; m0 < r_hi; m0 += ROWS) {  // passes (uniform)
    // activation DMA: instruction j of wave w covers rows 8 (4 j + w) .. +8,
    // lane l: row + l / 8, physical chunk l % 8
    const uint16_t* asrc[A_LD];
#pragma unroll
    for (int j = 0; j < A_LD; ++j) {
      const int r = 8 * (4 * j + wave) + (lane >> 3);
      const int pr = m0 + r < r_hi ? m0 + r : r_lo;  // rows past the group: valid, never stored
      const int ar = p.a_rows ? p.a_rows[pr] : pr;
      asrc[j] = A + static_cast<int64_t>(ar) * p.lda + (sw_chunk<8>(r, lane & 7) << 3);
    }
    auto issue = [&](int kc) {  // DMA of chunk kc into ring slot kc % NS
      uint8_t* base = ring + (kc % NS) * STAGE;
#pragma unroll
      for (int j = 0; j < W_LD; ++j)
        __builtin_amdgcn_global_load_lds((gbl_vptr)(wsrc[j] + static_cast<int64_t>(kc) * WB),
                                         (lds_vptr)(base + (4 * j + wave) * 1024), 16, 0, 0);
#pragma unroll
      for (int j = 0; j < A_LD; ++j)
        __builtin_amdgcn_global_load_lds((gbl_vptr)(asrc[j] + kc * 64),
                                         (lds_vptr)(base + W_BYTES + (4 * j + wave) * 1024), 16,
                                         0, 0);
    };
    f32x4 acc[TN][RT];
#pragma unroll
    for (int t = 0; t < TN; ++t)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) acc[t][rt] = f32x4{0.f, 0.f, 0.f, 0.f};

    // prologue: chunks 0 .. NS-2 in flight, chunk 0 landed everywhere
#pragma unroll
    for (int st = 0; st < NS - 1; ++st)
      if (st < KC) issue(st);
    if (KC >= NS - 1) wait_vmcnt<(NS - 2) * LD>();
    else wait_vmcnt<0>();
    wait_lgkm0();  // the scale table (int4) is written
    __builtin_amdgcn_s_barrier();
    for (int kc = 0; kc < KC; ++kc) {
      if (kc > 0) {
        // own part of chunk kc landed (kc+1 .. kc+NS-2 may fly); chunk kc-1
        // is no longer read by anyone after the barrier
        if (kc + NS - 2 < KC) wait_vmcnt<(NS - 2) * LD>();
        else wait_vmcnt<0>();
        wait_lgkm0();
        __builtin_amdgcn_s_barrier();
      }
      if (kc + NS - 1 < KC) issue(kc + NS - 1);  // into the slot chunk kc-1 used
      const uint8_t* sw = ring + (kc % NS) * STAGE;
      const uint8_t* sa = sw + W_BYTES;
      bf16x8 wlo[TN], whi[TN];
#pragma unroll
      for (int t = 0; t < TN; ++t) {
        const int row = wave * 64 + t * 16 + l16;
        WRaw<FMT> r;
        if constexpr (FMT == SMOE_BF16) {
          r.a = *reinterpret_cast<const u32x4*>(sw + row * WB + (sw_chunk<CPR>(row, 2 * q) << 4));
          r.b = *reinterpret_cast<const u32x4*>(sw + row * WB + (sw_chunk<CPR>(row, 2 * q + 1) << 4));
        } else {
          r.a = *reinterpret_cast<const u32x4*>(sw + row * WB + (sw_chunk<CPR>(row, q) << 4));
        }
        skinny_wconv<FMT>(r, wlo[t], whi[t]);
      }
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const int r = rt * 16 + l16;
        const bf16x8 blo = *reinterpret_cast<const bf16x8*>(sa + r * 128 + (sw_chunk<8>(r, 2 * q) << 4));
        const bf16x8 bhi = *reinterpret_cast<const bf16x8*>(sa + r * 128 + (sw_chunk<8>(r, 2 * q + 1) << 4));
#pragma unroll
        for (int t = 0; t < TN; ++t) {
          acc[t][rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wlo[t], blo, acc[t][rt], 0, 0, 0);
          acc[t][rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(whi[t], bhi, acc[t][rt], 0, 0, 0);
        }
      }
    }
    // lane: channels nb + 64 wave + 16 t + 4 q + (0..3) of row m0 + 16 rt + l16
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int row = m0 + rt * 16 + l16;
      if (row >= r_hi) continue;
#pragma unroll
      for (int t = 0; t < TN; ++t) {
        const int c = nb + wave * 64 + 16 * t + 4 * q;
        if (c >= p.N_out) continue;
        if constexpr (EPI == EPI_SWIGLU) {
          if (t >= 2) continue;
          const f32x4 v = acc[t][rt], up = acc[t + 2][rt];
          const int u0 = (c >> 6) * 32 + (c & 31);
          float o[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float gs = v[i] * col_scale(p, FMT, g, c + i);
            const float us = up[i] * col_scale(p, FMT, g, c + 32 + i) + bias_at(p, g, u0 + i);
            o[i] = silu(gs) * us;
          }
          const int64_t off = static_cast<int64_t>(row) * p.ldo + u0;
          if (p.out_dtype == SMOE_F32)
            *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(p.out) + off) = f32x4{o[0], o[1], o[2], o[3]};
          else
            *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(p.out) + off) =
                u32x2{pack_bf2(o[0], o[1]), pack_bf2(o[2], o[3])};
        } else {
          store4<EPI>(p, FMT, g, row, c, acc[t][rt]);
        }
      }
    }
    if (m0 + ROWS < r_hi) {  // another pass: every wave is done with the ring
      wait_lgkm0();
      __builtin_amdgcn_s_barrier();
    }
  }
}

// int4 weights at the stream kernel's row counts, with the dequant beside
// the MFMAs instead of before them: inside a chunk the 16 weights of tile
// t+1 are widened (about 3 VALU operations per weight) in the same stretch
// of code as tile t's MFMAs, so the VALU and the matrix pipe of a wave work
// side by side; only tile 0's widening is exposed.  The activation
// fragments of all live row tiles are read once per chunk.  The number of
// live 16-row tiles of a pass is a template parameter (one instantiation per
// count, chosen per pass), so tiles past the group's last row issue neither
// MFMAs nor activation DMA, and the loop body has no branches to split it.
// Waves whose channels all lie past N_out skip the arithmetic.  Work
// split, ring, swizzles and XCD-aware workgroup order are those
// of k_gemm_stream; the strip's group scales sit in an LDS table after the
// ring, in the same LDS object (with a second LDS object the compiler waits
// for every outstanding DMA before reads of the table, draining the ring's
// prefetch).  A wave owns TN 16-channel tiles (a strip of 64 TN channels);
// it brings its own channels' weights into the ring, WWB bytes per chunk in
// 1 KB DMA instructions, the last one on the lanes it needs when TN is odd.
// TN only decides which channels a wave holds: every output is summed in the
// same order, so the bits do not depend on it.
template <int EPI, int RT, int NS = 3, int TN = 4>
__global__ __launch_bounds__(256, 2) void k_gemm_stream4(const GemmArgs p) {
  constexpr int WB = 32, CPR = 2;  // int4: 32 B per channel per 64-k chunk
  constexpr int SW = 64 * TN;      // channels of a strip
  constexpr int ROWS = RT * 16;
  constexpr int WWB = 16 * TN * WB;  // a wave's weight bytes per chunk
  constexpr int W_BYTES = 4 * WWB, A_BYTES = ROWS * 128, STAGE = W_BYTES + A_BYTES;
  constexpr int W_LD = (WWB + 1023) / 1024;                 // DMA instructions per wave
  constexpr int W_TAIL = (WWB - 1024 * (W_LD - 1)) / 16;    // lanes of the last one
  constexpr int SC_BYTES = kStreamScaleMax * 4;
  static_assert(TN == 3 || TN == 4, "48- or 64-channel waves");
  static_assert(RT % 2 == 0 && RT >= 4 && RT <= 6, "whole DMA instructions per wave");
  static_assert(NS * STAGE + SC_BYTES <= 80 * 1024, "two workgroups per CU");
  static_assert(STAGE % 1024 == 0 && W_BYTES % 1024 == 0, "1 KB-aligned DMA bases");
  static_assert(EPI != EPI_SWIGLU || TN == 4, "SwiGLU pairs channel c with c + 32");
  __shared__ __attribute__((aligned(1024))) uint8_t ring[NS * STAGE + SC_BYTES];
  float* sc = reinterpret_cast<float*>(ring + NS * STAGE);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int q = lane >> 4, l16 = lane & 15;
  int g, nb;
  {
    const int S = gridDim.x, T = S * gridDim.y;
    const int bid = blockIdx.x + S * blockIdx.y;
    const int x = bid & 7, local = bid >> 3, base = T >> 3, rem = T & 7;
    const int logical = x * base + min(x, rem) + local;
    g = logical / S;
    nb = (logical - g * S) * SW;
  }
  int r_lo, r_hi;
  if (p.G == 0) {
    r_lo = 0;
    r_hi = p.single_rows;
  } else {
    r_lo = p.grp_off[g];
    r_hi = p.grp_off[g + 1];
  }
  if (r_hi <= r_lo) return;  // workgroup-uniform, before any barrier
  const int KC = p.K / 64;
  const int ng = p.K / p.group_size;
  const int gshift = __builtin_ctz(p.group_size);  // power of two, >= 16 (launcher)
  // the A rows of the first pass, requested beside the scales (its first
  // DMA needs them)
  int arow0[RT / 2];
#pragma unroll
  for (int j = 0; j < RT / 2; ++j) {
    const int r = 8 * (4 * j + wave) + (lane >> 3);
    const int pr = r_lo + r < r_hi ? r_lo + r : r_lo;
    arow0[j] = p.a_rows ? p.a_rows[pr] : pr;
  }
  // the strip's group scales, channel-major [SW][ng]: one contiguous run of
  // the scale array (channels past N_out read the last channel's).  The
  // loads are unconditional (indices clamped) and converted only after the
  // last one is issued, so all are in flight at once; a guarded load with
  // its conversion waits in its own block, one round trip per entry.
  {
    constexpr int SCJ = kStreamScaleMax / 256;
    float scv[SCJ];
    const int64_t sb = g * p.s_gstride + static_cast<int64_t>(nb) * ng;
    const int last = (min(p.N_out, nb + SW) - nb) * ng - 1;
    if (p.s_f16) {
      const _Float16* s16 = reinterpret_cast<const _Float16*>(p.S) + sb;
      _Float16 hv[SCJ];
#pragma unroll
      for (int j = 0; j < SCJ; ++j) hv[j] = s16[min(tid + 256 * j, last)];
#pragma unroll
      for (int j = 0; j < SCJ; ++j) scv[j] = static_cast<float>(hv[j]);
    } else {
      const float* s32 = reinterpret_cast<const float*>(p.S) + sb;
#pragma unroll
      for (int j = 0; j < SCJ; ++j) scv[j] = s32[min(tid + 256 * j, last)];
    }
#pragma unroll
    for (int j = 0; j < SCJ; ++j)
      if (tid + 256 * j < SW * ng) sc[tid + 256 * j] = scv[j];
  }
  const bool live = nb + 16 * TN * wave < p.N_out;  // wave-uniform: some channel of this wave is stored
  // byte b of the strip's row-major [SW][WB] chunk goes to byte b of the
  // ring slot's weight region.  Its first byte for DMA instruction j of this
  // wave: 256 channels, KB 4 j + w; 192 channels, wave w brings bytes
  // [w WWB, (w + 1) WWB) (lanes past the tail of the last instruction are
  // never issued; their address is clamped all the same).
  auto wdst = [&](int j) { return TN == 4 ? (4 * j + wave) * 1024 : wave * WWB + 1024 * j; };
  const uint8_t* wsrc[W_LD];
#pragma unroll
  for (int j = 0; j < W_LD; ++j) {
    const int b = TN == 4 ? wdst(j) + 16 * lane : wave * WWB + min(1024 * j + 16 * lane, WWB - 16);
    const int row = b / WB, pc = (b % WB) >> 4;
    const int lc = sw_chunk<CPR>(row, pc);
    const int n = min(nb + row, p.N_out - 1);  // channels past N_out: loaded, never stored
    wsrc[j] = reinterpret_cast<const uint8_t*>(p.W) +
              (g * p.w_gstride + static_cast<int64_t>(n) * p.ldw) / 2 + lc * 16;
  }
  const uint16_t* A = reinterpret_cast<const uint16_t*>(p.A);
  for (int m0 = r_lo; m0 < r_hi; m0 += ROWS) {  // passes (uniform)
    auto pass = [&](auto live_tiles) {
      constexpr int L = decltype(live_tiles)::value;  // live 16-row tiles of this pass
      constexpr int A_LD = (L + 1) / 2, LD = W_LD + A_LD;  // a DMA instruction of the 4 waves: 32 rows
      const uint16_t* asrc[A_LD];
#pragma unroll
      for (int j = 0; j < A_LD; ++j) {
        const int r = 8 * (4 * j + wave) + (lane >> 3);
        const int pr = m0 + r < r_hi ? m0 + r : r_lo;  // rows past the group: valid, never stored
        const int ar = m0 == r_lo ? arow0[j] : (p.a_rows ? p.a_rows[pr] : pr);
        asrc[j] = A + static_cast<int64_t>(ar) * p.lda + (sw_chunk<8>(r, lane & 7) << 3);
      }
      auto issue = [&](int kc) {  // DMA of chunk kc into ring slot kc % NS
        uint8_t* base = ring + (kc % NS) * STAGE;
#pragma unroll
        for (int j = 0; j < W_LD; ++j)
          if (j + 1 < W_LD || W_TAIL == 64 || lane < W_TAIL)
            __builtin_amdgcn_global_load_lds((gbl_vptr)(wsrc[j] + static_cast<int64_t>(kc) * WB),
                                             (lds_vptr)(base + wdst(j)), 16, 0, 0);
#pragma unroll
        for (int j = 0; j < A_LD; ++j)
          __builtin_amdgcn_global_load_lds((gbl_vptr)(asrc[j] + kc * 64),
                                           (lds_vptr)(base + W_BYTES + (4 * j + wave) * 1024), 16,
                                           0, 0);
      };
      f32x4 acc[TN][L];
#pragma unroll
      for (int t = 0; t < TN; ++t)
#pragma unroll
        for (int rt = 0; rt < L; ++rt) acc[t][rt] = f32x4{0.f, 0.f, 0.f, 0.f};
      // prologue: chunks 0 .. NS-2 in flight, chunk 0 landed everywhere
#pragma unroll
      for (int st = 0; st < NS - 1; ++st)
        if (st < KC) issue(st);
      if (KC >= NS - 1) wait_vmcnt<(NS - 2) * LD>();
      else wait_vmcnt<0>();
      wait_lgkm0();  // the scale table is written
      __builtin_amdgcn_s_barrier();
      for (int kc = 0; kc < KC; ++kc) {
        if (kc > 0) {
          if (kc + NS - 2 < KC) wait_vmcnt<(NS - 2) * LD>();
          else wait_vmcnt<0>();
          wait_lgkm0();
          __builtin_amdgcn_s_barrier();
        }
        if (kc + NS - 1 < KC) issue(kc + NS - 1);  // into the slot chunk kc-1 used
        if (!live) continue;
        const uint8_t* sw = ring + (kc % NS) * STAGE;
        const uint8_t* sa = sw + W_BYTES;
        const int kg = (kc * 64 + 16 * q) >> gshift;  // scale group of this lane's 16 k
        WRaw<SMOE_INT4> wr[TN];
#pragma unroll
        for (int t = 0; t < TN; ++t) {
          const int row = wave * 16 * TN + t * 16 + l16;
          wr[t].a = *reinterpret_cast<const u32x2*>(sw + row * WB + (sw_chunk<CPR>(row, q >> 1) << 4) +
                                                    ((q & 1) << 3));
          wr[t].s = sc[row * ng + kg];
        }
        bf16x8 alo[L], ahi[L];
#pragma unroll
        for (int rt = 0; rt < L; ++rt) {
          const int r = rt * 16 + l16;
          alo[rt] = *reinterpret_cast<const bf16x8*>(sa + r * 128 + (sw_chunk<8>(r, 2 * q) << 4));
          ahi[rt] = *reinterpret_cast<const bf16x8*>(sa + r * 128 + (sw_chunk<8>(r, 2 * q + 1) << 4));
        }
        bf16x8 wlo, whi;
        skinny_wconv<SMOE_INT4>(wr[0], wlo, whi);
#pragma unroll
        for (int t = 0; t < TN; ++t) {
          bf16x8 nlo = wlo, nhi = whi;
          if (t + 1 < TN) skinny_wconv<SMOE_INT4>(wr[t + 1], nlo, nhi);  // beside tile t's MFMAs
#pragma unroll
          for (int rt = 0; rt < L; ++rt) {
            acc[t][rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wlo, alo[rt], acc[t][rt], 0, 0, 0);
            acc[t][rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(whi, ahi[rt], acc[t][rt], 0, 0, 0);
          }
          wlo = nlo;
          whi = nhi;
        }
      }
      // lane: channels nb + 16 TN wave + 16 t + 4 q + (0..3) of row m0 + 16 rt + l16.
      // Its bias values and row weights are loaded before any math (one
      // memory round trip), at clamped indices for rows / channels never
      // stored.
      if (!live) return;
      constexpr bool HAS_RS = EPI == EPI_DOWN || EPI == EPI_ROWSCALE;
      f32x4 bq[TN];
#pragma unroll
      for (int t = 0; t < TN; ++t) {
        const int c = min(nb + wave * 16 * TN + 16 * t + 4 * q, p.N_out - 4);
        const int b0 = EPI == EPI_SWIGLU ? (c >> 6) * 32 + (c & 31) : c;
        bq[t] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (EPI != EPI_ROWSCALE && (EPI != EPI_SWIGLU || t < 2) && p.bias)
          bq[t] = *reinterpret_cast<const f32x4*>(p.bias + g * p.bias_gstride + b0);
      }
      float rsv[L];
#pragma unroll
      for (int rt = 0; rt < L; ++rt)
        rsv[rt] = HAS_RS ? p.row_scale[min(m0 + rt * 16 + l16, r_hi - 1)] : 1.f;
      // Stores count in vmcnt too: with a load still outstanding at a join
      // below, the compiler's wait there would also drain every store before
      // it.  One explicit wait here, and the output type resolved outside
      // the loops, leave the stores unserialised.
      wait_vmcnt<0>();
      auto emit = [&](auto f32_out) {
#pragma unroll
        for (int rt = 0; rt < L; ++rt) {
          const int row = m0 + rt * 16 + l16;
          if (row >= r_hi) continue;
#pragma unroll
          for (int t = 0; t < TN; ++t) {
            const int c = nb + wave * 16 * TN + 16 * t + 4 * q;
            if (c >= p.N_out || (EPI == EPI_SWIGLU && t >= 2)) continue;
            const f32x4 v = acc[t][rt];
            float o[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              if constexpr (EPI == EPI_SWIGLU) o[i] = silu(v[i]) * (acc[t + 2][rt][i] + bq[t][i]);
              else if constexpr (EPI == EPI_GELU) o[i] = gelu_erf(v[i] + bq[t][i]);
              else if constexpr (EPI == EPI_DOWN) o[i] = (v[i] + bq[t][i]) * rsv[rt];
              else if constexpr (EPI == EPI_ROWSCALE) o[i] = v[i] * rsv[rt];
              else o[i] = v[i] + bq[t][i];  // EPI_F32_BIAS
            }
            const int col = EPI == EPI_SWIGLU ? (c >> 6) * 32 + (c & 31) : c;
            const int64_t off = static_cast<int64_t>(row) * p.ldo + col;
            if constexpr (decltype(f32_out)::value)
              *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(p.out) + off) = f32x4{o[0], o[1], o[2], o[3]};
            else
              *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(p.out) + off) =
                  u32x2{pack_bf2(o[0], o[1]), pack_bf2(o[2], o[3])};
          }
        }
      };
      if (EPI == EPI_F32_BIAS || p.out_dtype == SMOE_F32) emit(std::true_type{});
      else emit(std::false_type{});
    };
    const int live_rt = min(RT, (r_hi - m0 + 15) >> 4);  // uniform
    switch (live_rt) {  // one instantiation per live tile count
      case 1: pass(std::integral_constant<int, 1>{}); break;
      case 2: pass(std::integral_constant<int, 2>{}); break;
      case 3: pass(std::integral_constant<int, 3>{}); break;
      case 4: pass(std::integral_constant<int, 4>{}); break;
      case 5: pass(std::integral_constant<int, RT >= 5 ? 5 : RT>{}); break;
      default: pass(std::integral_constant<int, RT>{}); break;
    }
    if (m0 + ROWS < r_hi) {  // another pass: every wave is done with the ring
      wait_lgkm0();
      __builtin_amdgcn_s_barrier();
    }
  }
}

// ------------------------------------------------- fp32 / any shape ----
// SIMT tile GEMM with fp32 FMAs: the fp32 models' path (FMT = SMOE_F32, A
// and W fp32) and the fallback for bf16 shapes the MFMA kernels do not take
// (K or a row pitch not a multiple of their vector width; FMT = SMOE_BF16,
// A and W bf16).  Any K and N_out: k past K reads as 0, which leaves every
// sum unchanged (fma(a, 0, acc) == acc).
template <int FMT>
__device__ __forceinline__ float elem(const void* base, int64_t i) {
  if constexpr (FMT == SMOE_F32) return reinterpret_cast<const float*>(base)[i];
  else return bf2f(reinterpret_cast<const uint16_t*>(base)[i]);
}

template <int BM, int BN, int EPI, int FMT>
__global__ __launch_bounds__(256) void k_gemm_simt(const GemmArgs p) {
  constexpr int BK = 16;
  constexpr int TM = BM / 16, TN = BN / 16;
  __shared__ float sA[BK][BM + 4];
  __shared__ float sB[BK][BN + 4];
  int g, m0, mrows;
  if (!find_tile(p, BM, blockIdx.x, g, m0, mrows)) return;
  const int n0 = blockIdx.y * BN;
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const int64_t wbase = g * p.w_gstride;
  float acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = 0.f;
  for (int k0 = 0; k0 < p.K; k0 += BK) {
    for (int e = tid; e < BM * BK; e += 256) {
      const int r = e / BK, kk = e % BK;
      float v = 0.f;
      if (r < mrows && k0 + kk < p.K) {
        const int ar = p.a_rows ? p.a_rows[m0 + r] : (m0 + r);
        v = elem<FMT>(p.A, static_cast<int64_t>(ar) * p.lda + k0 + kk);
      }
      sA[kk][r] = v;
    }
    for (int e = tid; e < BN * BK; e += 256) {
      const int r = e / BK, kk = e % BK;
      sB[kk][r] = (n0 + r < p.N_out && k0 + kk < p.K)
                      ? elem<FMT>(p.W, wbase + static_cast<int64_t>(n0 + r) * p.ldw + k0 + kk)
                      : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < BK; ++kk) {
      float a[TM], b[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) a[i] = sA[kk][ty + 16 * i];
#pragma unroll
      for (int j = 0; j < TN; ++j) b[j] = sB[kk][tx + 16 * j];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int lr = ty + 16 * i;
    if (lr >= mrows) continue;
#pragma unroll
    for (int j = 0; j < TN; ++j)
      if (n0 + tx + 16 * j < p.N_out) epi_one<EPI>(p, FMT, g, m0 + lr, n0 + tx + 16 * j, acc[i][j]);
  }
}

// ------------------------------------------------- weight tile layout ----
// out[(((g*T + t)*S + s)*2 + h)*64 + l][e] = w[g][16t + l%16][64s + 32h + 8(l/16) + e]
// (T = N/16, S = K/64): one thread per 16-byte fragment, 16-byte reads from
// the row-major weights, contiguous writes.
// One thread per 16-byte fragment f: block (g*T + t)*C + c (16 rows x 64
// bytes of row bytes 64c..64c+63), lane l = 16q + r taking row r's bytes
// 64c + 16q .. +15.  rb = bytes per row (K x element size).
__global__ __launch_bounds__(256) void k_pack_weight_tiles(const uint8_t* __restrict__ w,
                                                          int64_t frags, int N, int rb,
                                                          uint8_t* __restrict__ out) {
  const int64_t f = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (f >= frags) return;
  const int l = static_cast<int>(f & 63);
  const int64_t blk = f >> 6;  // (g*T + t)*C + c
  const int C = rb / 64, T = N / 16;
  const int c = static_cast<int>(blk % C);
  const int64_t gt = blk / C;  // g*T + t
  const int64_t g = gt / T, t = gt % T;
  const int64_t row = g * N + 16 * t + (l & 15);
  *reinterpret_cast<u32x4*>(out + f * 16) =
      *reinterpret_cast<const u32x4*>(w + row * rb + 64 * c + 16 * (l >> 4));
}

int launch_pack_weight_tiles(const void* w, int fmt, int G, int N, int K, void* out, hipStream_t s) {
  if (fmt != SMOE_BF16 && fmt != SMOE_FP8_E4M3) return SMOE_EUNSUPPORTED;
  if (!w || !out || G < 1 || N < 16 || K < 64 || N % 16 || K % 64) return SMOE_EINVAL;
  if (reinterpret_cast<uintptr_t>(w) % 16 || reinterpret_cast<uintptr_t>(out) % 16) return SMOE_EINVAL;
  const int rb = fmt == SMOE_BF16 ? 2 * K : K;
  const int64_t frags = static_cast<int64_t>(G) * N * rb / 16;
  hipLaunchKernelGGL(k_pack_weight_tiles, dim3(static_cast<unsigned>((frags + 255) / 256)), dim3(256),
                     0, s, reinterpret_cast<const uint8_t*>(w), frags, N, rb,
                     reinterpret_cast<uint8_t*>(out));
  return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
}

// int4 weights (packed [G, N, K/2], element 2i in the low nibble of byte i)
// -> the int4 tile layout the ping-pong GEMM reads, the same bytes
// rearranged: per group, per 64-row quad Q and 32-k stage st, a 1 KB block
// ((g * N/64 + Q) * K/32 + st) * 1024 holding the quad's four 16-row tiles
// (256 B each) of lane-ordered MFMA fragments: lane l of tile t takes the 4
// packed bytes of row 64 Q + 16 t + l % 16 that hold k = 32 st + 8 (l / 16)
// .. +7.  A stage of a 256-channel tile is then four contiguous 1 KB DMAs,
// and a lane's fragment one 4-byte LDS read.  One thread per 4-byte word.
__global__ __launch_bounds__(256) void k_pack_int4_qtiles(const uint8_t* __restrict__ q,
                                                          int64_t words, int N, int K,
                                                          uint8_t* __restrict__ out) {
  const int64_t f = blockIdx.x * static_cast<int64_t>(256) + threadIdx.x;
  if (f >= words) return;
  const int l = static_cast<int>(f & 63);
  const int t = static_cast<int>((f >> 6) & 3);
  const int64_t blk = f >> 8;  // (g * N/64 + Q) * K/32 + st
  const int S = K / 32, QN = N / 64;
  const int st = static_cast<int>(blk % S);
  const int64_t gq = blk / S;
  const int64_t g = gq / QN, qd = gq % QN;
  const int64_t row = g * N + 64 * qd + 16 * t + (l & 15);
  const int k = 32 * st + 8 * (l >> 4);
  *reinterpret_cast<uint32_t*>(out + f * 4) =
      *reinterpret_cast<const uint32_t*>(q + row * (K / 2) + k / 2);
}

int launch_pack_int4_qtiles(const void* q, int G, int N, int K, void* out, hipStream_t s) {
  if (!q || !out || G < 1 || N < 64 || K < 32 || N % 64 || K % 32) return SMOE_EINVAL;
  if (reinterpret_cast<uintptr_t>(q) % 4 || reinterpret_cast<uintptr_t>(out) % 16) return SMOE_EINVAL;
  const int64_t words = static_cast<int64_t>(G) * N * K / 8;
  hipLaunchKernelGGL(k_pack_int4_qtiles, dim3(static_cast<unsigned>((words + 255) / 256)), dim3(256),
                     0, s, reinterpret_cast<const uint8_t*>(q), words, N, K,
                     reinterpret_cast<uint8_t*>(out));
  return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
}

// --------------------------------------------------------------- launch ----
namespace {

int max_tiles(const GemmArgs& a, int BM) {
  if (a.G == 0) return (a.single_rows + BM - 1) / BM;
  // band-aligned tiles start up to 15 rows before their group
  const int pad = (a.At || a.out_tiles) ? 15 * a.G : 0;
  return (a.max_rows + pad + BM - 1) / BM + a.G;
}

template <int BM, int BN, int BK, int WM, int WN, int FMT>
int launch_mfma_fmt(const GemmArgs& a, hipStream_t s) {
  const dim3 grid(max_tiles(a, BM), (a.N_out + BN - 1) / BN);
  const dim3 block(WM * WN * 64);
  if (grid.x == 0) return SMOE_OK;
  switch (a.epi) {
    case EPI_F32_BIAS: SMOE_LAUNCH((k_gemm_mfma<BM, BN, BK, WM, WN, FMT, EPI_F32_BIAS>), grid, block, 0, s, a); break;
    case EPI_ROWSCALE: SMOE_LAUNCH((k_gemm_mfma<BM, BN, BK, WM, WN, FMT, EPI_ROWSCALE>), grid, block, 0, s, a); break;
    case EPI_GELU: SMOE_LAUNCH((k_gemm_mfma<BM, BN, BK, WM, WN, FMT, EPI_GELU>), grid, block, 0, s, a); break;
    case EPI_DOWN: SMOE_LAUNCH((k_gemm_mfma<BM, BN, BK, WM, WN, FMT, EPI_DOWN>), grid, block, 0, s, a); break;
    case EPI_SWIGLU:
      if constexpr ((BN / WN) % 64 == 0) {
        SMOE_LAUNCH((k_gemm_mfma<BM, BN, BK, WM, WN, FMT, EPI_SWIGLU>), grid, block, 0, s, a);
        break;
      }
      return SMOE_EINVAL;
    default: return SMOE_EINVAL;
  }
  return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
}

template <int BM, int BN, int BK, int WM, int WN>
int launch_mfma(const GemmArgs& a, hipStream_t s) {
  switch (a.fmt) {
    case SMOE_BF16: return launch_mfma_fmt<BM, BN, BK, WM, WN, SMOE_BF16>(a, s);
    case SMOE_FP8_E4M3: return launch_mfma_fmt<BM, BN, BK, WM, WN, SMOE_FP8_E4M3>(a, s);
    case SMOE_INT4: return launch_mfma_fmt<BM, BN, BK, WM, WN, SMOE_INT4>(a, s);
    default: return SMOE_EUNSUPPORTED;
  }
}

template <int BN, int NS, int GM, bool PK>
int launch_ring_fmt(const GemmArgs& a, hipStream_t s) {
  const int tiles = max_tiles(a, 256) * ((a.N_out + BN - 1) / BN);
  if (tiles == 0) return SMOE_OK;
  const dim3 grid(tiles), block(256);
  switch (a.epi) {
    case EPI_F32_BIAS: SMOE_LAUNCH((k_gemm_ring<BN, NS, GM, EPI_F32_BIAS, PK>), grid, block, 0, s, a); break;
    case EPI_ROWSCALE: SMOE_LAUNCH((k_gemm_ring<BN, NS, GM, EPI_ROWSCALE, PK>), grid, block, 0, s, a); break;
    case EPI_GELU: SMOE_LAUNCH((k_gemm_ring<BN, NS, GM, EPI_GELU, PK>), grid, block, 0, s, a); break;
    case EPI_SWIGLU: SMOE_LAUNCH((k_gemm_ring<BN, NS, GM, EPI_SWIGLU, PK>), grid, block, 0, s, a); break;
    case EPI_DOWN: SMOE_LAUNCH((k_gemm_ring<BN, NS, GM, EPI_DOWN, PK>), grid, block, 0, s, a); break;
    default: return SMOE_EINVAL;
  }
  return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
}

// bf16 weights with a weight tile copy: contiguous 1 KB weight-operand DMA
template <int BN, int NS, int GM>
int launch_ring(const GemmArgs& a, hipStream_t s) {
  return a.Wt && a.fmt == SMOE_BF16 && a.N_out % 16 == 0 ? launch_ring_fmt<BN, NS, GM, true>(a, s)
                                   : launch_ring_fmt<BN, NS, GM, false>(a, s);
}

template <int NS, int GM, int BM, bool PK>
int launch_pp_fmt(const GemmArgs& a, hipStream_t s) {
  const int tiles = max_tiles(a, BM) * ((a.N_out + 255) / 256);
  if (tiles == 0) return SMOE_OK;
  const dim3 grid(tiles), block(512);
  switch (a.epi) {
    case EPI_ROWSCALE: SMOE_LAUNCH((k_gemm_pp<NS, GM, EPI_ROWSCALE, BM, PK>), grid, block, 0, s, a); break;
    case EPI_GELU: SMOE_LAUNCH((k_gemm_pp<NS, GM, EPI_GELU, BM, PK>), grid, block, 0, s, a); break;
    case EPI_SWIGLU: SMOE_LAUNCH((k_gemm_pp<NS, GM, EPI_SWIGLU, BM, PK>), grid, block, 0, s, a); break;
    case EPI_DOWN: SMOE_LAUNCH((k_gemm_pp<NS, GM, EPI_DOWN, BM, PK>), grid, block, 0, s, a); break;
    default: return SMOE_EINVAL;
  }
  return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
}

// fp8-e4m3 weights (their tile copy; the expert FFN's epilogues)
template <int NS, int GM, int BM>
int launch_pp_fp8(const GemmArgs& a, hipStream_t s) {
  const int tiles = max_tiles(a, BM) * ((a.N_out + 255) / 256);
  if (tiles == 0) return SMOE_OK;
  const dim3 grid(tiles), block(512);
  constexpr int F8 = SMOE_FP8_E4M3;
  switch (a.epi) {
    case EPI_GELU: SMOE_LAUNCH((k_gemm_pp<NS, GM, EPI_GELU, BM, true, F8>), grid, block, 0, s, a); break;
    case EPI_SWIGLU: SMOE_LAUNCH((k_gemm_pp<NS, GM, EPI_SWIGLU, BM, true, F8>), grid, block, 0, s, a); break;
    case EPI_DOWN: SMOE_LAUNCH((k_gemm_pp<NS, GM, EPI_DOWN, BM, true, F8>), grid, block, 0, s, a); break;
    default: return SMOE_EINVAL;
  }
  return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
}

// bf16 weights with a weight tile copy: the W operand's DMA reads each
// 16-row x 32-k block as one contiguous 1 KB of lane-ordered fragments;
// fp8 weights always come from their tile copy
// int4 weights (their int4 tile copy; the expert FFN's epilogues)
template <int NS, int GM, int BM>
int launch_pp_int4(const GemmArgs& a, hipStream_t s) {
  const int tiles = max_tiles(a, BM) * ((a.N_out + 255) / 256);
  if (tiles == 0) return SMOE_OK;
  const dim3 grid(tiles), block(512);
  constexpr int I4 = SMOE_INT4;
  switch (a.epi) {
    case EPI_GELU: SMOE_LAUNCH((k_gemm_pp<NS, GM, EPI_GELU, BM, true, I4>), grid, block, 0, s, a); break;
    case EPI_SWIGLU: SMOE_LAUNCH((k_gemm_pp<NS, GM, EPI_SWIGLU, BM, true, I4>), grid, block, 0, s, a); break;
    case EPI_DOWN: SMOE_LAUNCH((k_gemm_pp<NS, GM, EPI_DOWN, BM, true, I4>), grid, block, 0, s, a); break;
    default: return SMOE_EINVAL;
  }
  return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
}

template <int NS, int GM, int BM>
int launch_pp(const GemmArgs& a, hipStream_t s) {
  if (a.fmt == SMOE_FP8_E4M3) return launch_pp_fp8<NS, GM, BM>(a, s);
  if (a.fmt == SMOE_INT4) return launch_pp_int4<NS, GM, BM>(a, s);
  return a.Wt && a.fmt == SMOE_BF16 && a.N_out % 16 == 0 ? launch_pp_fmt<NS, GM, BM, true>(a, s)
                                   : launch_pp_fmt<NS, GM, BM, false>(a, s);
}

template <int BM, int BN, int FMT>
int launch_simt_bn(const GemmArgs& a, hipStream_t s) {
  const dim3 grid(max_tiles(a, BM), (a.N_out + BN - 1) / BN);
  if (grid.x == 0) return SMOE_OK;
  switch (a.epi) {
    case EPI_F32_BIAS: SMOE_LAUNCH((k_gemm_simt<BM, BN, EPI_F32_BIAS, FMT>), grid, dim3(256), 0, s, a); break;
    case EPI_ROWSCALE: SMOE_LAUNCH((k_gemm_simt<BM, BN, EPI_ROWSCALE, FMT>), grid, dim3(256), 0, s, a); break;
    case EPI_GELU: SMOE_LAUNCH((k_gemm_simt<BM, BN, EPI_GELU, FMT>), grid, dim3(256), 0, s, a); break;
    case EPI_DOWN: SMOE_LAUNCH((k_gemm_simt<BM, BN, EPI_DOWN, FMT>), grid, dim3(256), 0, s, a); break;
    default: return SMOE_EUNSUPPORTED;  // SwiGLU pairs need the MFMA kernels' shapes
  }
  return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
}

template <int FMT>
int launch_simt(const GemmArgs& a, hipStream_t s) {
  if (a.N_out <= 16) return launch_simt_bn<64, 16, FMT>(a, s);
  if (a.N_out <= 32) return launch_simt_bn<64, 32, FMT>(a, s);
  return launch_simt_bn<64, 64, FMT>(a, s);
}

template <int FMT, int RT, int KSPLIT, bool PK>
int launch_decode_fmt(const GemmArgs& a, hipStream_t s) {
  // one workgroup per (4 / KSPLIT slices of 64 channels, tile of 16*RT rows);
  // 3 steps in flight per wave
  constexpr int TNW = 4, D = 3, CS = 4 / KSPLIT;
  const int tiles = max_tiles(a, 16 * RT);
  if (tiles == 0) return SMOE_OK;
  const int slices = (a.N_out + 16 * TNW - 1) / (16 * TNW);
  const dim3 grid((slices + CS - 1) / CS, tiles, 1);
  switch (a.epi) {
    case EPI_F32_BIAS: SMOE_LAUNCH((k_gemm_decode<FMT, EPI_F32_BIAS, TNW, RT, KSPLIT, D, PK>), grid, dim3(256), 0, s, a); break;
    case EPI_ROWSCALE: SMOE_LAUNCH((k_gemm_decode<FMT, EPI_ROWSCALE, TNW, RT, KSPLIT, D, PK>), grid, dim3(256), 0, s, a); break;
    case EPI_GELU: SMOE_LAUNCH((k_gemm_decode<FMT, EPI_GELU, TNW, RT, KSPLIT, D, PK>), grid, dim3(256), 0, s, a); break;
    case EPI_DOWN: SMOE_LAUNCH((k_gemm_decode<FMT, EPI_DOWN, TNW, RT, KSPLIT, D, PK>), grid, dim3(256), 0, s, a); break;
    case EPI_SWIGLU: SMOE_LAUNCH((k_gemm_decode<FMT, EPI_SWIGLU, TNW, RT, KSPLIT, D, PK>), grid, dim3(256), 0, s, a); break;
    default: return SMOE_EINVAL;
  }
  return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
}

template <int FMT, int RT, bool PK = false>
int launch_decode_split(const GemmArgs& a, int ksplit, hipStream_t s) {
  if (ksplit == 1) return launch_decode_fmt<FMT, RT, 1, PK>(a, s);
  if (ksplit == 2) return launch_decode_fmt<FMT, RT, 2, PK>(a, s);
  return launch_decode_fmt<FMT, RT, 4, PK>(a, s);
}

}  // namespace

int device_cus();

// Decode weight streams (few rows per group, N_out >= 128): 64 channels per
// wave and K split over the fewest waves (1, 2 or 4) that still give the
// chip 8 waves per CU, each part keeping >= 3 steps.  C2's up GEMM (88 x 64
// channels x 16 groups, K 1024) takes a split of 2: 19.9 us against 22.3 at
// 4 and 23.7 at 1; its down and edge GEMMs (16 x 64 channels x 16 groups)
// take 4: 11.3 us against 16.8 at 2.  64-channel slices beat 32-channel
// ones (half the activation loads per weight byte), and a ring of 3 steps
// beats 2 and 4.
int launch_decode(const GemmArgs& a, hipStream_t s) {
  // 32-row tiles above 8 rows per group on average: routed groups are ragged,
  // and a group past its tile takes a second tile that streams the same
  // weights again (C2's destination groups, 16 rows on average: 12.4 us with
  // 16-row tiles)
  const int rpg = a.G == 0 ? a.single_rows : a.max_rows / a.G;
  const int rt = rpg <= 8 ? 1 : 2;
  const int steps = a.K / 64;
  // waves per split: 64-channel strips x row tiles (every group of a dispatch
  // holds at least one tile, ragged groups rarely more at these sizes)
  const int tiles = a.G == 0 ? (a.single_rows + 16 * rt - 1) / (16 * rt)
                             : max(min(a.G, a.max_rows), (a.max_rows + 16 * rt - 1) / (16 * rt));
  const long long strips = (long long)((a.N_out + 63) / 64) * tiles;
  const int cus = device_cus();
  const long long want = 8LL * (cus > 0 ? cus : 256);
  int ksplit = 1;
  while (ksplit < 4 && strips * ksplit < want && steps / (2 * ksplit) >= 3) ksplit *= 2;
  switch (a.fmt) {
    case SMOE_BF16:
      if (a.Wt && a.N_out % 16 == 0)  // the weight tile layout: contiguous 1 KB loads
        return rt == 1 ? launch_decode_split<SMOE_BF16, 1, true>(a, ksplit, s)
                       : launch_decode_split<SMOE_BF16, 2, true>(a, ksplit, s);
      return rt == 1 ? launch_decode_split<SMOE_BF16, 1>(a, ksplit, s)
                     : launch_decode_split<SMOE_BF16, 2>(a, ksplit, s);
    case SMOE_FP8_E4M3:
      if (a.Wt && a.N_out % 16 == 0)
        return rt == 1 ? launch_decode_split<SMOE_FP8_E4M3, 1, true>(a, ksplit, s)
                       : launch_decode_split<SMOE_FP8_E4M3, 2, true>(a, ksplit, s);
      return rt == 1 ? launch_decode_split<SMOE_FP8_E4M3, 1>(a, ksplit, s)
                     : launch_decode_split<SMOE_FP8_E4M3, 2>(a, ksplit, s);
    case SMOE_INT4:
      return rt == 1 ? launch_decode_split<SMOE_INT4, 1>(a, ksplit, s)
                     : launch_decode_split<SMOE_INT4, 2>(a, ksplit, s);
    default: return SMOE_EUNSUPPORTED;
  }
}

template <int FMT, int TN, int RT, int NW, int U>
int launch_skinny_fmt(const GemmArgs& a, hipStream_t s) {
  // one workgroup per (strip of 16*TN channels, tile of 16*RT rows)
  const int tiles = max_tiles(a, 16 * RT);
  if (tiles == 0) return SMOE_OK;
  const dim3 grid((a.N_out + 16 * TN - 1) / (16 * TN), tiles, 1);
  const dim3 block(NW * 64);
  switch (a.epi) {
    case EPI_F32_BIAS: SMOE_LAUNCH((k_gemm_skinny<FMT, EPI_F32_BIAS, TN, RT, NW, U>), grid, block, 0, s, a); break;
    case EPI_ROWSCALE: SMOE_LAUNCH((k_gemm_skinny<FMT, EPI_ROWSCALE, TN, RT, NW, U>), grid, block, 0, s, a); break;
    case EPI_GELU: SMOE_LAUNCH((k_gemm_skinny<FMT, EPI_GELU, TN, RT, NW, U>), grid, block, 0, s, a); break;
    case EPI_DOWN: SMOE_LAUNCH((k_gemm_skinny<FMT, EPI_DOWN, TN, RT, NW, U>), grid, block, 0, s, a); break;
    case EPI_SWIGLU:
      if constexpr (TN == 4) {
        SMOE_LAUNCH((k_gemm_skinny<FMT, EPI_SWIGLU, TN, RT, NW, U>), grid, block, 0, s, a);
        break;
      }
      return SMOE_EINVAL;
    default: return SMOE_EINVAL;
  }
  return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
}

template <int TN, int RT>
int launch_skinny(const GemmArgs& a, hipStream_t s) {
  switch (a.fmt) {
    case SMOE_BF16: return launch_skinny_fmt<SMOE_BF16, TN, RT, 4, 2>(a, s);
    case SMOE_FP8_E4M3: return launch_skinny_fmt<SMOE_FP8_E4M3, TN, RT, 4, 4>(a, s);
    case SMOE_INT4: return launch_skinny_fmt<SMOE_INT4, TN, RT, 4, 4>(a, s);
    default: return SMOE_EUNSUPPORTED;
  }
}

template <int FMT, int RT, int NS, int WGS>
int launch_stream_fmt(const GemmArgs& a, hipStream_t s) {
  const dim3 grid((a.N_out + 255) / 256, a.G == 0 ? 1 : a.G), block(256);
  switch (a.epi) {
    case EPI_F32_BIAS: SMOE_LAUNCH((k_gemm_stream<FMT, EPI_F32_BIAS, RT, NS, WGS>), grid, block, 0, s, a); break;
    case EPI_ROWSCALE: SMOE_LAUNCH((k_gemm_stream<FMT, EPI_ROWSCALE, RT, NS, WGS>), grid, block, 0, s, a); break;
    case EPI_GELU: SMOE_LAUNCH((k_gemm_stream<FMT, EPI_GELU, RT, NS, WGS>), grid, block, 0, s, a); break;
    case EPI_SWIGLU: SMOE_LAUNCH((k_gemm_stream<FMT, EPI_SWIGLU, RT, NS, WGS>), grid, block, 0, s, a); break;
    case EPI_DOWN: SMOE_LAUNCH((k_gemm_stream<FMT, EPI_DOWN, RT, NS, WGS>), grid, block, 0, s, a); break;
    default: return SMOE_EINVAL;
  }
  return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
}

template <int RT, int NS = 3, int TN = 4>
int launch_stream4(const GemmArgs& a, hipStream_t s) {
  const dim3 grid((a.N_out + 64 * TN - 1) / (64 * TN), a.G == 0 ? 1 : a.G), block(256);
  switch (a.epi) {
    case EPI_F32_BIAS: SMOE_LAUNCH((k_gemm_stream4<EPI_F32_BIAS, RT, NS, TN>), grid, block, 0, s, a); break;
    case EPI_ROWSCALE: SMOE_LAUNCH((k_gemm_stream4<EPI_ROWSCALE, RT, NS, TN>), grid, block, 0, s, a); break;
    case EPI_GELU: SMOE_LAUNCH((k_gemm_stream4<EPI_GELU, RT, NS, TN>), grid, block, 0, s, a); break;
    case EPI_SWIGLU:
      if constexpr (TN == 4) {
        SMOE_LAUNCH((k_gemm_stream4<EPI_SWIGLU, RT, NS, TN>), grid, block, 0, s, a);
        break;
      }
      return SMOE_EINVAL;
    case EPI_DOWN: SMOE_LAUNCH((k_gemm_stream4<EPI_DOWN, RT, NS, TN>), grid, block, 0, s, a); break;
    default: return SMOE_EINVAL;
  }
  return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
}

// The int4 strip width: 256 channels (four 64-channel waves), or 192 where
// that fills the two workgroup slots per CU in fewer rounds of less work
// each (C4's up GEMM, N_out 1408 over 64 groups: 6 strips of 256 fill 384 of
// 512 slots, where the 128 CUs holding two workgroups set the time; 8 strips
// of 192 fill all 512 with three quarters of the work each).  The cost of a
// width is its rounds of workgroups times the work of one.
int stream4_tn(const GemmArgs& a) {
  if (a.epi == EPI_SWIGLU) return 4;
  const int cus = device_cus();
  const long long slots = 2LL * (cus > 0 ? cus : 256);
  const long long groups = a.G == 0 ? 1 : a.G;
  auto cost = [&](int tn) {
    const long long wgs = (a.N_out + 64LL * tn - 1) / (64LL * tn) * groups;
    return (wgs + slots - 1) / slots * tn;
  };
  return cost(3) < cost(4) ? 3 : 4;
}

// Two workgroups per CU (one's dequant and waits overlap the other's MFMAs):
// LDS per workgroup int4 3 x 20 KB + 16 KB scales, fp8 3 x 24 KB (64-row
// passes), bf16 3 x 40 KB (one workgroup per CU).
int launch_stream(const GemmArgs& a, hipStream_t s) {
  switch (a.fmt) {
    case SMOE_BF16: return launch_stream_fmt<SMOE_BF16, 4, 3, 1>(a, s);
    case SMOE_FP8_E4M3: return launch_stream_fmt<SMOE_FP8_E4M3, 4, 3, 2>(a, s);
    case SMOE_INT4:
      if (256 * (a.K / a.group_size) > kStreamScaleMax || (a.group_size & (a.group_size - 1)))
        return SMOE_EUNSUPPORTED;
      return stream4_tn(a) == 3 ? launch_stream4<6, 3, 3>(a, s) : launch_stream4<6>(a, s);
    default: return SMOE_EUNSUPPORTED;
  }
}

// Whether the weight-streaming kernels can take the GEMM: every 16-byte
// (int4: 8-byte) load they issue aligned, K in 64-wide steps.
bool stream_aligned(const GemmArgs& a) {
  if (a.K % 64 || a.N_out % 4 || a.ldo % 4 || a.lda % 8) return false;
  const int walign = a.fmt == SMOE_BF16 ? 8 : 16;  // elements per aligned load
  if (a.ldw % walign || a.w_gstride % walign) return false;
  if (a.fmt == SMOE_INT4 && a.group_size % 16) return false;
  if (a.bias && a.bias_gstride % 4) return false;  // 16-byte bias loads (int4 epilogue)
  return a.fmt == SMOE_BF16 || a.fmt == SMOE_FP8_E4M3 || a.fmt == SMOE_INT4;
}

// Whether every 16-byte (int4: 8-byte) load the skinny kernel issues is
// aligned and K comes in 64-wide steps.
bool skinny_aligned(const GemmArgs& a) {
  if (a.K % 64 || a.N_out % 4 || a.ldo % 4 || a.lda % 8) return false;
  const int walign = a.fmt == SMOE_BF16 ? 8 : 16;  // elements per aligned load
  if (a.ldw % walign || a.w_gstride % walign) return false;
  if (a.fmt == SMOE_INT4 && a.group_size % 16) return false;
  return a.fmt == SMOE_BF16 || a.fmt == SMOE_FP8_E4M3 || a.fmt == SMOE_INT4;
}

// Whether the skinny kernel takes the GEMM as a weight stream: few rows per
// group, aligned.
bool skinny_fits(const GemmArgs& a) {
  const int rows_per_group = a.G == 0 ? a.single_rows : a.max_rows / a.G;
  if (rows_per_group > (a.G == 0 ? 64 : 32)) return false;
  return skinny_aligned(a);
}

int launch_front_gemm(const GemmArgs& a, hipStream_t s) {
  if (a.fmt != SMOE_BF16 || a.epi != EPI_F32_BIAS || a.G != 0 || a.single_rows < 1 ||
      a.single_rows > kFrontMaxN || !a.A || !a.W || !a.out || a.N_out <= 0)
    return SMOE_EINVAL;
  if (a.W2 && (a.n_split < 0 || a.n_split > a.N_out || a.n_split % 4 || a.ldw2 % 8))
    return SMOE_EINVAL;
  if (a.K % 64 || a.N_out % 4 || a.ldo % 4 || a.lda % 8 || a.ldw % 8) return SMOE_EINVAL;
  // 16 channels and 16 rows per workgroup: the few hundred output channels
  // and up to 4 row tiles spread over enough workgroups to stream the
  // weights at a useful rate; each wave requests its 4 K steps at once
  // (C2's 64 x 272 front: 4.5 us against 5.6 with 32-row tiles and 2-step
  // batches)
  return launch_skinny_fmt<SMOE_BF16, 1, 1, 4, 4>(a, s);
}

// CUs of the current device (cached per device; 0 if unknown).
int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cus[dev] = n;
  }
  return cus[dev];
}

// 320- or 256-row ping-pong tiles for groups of >= 512 rows: the estimated
// tile count (each group's last tile partial) in rounds of one workgroup per
// CU, a 320-row round costing 1.15 256-row rounds (measured at 2048-row
// groups, K 2816, and with the SwiGLU epilogue at K 1024: C1 up 393 -> 383 us
// per launch; C3 down, K 1408: 0.928 -> 0.895 ms per step).  The edge
// projections (C1 / C3, K 1024) measured slower with 320 rows (C1 124 ->
// 143 us per launch): their worst-case rows per group (N*S / E) overstate the
// real ones, so the estimate picks 320 where 256 already had few rounds.
bool pp_rows_320(const GemmArgs& a, int rpg) {
  const int cus = device_cus();
  if (cus <= 0) return false;
  const int64_t groups = a.G == 0 ? 1 : a.G, tn = (a.N_out + 255) / 256;
  auto rounds = [&](int bm) {
    const int64_t tiles = groups * (rpg / bm + 1) * tn;
    return (tiles + cus - 1) / cus;
  };
  return 115 * rounds(320) < 100 * rounds(256);
}

// Weights the ping-pong kernels read: bf16; fp8-e4m3 from its tile copy;
// int4 from its int4 tile copy, with 32 | group_size and at most
// kPpScaleMax / 256 scale groups along K (neither for the edge
// projection's row-scale epilogue).
bool pp_weights(const GemmArgs& a) {
  if (a.fmt == SMOE_INT4)
    return a.Wt && a.N_out % 64 == 0 && a.epi != EPI_ROWSCALE && a.group_size > 0 &&
           a.group_size % 32 == 0 && (a.group_size & (a.group_size - 1)) == 0 &&
           a.K % a.group_size == 0 && 256 * (a.K / a.group_size) <= kPpScaleMax;
  return a.fmt == SMOE_BF16 || (a.fmt == SMOE_FP8_E4M3 && a.Wt && a.N_out % 16 == 0 &&
                                a.epi != EPI_ROWSCALE);
}

bool gemm_takes_row_tiles(const GemmArgs& a) {
  if (a.W2 || !pp_weights(a) || a.out_dtype != SMOE_BF16 || a.epi == EPI_F32_BIAS) return false;
  if (a.K % 64 || a.ldw % 8 || a.lda % 8 || a.ldo % 32 || a.w_gstride % 8 || a.N_out % 256)
    return false;
  return (a.G == 0 ? a.single_rows : a.max_rows / a.G) >= 256;
}

int launch_grouped_gemm(const GemmArgs& a, hipStream_t s) {
  if (g_launch_ev[0] && g_clock_ctr && !a.clk) {  // a profiled launch: its clock too
    GemmArgs b = a;
    b.clk = g_clock_ctr;
    return launch_grouped_gemm(b, s);
  }
  if (a.N_out <= 0 || a.K <= 0) return SMOE_EINVAL;
  if (a.W2) return SMOE_EINVAL;  // two weight segments: launch_front_gemm
  // pointers every launched workgroup dereferences
  if (!(a.A || a.At) || !a.W || !a.out || (a.G > 0 && !a.grp_off)) return SMOE_EINVAL;
  // row-tile operands / outputs: only the ping-pong kernels below read them
  if ((a.At || a.out_tiles) && !gemm_takes_row_tiles(a)) return SMOE_EINVAL;
  if ((a.epi == EPI_ROWSCALE || a.epi == EPI_DOWN) && !a.row_scale) return SMOE_EINVAL;
  if ((a.fmt == SMOE_FP8_E4M3 || a.fmt == SMOE_INT4) && !a.S) return SMOE_EINVAL;
  // BN: the whole N range when it is small (router / edge logits: N_out = E),
  // otherwise 128 (64 for fp32); a partial last N tile is masked.
  if (a.fmt == SMOE_F32) {
    if (a.epi == EPI_SWIGLU) return SMOE_EUNSUPPORTED;
    return launch_simt<SMOE_F32>(a, s);
  }
  if (a.fmt == SMOE_INT4 && (a.group_size <= 0 || a.group_size % 8 || a.K % a.group_size))
    return SMOE_EINVAL;
  const int bk = (a.K % 64 == 0) ? 64 : (a.K % 32 == 0 ? 32 : 0);
  // bf16 shapes off the MFMA kernels' grid (K not a multiple of 32, or
  // operand rows / groups not 16-byte aligned): the SIMT kernel
  if (a.fmt == SMOE_BF16 && a.epi != EPI_SWIGLU &&
      (!bk || a.lda % 8 || a.ldw % 8 || a.w_gstride % 8))
    return launch_simt<SMOE_BF16>(a, s);
  if (!bk) return SMOE_EINVAL;
  if (a.epi == EPI_SWIGLU && a.N_out % 128) return SMOE_EINVAL;
  // decode: a few rows per group, weight streaming; also narrow outputs
  // (router / edge logits, N_out <= 64) of one group at any row count or of
  // groups of up to 256 rows, where the activations are the stream (grouped
  // ones with thousands of rows per group run faster as 64-row MFMA tiles)
  const int rpg_all = a.G == 0 ? a.single_rows : a.max_rows / a.G;
  if (skinny_fits(a) || (a.N_out <= 64 && a.epi != EPI_SWIGLU && (a.G == 0 || rpg_all <= 256) &&
                         skinny_aligned(a))) {
    const int rpg = a.G == 0 ? a.single_rows : a.max_rows / a.G;
    if (a.N_out >= 128 && skinny_fits(a)) return launch_decode(a, s);
    if (a.N_out <= 16) return rpg <= 16 ? launch_skinny<1, 1>(a, s) : launch_skinny<1, 2>(a, s);
    if (a.N_out <= 32 && a.epi != EPI_SWIGLU)
      return rpg <= 16 ? launch_skinny<2, 1>(a, s) : launch_skinny<2, 2>(a, s);
    // one group of many rows (router logits at E = 64): 16-row tiles double
    // the workgroups (C4: 11.8 us against 14.9 with 32-row tiles); grouped
    // rows (edge logits) keep 32-row tiles, which share each group's weights
    // between more rows; grouped outputs of up to 64 channels in two 32-channel
    // strips (C4 edge logits, 64 groups of ~68 rows: 20.4 -> 18.7 us, twice
    // the workgroups on a grid of 200 row tiles)
    if (a.G > 0 && a.epi != EPI_SWIGLU && a.N_out <= 64 && rpg > 8) return launch_skinny<2, 2>(a, s);
    return rpg <= 8 || a.G == 0 ? launch_skinny<4, 1>(a, s) : launch_skinny<4, 2>(a, s);
  }
  // a few dozen to 128 rows per group (mixed decode + prefill): one
  // workgroup per (group, 256-channel strip) over all the group's rows,
  // weights and activations streamed through an LDS ring
  {
    const int rpg = a.G == 0 ? a.single_rows : a.max_rows / a.G;
    if (a.G > 0 && rpg <= 128 && a.N_out >= 128 && stream_aligned(a) &&
        (a.fmt != SMOE_INT4 || (256 * (a.K / a.group_size) <= kStreamScaleMax &&
                                (a.group_size & (a.group_size - 1)) == 0)))
      return launch_stream(a, s);
  }
  // large bf16 / fp8 (tile copy) problems (K % 64): 256 x 256 tiles, 8 waves in two ping-pong
  // groups when N_out % 256 == 0 (128-row tiles, two workgroups per CU, for
  // groups of a few hundred rows); otherwise 256 x 128 ring tiles, two
  // workgroups per CU (a half-empty 256-wide last tile costs more than the
  // ring's weaker main loop).  A 384 x 128 single-workgroup tile for groups
  // of ~260 rows (each weight strip fetched once, dead 16-row tiles skipped)
  // measured 27% slower than the 128-row tiles at that shape.
  if (pp_weights(a) && a.out_dtype == SMOE_BF16 && a.epi != EPI_F32_BIAS && a.K % 64 == 0 &&
      a.ldw % 8 == 0 && a.lda % 8 == 0 && a.ldo % 8 == 0 &&
      (a.G == 0 ? a.single_rows : a.max_rows / (a.G > 0 ? a.G : 1)) >= 256) {
    const int rpg = a.G == 0 ? a.single_rows : a.max_rows / a.G;
    if (a.N_out % 256 == 0) {
      if (rpg > 256 && rpg <= 320) return launch_pp<4, 4, 320>(a, s);
      if (rpg < 512) return launch_pp<3, 4, 128>(a, s);
      // 320-row tiles where they save rounds, except for the edge projection
      // (EPI_ROWSCALE), whose worst-case row count overstates its groups
      return a.epi != EPI_ROWSCALE && pp_rows_320(a, rpg) ? launch_pp<4, 4, 320>(a, s)
                                                : launch_pp<4, 4, 256>(a, s);
    }
    if (a.N_out % 128 == 0 && a.fmt == SMOE_BF16) return launch_ring<128, 3, 4>(a, s);
  }
  const bool b64 = bk == 64;
  // narrow outputs (router / edge logits, N_out = E): 64-row tiles, one
  // 16-row MFMA strip per wave, so the grid has enough workgroups
  if (a.N_out <= 16)
    return b64 ? launch_mfma<64, 16, 64, 4, 1>(a, s) : launch_mfma<64, 16, 32, 4, 1>(a, s);
  if (a.N_out <= 32)
    return b64 ? launch_mfma<64, 32, 64, 4, 1>(a, s) : launch_mfma<64, 32, 32, 4, 1>(a, s);
  if (a.N_out <= 64)
    return b64 ? launch_mfma<64, 64, 64, 4, 1>(a, s) : launch_mfma<64, 64, 32, 4, 1>(a, s);
  return b64 ? launch_mfma<128, 128, 64, 2, 2>(a, s) : launch_mfma<128, 128, 32, 2, 2>(a, s);
}

int launch_decode_edge(const GemmArgs& a, const DecPlan& q, hipStream_t s) {
  const int E = a.G, N = a.sel_n, km = a.sel_km;
  if (!a.sel_idx || !a.sel_w || !a.A || !a.Wt || !a.out) return SMOE_EINVAL;
  if (a.fmt != SMOE_BF16 || a.epi != EPI_ROWSCALE || a.N_out < 128 || a.N_out % 16 ||
      a.K % 64 || !skinny_aligned(a) || km < 4 || km > 16 || km % 4 ||
      reinterpret_cast<uintptr_t>(a.sel_idx) % 16 || reinterpret_cast<uintptr_t>(a.sel_w) % 16 ||
      N < 1 || N > kFrontMaxN || E < 1 || E > 64 || q.K > 4 || q.N != N || q.E != E ||
      q.K * q.M != km || !decode_plan_fits(q))
    return SMOE_EUNSUPPORTED;
  // row tiles and K split as launch_decode picks them for the same groups
  // through the destination plan, so both give the same bits
  const int rows = N * q.S;
  const int rpg = rows / E;
  if (rpg > 32) return SMOE_EUNSUPPORTED;  // launch_grouped_gemm's decode range
  const int rt = rpg <= 8 ? 1 : 2;
  const int steps = a.K / 64;
  const int tiles = max(min(E, rows), (rows + 16 * rt - 1) / (16 * rt));
  const long long strips = (long long)((a.N_out + 63) / 64) * tiles;
  const int cus = device_cus();
  const long long want = 8LL * (cus > 0 ? cus : 256);
  int ksplit = 1;
  while (ksplit < 4 && strips * ksplit < want && steps / (2 * ksplit) >= 3) ksplit *= 2;
  GemmArgs b = a;
  b.sel_tpg = (N + 16 * rt - 1) / (16 * rt);
  const int slices = (a.N_out + 63) / 64, cs = 4 / ksplit;
  const dim3 grid((slices + cs - 1) / cs, 1 + E * b.sel_tpg, 1);  // the plans' row, then the tiles
  auto go = [&](auto rtc, auto ksc) {
    SMOE_LAUNCH((k_decode_edge<decltype(rtc)::value, decltype(ksc)::value>), grid, dim3(256), 0, s,
                b, q);
    return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
  };
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I4 = std::integral_constant<int, 4>;
  if (rt == 1) return ksplit == 1 ? go(I1{}, I1{}) : ksplit == 2 ? go(I1{}, I2{}) : go(I1{}, I4{});
  return ksplit == 1 ? go(I2{}, I1{}) : ksplit == 2 ? go(I2{}, I2{}) : go(I2{}, I4{});
}

}  // namespace smoe
