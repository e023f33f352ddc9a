// Prefill logits of the Spider-MoE block in one pass over the hidden states.
//
// The router logits (spider_moe/model.py:255-256: h W_r^T + the loop's
// router bias) and, when the expert count is small, the edge generator
// logits of every source expert (model.py:261-268: [h, loop embedding]
// W_g^T + b_g, the embedding's part folded into the per-loop edge bias) come
// out of one GEMM over [W_r; W_g], so the edge logits need neither the
// expert plan (to group the selected (token, source) rows) nor a second read
// of h.  At E = 16 that is 16 + 256 output channels per token: a GEMM far
// too narrow for the ping-pong tiles and too wide for the skinny kernel,
// with its own shape here.
#include "smoe_common.hpp"
#include "smoe_internal.hpp"
#include "smoe_routing.hpp"

namespace smoe {
namespace {

constexpr int kFlRows = 64;   // rows (tokens) per workgroup
constexpr int kFlStages = 6;  // activation ring: 64 rows x 64 k (8 KB) per stage
constexpr int kFlMaxTpw = 5;  // 16-channel tiles per wave: N_out <= 320
// Weight stages in flight per wave (register ring) and the activation DMA's
// cache policy.  C1's prefill front (rocprof, same box): 38.9 us per launch
// with 2 stages and the default policy, 40.0 with 3 stages and non-temporal
// activations, 39.9 / 39.7 with either alone.
constexpr int kFlAhead = 2;
constexpr int kFlAPolicy = 0;
constexpr int kFpWaves = 8;  // waves of the prefill front's workgroup (two per SIMD)

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

// A workgroup owns 64 consecutive rows and every output channel; wave w
// takes the 16-channel tiles w, w + 4, .. (TPW of them; a wave past the last
// tile repeats its previous one, whose loads then hit in cache, and stores
// nothing for it).  Output channel c < n_split reads W row c (ldw apart) and
// adds bias[c]; c >= n_split reads W2 row c - n_split (ldw2) and adds
// bias2[c - n_split].
//   activations: 64 rows x 64 k per stage, global -> LDS by DMA into a
//                kFlStages ring (128-byte rows, sw_chunk<8> swizzle),
//                kFlStages - 1 stages ahead
//   weights:     global -> registers, each lane the two 16-byte pieces of
//                its channel row at k 8q.. and 32 + 8q.. of a 64-k stage
//                (the MFMA operand layout), kFlAhead stages ahead; the weights
//                (at most 320 rows) stay in the L2 that every workgroup
//                reads them from
//   MFMAs:       per stage and tile, two v_mfma_f32_16x16x32_bf16 per
//                16-row tile (k 0-31 and 32-63)
// Per stage the wave issues A(s + 5) and then W(s + D); the wait for stage
// s counts the loads issued after W(s) (those of D - 1 stages: 2 DMAs and
// 2 TPW weight loads each), and W(s) was issued after A(s), so one vmcnt
// wait covers both.  One barrier per stage.
template <int TPW, int NW = 4, int D = kFlAhead>
__device__ __forceinline__ void logits_mainloop(const GemmArgs& p, uint8_t* ring,
                                                f32x4 (&acc)[TPW][4]) {
  constexpr int NS = kFlStages, STAGE = kFlRows * 128, PA = NS - 1;
  constexpr int ALD = 8 / NW;  // activation DMAs per wave per stage (8 x 1 KB)
  constexpr int WAITN = (D - 1) * (ALD + 2 * TPW);
  static_assert(NW == 4 || NW == 8, "4 or 8 waves");
  static_assert(PA >= D && WAITN < 64, "A(s) goes out before W(s); vmcnt range");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int q = lane >> 4, l16 = lane & 15;
  const int N = p.single_rows, m0 = blockIdx.x * kFlRows;
  const int NT = (p.N_out + 15) >> 4;
  const int KS = p.K >> 6;
  const int nsplit = p.W2 ? p.n_split : p.N_out;
  const uint16_t* W = reinterpret_cast<const uint16_t*>(p.W);
  const uint16_t* W2 = reinterpret_cast<const uint16_t*>(p.W2);
  const uint16_t* wrow[TPW];
  {
    int prev = NT - 1;
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const int tl = wave + NW * t < NT ? wave + NW * t : prev;
      prev = tl;
      const int c = min(16 * tl + l16, p.N_out - 1);
      wrow[t] = c < nsplit ? W + static_cast<int64_t>(c) * p.ldw
                           : W2 + static_cast<int64_t>(c - nsplit) * p.ldw2;
    }
  }
  const uint16_t* A = reinterpret_cast<const uint16_t*>(p.A);
  const uint16_t* asrc[ALD];
#pragma unroll
  for (int j = 0; j < ALD; ++j) {
    const int r = 8 * (NW * j + wave) + (lane >> 3);
    const int row = min(m0 + r, N - 1);  // rows past N: a valid row, never stored
    asrc[j] = A + static_cast<int64_t>(row) * p.lda + (sw_chunk<8>(r, lane & 7) << 3);
  }
  auto issue_a = [&](int s) {  // stage s (past the end: the last again) into slot s % NS
    const int sc = min(s, KS - 1);
    uint8_t* base = ring + (s % NS) * STAGE;
#pragma unroll
    for (int j = 0; j < ALD; ++j)
      __builtin_amdgcn_global_load_lds((gbl_vptr)(asrc[j] + sc * 64),
                                       (lds_vptr)(base + (NW * j + wave) * 1024), 16, 0,
                                       kFlAPolicy);
  };
  u32x4 wa[D][TPW], wb[D][TPW];
  auto fetch_w = [&](int d, int s) {  // register slot d <- stage s (clamped)
    const int k0 = 64 * min(s, KS - 1);
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      wa[d][t] = *reinterpret_cast<const u32x4*>(wrow[t] + k0 + 8 * q);
      wb[d][t] = *reinterpret_cast<const u32x4*>(wrow[t] + k0 + 32 + 8 * q);
    }
  };
#pragma unroll
  for (int t = 0; t < TPW; ++t)
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) acc[t][rt] = f32x4{0.f, 0.f, 0.f, 0.f};
  // prologue, in the order the waits assume: A(0), W(0), .., A(D-1), W(D-1), A(D..PA-1)
#pragma unroll
  for (int s = 0; s < D; ++s) {
    issue_a(s);
    fetch_w(s, s);
  }
#pragma unroll
  for (int s = D; s < PA; ++s) issue_a(s);
  auto step = [&](int d, int s) {
    wait_vmcnt<WAITN>();  // A(s) and W(s) have landed (this wave's part)
    wait_lgkm0();         // and this wave's reads of stage s - 1 are done
    __builtin_amdgcn_s_barrier();
    issue_a(s + PA);  // into the slot of stage s - 1
    const uint8_t* sa = ring + (s % NS) * STAGE;
    bf16x8 alo[4], ahi[4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      const int r = 16 * rt + l16;
      alo[rt] = *reinterpret_cast<const bf16x8*>(sa + r * 128 + (sw_chunk<8>(r, q) << 4));
      ahi[rt] = *reinterpret_cast<const bf16x8*>(sa + r * 128 + (sw_chunk<8>(r, 4 + q) << 4));
    }
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        acc[t][rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8, wa[d][t]), alo[rt], acc[t][rt], 0, 0, 0);
        acc[t][rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8, wb[d][t]), ahi[rt], acc[t][rt], 0, 0, 0);
      }
    fetch_w(d, s + D);
  };
  int s0 = 0;
  for (; s0 + D <= KS; s0 += D)  // stage s in register slot s % D
#pragma unroll
    for (int d = 0; d < D; ++d) step(d, s0 + d);
#pragma unroll
  for (int d = 0; d + 1 < D; ++d)  // the last KS % D stages
    if (s0 + d < KS) step(d, s0 + d);
  wait_vmcnt<0>();  // the clamped refills past the end have landed before the workgroup ends
}

template <int TPW>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void k_front_logits(const GemmArgs p) {
  __shared__ __attribute__((aligned(1024))) uint8_t ring[kFlStages * kFlRows * 128];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = lane >> 4, l16 = lane & 15;
  const int N = p.single_rows, m0 = blockIdx.x * kFlRows;
  const int NT = (p.N_out + 15) >> 4;
  const int nsplit = p.W2 ? p.n_split : p.N_out;
  f32x4 acc[TPW][4];
  logits_mainloop<TPW>(p, ring, acc);
  // lane: channels 16 tile + 4 q + (0..3) of rows m0 + 16 rt + l16
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const int c = 16 * (wave + 4 * t) + 4 * q;
    if (wave + 4 * t >= NT || c >= p.N_out) continue;  // N_out % 4 == 0: c .. c + 3 all stored
    float bv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int n = c + i;
      const float* bp = n < nsplit ? p.bias : p.bias2;
      bv[i] = bp ? bp[n < nsplit ? n : n - nsplit] : 0.f;
    }
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      const int row = m0 + 16 * rt + l16;
      if (row >= N) continue;
      const f32x4 v = acc[t][rt];
      *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(p.out) + static_cast<int64_t>(row) * p.ldo + c) =
          f32x4{v[0] + bv[0], v[1] + bv[1], v[2] + bv[2], v[3] + bv[3]};
    }
  }
}

// The one-pass prefill front (E <= 16): a workgroup's 64 tokens are one
// chunk of the dispatch plans, so after its logits GEMM the workgroup also
// routes them and ranks them for both plans, with the logits in LDS.  Eight
// waves (two per SIMD, so one wave's barrier and LDS round trips overlap the
// other's MFMAs: C1 38.7 -> 35.3 us per launch against four waves):
//   1 the GEMM above over [router | every edge generator row]; the tile of
//     [64, E + E*E] logits (+ biases) goes to LDS (over the ring) and the
//     router logits also to `logits` (the statistics read them)
//   2 wave w routes tokens 8 w .. 8 w + 7, a segment of 16 lanes per token
//     (topk_seg, then topm_seg over the token's selected sources, ascending),
//     writing what k_route_topk / k_edge_topm write (edges in slot order,
//     rows t * K + j of slot_idx / slot_w) and copies of the tokens' sources
//     and destinations in LDS
//   3 wave 0 ranks the chunk for the expert plan, wave 1 for the destination
//     plan (rank_chunk over the LDS copies, all groups in one window),
//     writing the chunk's column of each plan's [G, C] count matrices and the
//     entries' ranks; launch_plan2_finish scans and scatters.
// The logits tile ends the GEMM's ring (its DMAs have landed, every wave is
// past its last read) and reuses its bytes.
template <int KB>
constexpr int fp_smem_bytes() {
  return (kFlRows * 272 * 4 > kFlStages * kFlRows * 128 ? kFlRows * 272 * 4
                                                        : kFlStages * kFlRows * 128) +
         kFlRows * 16 * 8 + kFlRows * KB * 8;
}

template <int TPW, int KB>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_front_prefill(
    const GemmArgs p, const FrontPrefill f) {
  constexpr int FT = kFlRows * 272 * 4 > kFlStages * kFlRows * 128 ? kFlRows * 272 * 4
                                                                  : kFlStages * kFlRows * 128;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[fp_smem_bytes<KB>()];
  float* ft = reinterpret_cast<float*>(smem);                  // [64, ldf] logits
  int32_t* s_d = reinterpret_cast<int32_t*>(smem + FT);        // [64, S <= 16] destinations
  float* s_dc = reinterpret_cast<float*>(s_d + kFlRows * 16);  // and coefficients
  int32_t* s_e = reinterpret_cast<int32_t*>(s_dc + kFlRows * 16);  // [64, K] sources
  float* s_ew = reinterpret_cast<float*>(s_e + kFlRows * KB);      // and weights
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = lane >> 4, l16 = lane & 15;
  const int N = f.N, E = f.E, K = f.K, ldf = p.N_out;
  const int chunk = blockIdx.x, t0 = chunk * kFlRows;
  const int NT = (p.N_out + 15) >> 4;
  f32x4 acc[TPW][4];
  logits_mainloop<TPW, kFpWaves>(p, smem, acc);
  wait_lgkm0();
  __syncthreads();  // every wave is past its last ring read
  // 1 the logits tile (+ biases) into LDS, the router's columns to memory
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const int c = 16 * (wave + kFpWaves * t) + 4 * q;
    if (wave + kFpWaves * t >= NT || c >= ldf) continue;  // ldf % 4 == 0
    float bv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int n = c + i;
      bv[i] = n < E ? p.bias[n] : p.bias2[n - E];
    }
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      const int r = 16 * rt + l16;
      const f32x4 v = acc[t][rt];
      const f32x4 o = f32x4{v[0] + bv[0], v[1] + bv[1], v[2] + bv[2], v[3] + bv[3]};
      *reinterpret_cast<f32x4*>(ft + r * ldf + c) = o;
      if (c < E && t0 + r < N)  // E % 4 == 0: the four columns are all router logits
        *reinterpret_cast<f32x4*>(f.logits + static_cast<int64_t>(t0 + r) * E + c) = o;
    }
  }
  __syncthreads();
  // 2 routing: 2 passes of 4 tokens per wave
  const int e = lane & 15, le = e < E ? e : E - 1;
#pragma unroll 1
  for (int ps = 0; ps < kFlRows / (4 * kFpWaves); ++ps) {
    const int tl = (kFlRows / kFpWaves) * wave + 4 * ps + (lane >> 4);
    const int t = t0 + tl;
    const bool ok = t < N;
    const float* row = ft + tl * ldf;
    const float v = row[le];
    const bool live = !f.active || f.active[ok ? t : N - 1] != 0;
    uint64_t m = topk_seg<16>(v, t, ok, live, E, K, f.top_idx, f.top_w, f.tok_e, f.tok_ew, s_e,
                              s_ew, tl);
    if (!live) m = 0;  // a token that has left: no sources (tok_e holds -1)
    float ev[KB];
    int rw[KB];
    bool lv[KB];
#pragma unroll
    for (int j = 0; j < KB; ++j) {  // the selected sources, ascending
      const int sj = m ? __builtin_ctzll(m) : 0;
      lv[j] = ok && j < K && m != 0;
      m &= m - 1;
      rw[j] = t * K + j;
      ev[j] = row[E + sj * E + le];
    }
    topm_seg<16, KB>(ev, rw, lv, t, ok, E, f.M, f.S, f.slot_idx, f.slot_w, f.tok_d, f.tok_dc, s_d,
                     s_dc, tl);
  }
  __syncthreads();
  // 3 the chunk's ranks: wave 0 the expert plan, wave 1 the destination plan
  if (wave == 0)
    rank_chunk(s_e, s_ew, N, K, E, 0, t0, 0, 64, f.e_ccnt + chunk, f.e_cacnt + chunk, f.C,
               f.e_tokrow, t0);
  else if (wave == 1)
    rank_chunk(s_d, s_dc, N, f.S, E, 1, t0, 0, 64, f.d_ccnt + chunk, f.d_cacnt + chunk, f.C,
               f.d_tokrow, t0);
}

int launch_front_logits(const GemmArgs& a, hipStream_t s) {
  if (a.fmt != SMOE_BF16 || a.epi != EPI_F32_BIAS || a.G != 0 || a.single_rows < 1 || !a.A ||
      !a.W || !a.out || a.N_out <= 0 || a.K < 64)
    return SMOE_EINVAL;
  if (a.K % 64 || a.N_out % 4 || a.ldo % 4 || a.ldo < a.N_out || a.lda % 8 || a.lda < a.K ||
      a.ldw % 8 || a.ldw < a.K)
    return SMOE_EINVAL;
  if (a.W2 && (a.n_split < 0 || a.n_split > a.N_out || a.n_split % 4 || a.ldw2 % 8 || a.ldw2 < a.K ||
               !aligned16(a.W2)))
    return SMOE_EINVAL;
  if (!aligned16(a.A) || !aligned16(a.W) || !aligned16(a.out)) return SMOE_EINVAL;
  const int nt = (a.N_out + 15) / 16, tpw = (nt + 3) / 4;
  if (tpw > kFlMaxTpw) return SMOE_EUNSUPPORTED;
  const dim3 grid(static_cast<unsigned>((a.single_rows + kFlRows - 1) / kFlRows)), block(256);
  switch (tpw) {
    case 1: SMOE_LAUNCH(k_front_logits<1>, grid, block, 0, s, a); break;
    case 2: SMOE_LAUNCH(k_front_logits<2>, grid, block, 0, s, a); break;
    case 3: SMOE_LAUNCH(k_front_logits<3>, grid, block, 0, s, a); break;
    case 4: SMOE_LAUNCH(k_front_logits<4>, grid, block, 0, s, a); break;
    default: SMOE_LAUNCH(k_front_logits<5>, grid, block, 0, s, a); break;
  }
  return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
}

int launch_front_prefill(const GemmArgs& a, const FrontPrefill& f, hipStream_t s) {
  if (a.fmt != SMOE_BF16 || a.epi != EPI_F32_BIAS || a.G != 0 || !a.A || !a.W || !a.W2 ||
      !a.bias || !a.bias2 || a.K < 64 || a.K % 64 || a.lda % 8 || a.lda < a.K || a.ldw % 8 ||
      a.ldw < a.K || a.ldw2 % 8 || a.ldw2 < a.K)
    return SMOE_EINVAL;
  if (f.E < 4 || f.E > 16 || f.E % 4 || a.N_out != f.E + f.E * f.E || a.n_split != f.E ||
      a.single_rows != f.N || f.N < 1 || f.K < 1 || f.K > f.E || f.M < 1 || f.M > f.E ||
      f.S < 1 || f.S > f.E || f.C != (f.N + kFlRows - 1) / kFlRows)
    return SMOE_EINVAL;
  if (!f.logits || !f.top_idx || !f.top_w || !f.tok_e || !f.tok_ew || !f.slot_idx || !f.slot_w ||
      !f.tok_d || !f.tok_dc || !f.e_tokrow || !f.d_tokrow || !f.e_ccnt || !f.e_cacnt ||
      !f.d_ccnt || !f.d_cacnt)
    return SMOE_EINVAL;
  if (!aligned16(a.A) || !aligned16(a.W) || !aligned16(a.W2) || !aligned16(f.logits))
    return SMOE_EINVAL;
  const int tpw = ((a.N_out + 15) / 16 + kFpWaves - 1) / kFpWaves;
  const dim3 grid(static_cast<unsigned>(f.C)), block(64 * kFpWaves);
#define SMOE_FP(T, KB) SMOE_LAUNCH((k_front_prefill<T, KB>), grid, block, 0, s, a, f)
#define SMOE_FP_K(T)                 \
  do {                               \
    if (f.K <= 2) SMOE_FP(T, 2);     \
    else if (f.K <= 4) SMOE_FP(T, 4); \
    else SMOE_FP(T, 16);             \
  } while (0)
  switch (tpw) {  // E 4, 8, 12, 16: 20, 72, 156, 272 channels over 8 waves
    case 1: SMOE_FP_K(1); break;
    case 2: SMOE_FP_K(2); break;
    default: SMOE_FP_K(3); break;
  }
#undef SMOE_FP_K
#undef SMOE_FP
  return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP;
}

}  // namespace smoe
