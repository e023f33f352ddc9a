// Host-side launcher interfaces shared by the .hip translation units.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "smoe.h"

namespace smoe {

// Start / stop events for the next GEMM launch (stage timing of the
// single-kernel stages): when set, the launch records them itself
// (hipExtLaunchKernelGGL), so the interval is the kernel's own execution,
// without the gaps two separate event packets would add; the launch clears
// them.  Diagnostics state of one host thread at a time, like the stage
// profiler that sets it.
extern thread_local hipEvent_t g_launch_ev[2];
// Device counters [2] that a profiled GEMM launch (g_launch_ev set) passes to
// its kernel as GemmArgs::clk (smoe_profile_clock); the calling thread's.
extern thread_local unsigned long long* g_clock_ctr;

#define SMOE_LAUNCH(kernel, grid, block, shm, stream, ...)                                   \
  do {                                                                                       \
    if (::smoe::g_launch_ev[0]) {                                                            \
      hipExtLaunchKernelGGL(kernel, grid, block, shm, stream, ::smoe::g_launch_ev[0],        \
                            ::smoe::g_launch_ev[1], 0, __VA_ARGS__);                         \
      ::smoe::g_launch_ev[0] = ::smoe::g_launch_ev[1] = nullptr;                             \
    } else {                                                                                 \
      hipLaunchKernelGGL(kernel, grid, block, shm, stream, __VA_ARGS__);                     \
    }                                                                                        \
  } while (0)

// Epilogues of the grouped GEMM  C[row, n] = sum_k A[a_row(row), k] * W_g[n, k]
enum Epi : int {
  EPI_F32_BIAS = 0,  // out f32 = acc*cs + col_bias[g*bias_gstride + n]           (logits)
  EPI_ROWSCALE = 1,  // out     = acc * row_scale[row]                            (edge projection)
  EPI_GELU = 2,      // out     = gelu_erf(acc*cs + bias[g*bias_gstride + n])      (expert up)
  EPI_SWIGLU = 3,    // out[u]  = silu(gate) * (up + bias[g*bias_gstride + u])     (expert gate/up)
  EPI_DOWN = 4,      // out     = (acc*cs + bias[g*bias_gstride + n]) * row_scale  (expert down)
};

struct GemmArgs {
  int fmt = SMOE_BF16;     // weight format; A is f32 for SMOE_F32, bf16 otherwise
  int epi = EPI_F32_BIAS;
  const void* A = nullptr;
  int lda = 0;                   // elements
  const int32_t* a_rows = nullptr;  // plan row -> A row; nullptr = identity
  const void* W = nullptr;
  const void* Wt = nullptr;      // bf16 / fp8: W in the weight tile layout (or nullptr);
                                 // int4: bf16 tiles of the dequantized W (large-tile GEMMs)
  int64_t w_gstride = 0;         // elements between groups
  int ldw = 0;                   // elements between rows of W
  const void* S = nullptr;       // fp8: f32 [G, N_out]; int4: [G, N_out, K/gs]
  int64_t s_gstride = 0;
  int s_f16 = 0;
  int group_size = 0;            // int4
  int K = 0, N_out = 0;
  const int32_t* grp_off = nullptr;  // [G+1]; G == 0 -> one group of single_rows rows
  int G = 0;
  int single_rows = 0;
  int max_rows = 0;              // worst-case total rows (grid sizing)
  // The row-tile layout over plan rows (that of the weight tiles: 16 rows x
  // 32 k = 1 KB of lane-ordered MFMA fragments, blocks of one 16-row band
  // consecutive in k; plan row p sits in band p / 16): At, when set, is A in
  // it (K columns; rows = plan rows, a_rows / lda unused), and out_tiles = 1
  // writes out in it (ldo columns).  Only the ping-pong kernels take these
  // (gemm_takes_row_tiles); their row tiles then start on 16-row bands.
  const void* At = nullptr;
  int out_tiles = 0;
  void* out = nullptr;
  int ldo = 0;
  int out_dtype = SMOE_F32;      // SMOE_F32 / SMOE_BF16
  const float* bias = nullptr;
  int64_t bias_gstride = 0;
  const float* row_scale = nullptr;
  // optional second weight segment (launch_front_gemm only): output channels
  // n >= n_split take row n - n_split of W2 (ldw2 elements apart) and bias2
  const void* W2 = nullptr;
  int ldw2 = 0;
  int n_split = 0;
  const float* bias2 = nullptr;
  // diagnostics: when set, the ping-pong kernel adds each workgroup's
  // shader-clock cycles (s_memtime) to clk[0] and its 100 MHz wall-clock
  // ticks (s_memrealtime) to clk[1], so clk[0] / clk[1] * 100 MHz is the
  // clock the launch ran at
  unsigned long long* clk = nullptr;
  // decode edge projection (launch_decode_edge): group g's rows are the
  // tokens t < sel_n whose destination coefficient c[t, g] (their selected
  // edges to g, sel_idx / sel_w [sel_n, sel_km], summed in order) is
  // nonzero, in token order; A row t, out row g * sel_n + t, row scale
  // c[t, g]; grp_off / a_rows / row_scale unused.  sel_tpg: row tiles per
  // group.
  const int32_t* sel_idx = nullptr;
  const float* sel_w = nullptr;
  int sel_km = 0, sel_n = 0, sel_tpg = 0;
};

int launch_grouped_gemm(const GemmArgs& a, hipStream_t s);
// true when launch_grouped_gemm runs `a` on a ping-pong kernel, which reads
// At and writes out_tiles (the fields themselves are ignored here)
bool gemm_takes_row_tiles(const GemmArgs& a);
// elements of a plan-row tile buffer of `rows` rows x `cols` columns
inline int64_t row_tile_elems(int64_t rows, int64_t cols) { return (rows + 15) / 16 * 16 * cols; }
// bf16 / fp8 w [G,N,K] -> the weight tile layout (smoe_pack_weight_tiles)
int launch_pack_weight_tiles(const void* w, int fmt, int G, int N, int K, void* out, hipStream_t s);
// int4 [G,N,K/2] + group scales -> bf16 tiles of the dequantized weights
int launch_pack_int4_qtiles(const void* q, int G, int N, int K, void* out, hipStream_t s);
// One bf16 GEMM over a few rows (G == 0, single_rows <= 64) with f32 logits
// out (EPI_F32_BIAS) from two weight segments: the router and all edge
// generator rows of a small decode step in one pass.
int launch_front_gemm(const GemmArgs& a, hipStream_t s);

// Prefill logits in one pass (k_front_logits): bf16 A [single_rows, K] (G ==
// 0) times W rows (channels < n_split, ldw) and W2 rows (the rest, ldw2; W2
// null: every channel from W) -> f32 out [rows, ldo] plus bias / bias2;
// N_out <= 320, n_split and N_out multiples of 4, K % 64 == 0.
// SMOE_EUNSUPPORTED past 320 output channels.
int launch_front_logits(const GemmArgs& a, hipStream_t s);

// ---- routing ----
int launch_route_topk(const float* logits, int N, int E, int K, int32_t* top_idx, float* top_w,
                      int32_t* tok_e, float* tok_ew, const int32_t* active, hipStream_t s);
int launch_merge_slots(const int32_t* idx, const float* w, int N, int K, int E, int drop_nonpos,
                       int32_t* tok_g, float* tok_w, hipStream_t s);
int launch_edge_topm(const float* edge_logit, const int32_t* tok_e, const int32_t* e_tokrow,
                     int N, int E, int K, int M, int S, int32_t* edge_idx, float* edge_w,
                     int32_t* tok_d, float* tok_dc, hipStream_t s);
// per-source top-m rows of the expert plan -> [N,K,M] in the caller's slot order
int launch_gather_topm(const int32_t* src_idx, const int32_t* tok_e, const int32_t* e_tokrow,
                       const int32_t* edge_idx, const float* edge_w, int N, int K, int M,
                       int32_t* out_idx, float* out_w, hipStream_t s);
// given edges [N,K,M] -> per-token destination coefficients (S per token)
int launch_dest_coeffs(const int32_t* src_idx, const int32_t* eidx, const float* ew, int N, int K,
                       int M, int E, int S, int32_t* tok_d, float* tok_dc, hipStream_t s);
size_t plan_scratch_bytes(int N, int G);
// One plan's operands for launch_plan2 (those of launch_plan), with an
// optional payload of pay_m values per entry moved from slot order to the
// plan rows by the scatter (first plan only).
struct PlanSpec {
  const int32_t* tok_g = nullptr;
  const float* tok_w = nullptr;
  int S = 0, G = 0, drop = 0;
  int32_t *cnt = nullptr, *acnt = nullptr, *off = nullptr, *rows = nullptr;
  float* roww = nullptr;
  int32_t* tokrow = nullptr;
  const int32_t* pay_idx = nullptr;
  const float* pay_w = nullptr;
  int32_t* out_idx = nullptr;
  float* out_w = nullptr;
  int pay_m = 0;
};
// The scan and scatter of two plans over the same N tokens whose chunk
// counts and ranks are in place (launch_front_prefill): one launch each.
// scratch: plan a's [G, C] count and positive-count matrices, then plan
// b's (plan_scratch_bytes(N, a.G) + plan_scratch_bytes(N, b.G)).
int launch_plan2_finish(const PlanSpec& a, const PlanSpec& b, int N, void* scratch, hipStream_t s);
// The prefill front's routing outputs (launch_front_prefill).
struct FrontPrefill {
  int N = 0, E = 0, K = 0, M = 0, S = 0, C = 0;  // C = ceil(N / 64) plan chunks
  float* logits = nullptr;
  int32_t* top_idx = nullptr;
  float* top_w = nullptr;
  int32_t* tok_e = nullptr;
  float* tok_ew = nullptr;
  int32_t* slot_idx = nullptr;  // per-source edges in slot order [N*K, M]
  float* slot_w = nullptr;
  int32_t* tok_d = nullptr;
  float* tok_dc = nullptr;
  int32_t* e_tokrow = nullptr;  // the entries' ranks within their chunk (plan scratch)
  int32_t* d_tokrow = nullptr;
  int32_t *e_ccnt = nullptr, *e_cacnt = nullptr, *d_ccnt = nullptr, *d_cacnt = nullptr;
  const int32_t* active = nullptr;
};
// Prefill steps at E <= 16 (E % 4 == 0): the logits GEMM over [router | every
// edge generator row] (a: A, W = router, W2 = edge generator rows, n_split
// = E, bias / bias2, N_out = E + E*E), then in the same workgroups top-k,
// per-source top-m, destination coefficients and both plans' chunk ranks.
int launch_front_prefill(const GemmArgs& a, const FrontPrefill& f, hipStream_t s);
int launch_plan(const int32_t* tok_g, const float* tok_w, int N, int S, int G, int drop_nonpos,
                int32_t* cnt, int32_t* acnt, int32_t* off, int32_t* rows, float* roww,
                int32_t* tokrow, void* scratch, hipStream_t s);
// Small N: router top-k, expert plan, edge top-m over the dense per-source
// edge logits and the destination plan in one workgroup.  front: f32
// [N, ldf] with router logits in columns [0, E) and the edge logits of
// source s in columns E + s E .. E + s E + E - 1.  Writes every output the
// separate stages write (logits and edge_logit too).
int launch_front_route(const float* front, int ldf, int N, int E, int K, int M, int S,
                       float* logits, int32_t* top_idx, float* top_w, int32_t* tok_e,
                       float* tok_ew, int32_t* e_cnt, int32_t* e_acnt, int32_t* e_off,
                       int32_t* e_rows, float* e_roww, int32_t* e_tokrow, float* edge_logit,
                       int32_t* edge_idx, float* edge_w, int32_t* tok_d, float* tok_dc,
                       int32_t* d_cnt, int32_t* d_acnt, int32_t* d_off, int32_t* d_rows,
                       float* d_roww, int32_t* d_tokrow, const int32_t* active,
                       hipStream_t s);
constexpr int kFrontMaxN = 64;

// ---- Forge surfaces (smoe_forge.hip) ----
// top-k of f32 logits [N, E] (E <= 64): mode 0 the router's softmax / top-k
// / renorm, mode 1 top-k on the logits then softmax over the k values
// fp8 x fp8 (smoe_fp8.hip): e4m3 quantization of x [rows, cols] into codes
// [rows, ld_out] (zero codes past cols) + the f32 scale (per tensor, with a
// workspace of quantize_fp8_workspace_bytes(), or per row); the GEMM over
// those codes.
size_t quantize_fp8_workspace_bytes();
int launch_quantize_fp8(const void* x, int xdt, int rows, int cols, int ld_out, int per_row,
                        uint8_t* codes, float* scale, void* workspace, hipStream_t s);
int launch_gemm_f8f8(const uint8_t* xq, int ldx, const float* xs, const uint8_t* wq, int ldw,
                     const float* ws, const float* bias, int N, int K, int N_out, int gelu,
                     void* out, int odt, int ldo, hipStream_t s);
int launch_select_topk(const float* logits, int N, int E, int K, int mode, float* top_w,
                       int32_t* top_idx, hipStream_t s);
// out[t] = sum over the token's rows tok_row [N, K] of y[row] * row_w[row]
int launch_combine_rows(const void* y, int ydt, const float* row_w, const int32_t* tok_row,
                        int N, int K, int H, void* out, int odt, hipStream_t s);
// out[i] = map[ids[i]] for ids in [0, E), else -1
int launch_remap_ids(const int32_t* ids, int64_t n, const int32_t* map, int E, int32_t* out,
                     hipStream_t s);

// ---- the reference's native loop (smoe_compat.hip), for the host entry
// points of smoe_host_abi.hip ----
// logits = h . router_w ([H, E], double sums), then the router on
// logits + bias_row (E <= 64)
int ref_logits_router(const float* h, const float* router_w, const float* bias_row, int B, int H,
                      int E, int K, float* w, int32_t* idx, hipStream_t s);
int ref_copy_f32(const float* src, float* dst, int64_t n, hipStream_t s);

// ---- decode loop (bf16, N <= 64): two launches in place of the front GEMM,
// the routing workgroup and the previous loop's epilogue ----
// k_decode_front: per (strip, 16-token tile); every strip computes the
// router logits and top-k of its tokens; strip 0 writes them, strip s + 1
// computes source s's E edge logits, and for each token that selected s its
// top-m and softmax weights, written at the source's rank among the token's
// sources (ascending).  With `y` set it first computes the tile's input rows
// as the previous loop's LayerNorm (h_{r-1}, its expert rows y and routing
// tok_e / tok_ew / e_tokrow, x0), and strip 0 writes them to h_out.
struct DecFront {
  const void* h = nullptr;  // the loop's input (no y) or the previous loop's input (y set)
  const void* x0 = nullptr;
  const void* y = nullptr;  // previous loop's expert rows (bf16), or null
  const int32_t* tok_e = nullptr;
  const float* tok_ew = nullptr;
  const int32_t* e_tokrow = nullptr;
  const float* ln_w = nullptr;
  const float* ln_b = nullptr;
  float alpha = 0.f, beta = 0.f, eps = 0.f;
  void* h_out = nullptr;  // y set: the LayerNorm rows (this loop's input)
  const void* router_w = nullptr;  // bf16 [E, H]
  const float* router_bias = nullptr;  // [E]
  const void* edge_w = nullptr;  // bf16 [E * E, ldw]
  int ldw = 0;
  const float* edge_bias = nullptr;  // [E * E]
  int N = 0, H = 0, E = 0, K = 0, M = 0;
  float* logits = nullptr;   // [N, E]
  int32_t* top_idx = nullptr;  // [N, K]
  float* top_w = nullptr;
  int32_t* sel_idx = nullptr;  // [N, K, M] top-m destinations of each selected source
  float* sel_w = nullptr;      // their softmax weights
  // the early-exit gate (ExitGate), or active null: tokens with active[t] ==
  // 0 take no part in the loop (with y set, their h passes through); with y
  // and exit_wb set, the previous loop's epilogue gate is taken here on the
  // LayerNorm rows (k_epilogue's operations), updating active and loops
  const float* exit_wb = nullptr;
  float threshold = 0.f;
  int32_t* active = nullptr;
  int32_t* loops = nullptr;
};
// shapes the decode loop takes (else the general stages run)
bool decode_front_fits(int N, int H, int E, int K, int M, int S, int ldw);
int launch_decode_front(const DecFront& a, hipStream_t s);
// The plans of a decode loop: the tokens' sources ascending (tok_e /
// tok_ew), the expert plan and each source row's edges at its plan row; the
// destination coefficients (tok_d / tok_dc) and the destination plan.
struct DecPlan {
  const int32_t* top_idx = nullptr;  // [N, K] and [N, K]: the router top-k
  const float* top_w = nullptr;
  const int32_t* sel_idx = nullptr;  // [N, K, M] and [N, K, M]: the sources' top-m
  const float* sel_w = nullptr;
  int N = 0, E = 0, K = 0, M = 0, S = 0;
  int32_t *tok_e = nullptr, *e_cnt = nullptr, *e_acnt = nullptr, *e_off = nullptr,
          *e_rows = nullptr, *e_tokrow = nullptr, *edge_idx = nullptr, *tok_d = nullptr,
          *d_cnt = nullptr, *d_acnt = nullptr, *d_off = nullptr, *d_rows = nullptr,
          *d_tokrow = nullptr;
  float *tok_ew = nullptr, *e_roww = nullptr, *edge_w = nullptr, *tok_dc = nullptr,
        *d_roww = nullptr;
  const int32_t* active = nullptr;  // the early-exit gate's: tokens with 0 take no part
};
bool decode_plan_fits(const DecPlan& q);
// k_decode_plan: the plans in one workgroup of their own
int launch_decode_plan(const DecPlan& q, hipStream_t s);
// The decode edge projection (bf16 weight tiles, EPI_ROWSCALE, the sel_*
// fields of `a` set) with the loop's plans in one more workgroup, which runs
// beside the weight streams: the projection reads only the front's
// selections.  SMOE_EUNSUPPORTED for shapes it does not take (the caller
// runs launch_decode_plan and the grouped GEMM instead).
int launch_decode_edge(const GemmArgs& a, const DecPlan& q, hipStream_t s);
int launch_edge_loop_bias(const void* wg, int act_dtype, const float* bg, const float* emb, int E,
                          int H, int L, int R, float* out, hipStream_t s);

// ---- combine ----
// Exit gate of the early-exit decode, fused into the epilogue: exit_wb f32
// [H + 1] (exit_head weight, then bias), active i32 [N] in/out (nonzero = in
// orbit), loops i32 [N] in/out or null (loops run per token).
struct ExitGate {
  const float* exit_wb;
  float threshold;
  int32_t* active;
  int32_t* loops;
};
// dense_n > 0: the projection rows of launch_decode_edge (token t's row of
// destination d at d * dense_n + t; d_tokrow unused)
int launch_msg_combine(const void* proj, int proj_dtype, const int32_t* tok_d,
                       const int32_t* d_tokrow, int N, int S, int H, void* msg, int msg_dtype,
                       hipStream_t s, int dense_n = 0);
int launch_epilogue(const void* h, const void* x0, int act_dtype, const void* y, int y_dtype,
                    const int32_t* tok_e, const float* tok_ew, const int32_t* e_tokrow, int N,
                    int K, int H, float alpha, float beta, const float* ln_w, const float* ln_b,
                    float eps, void* out, const ExitGate* gate, hipStream_t s);
int launch_delta_combine(const void* y, int y_dtype, const int32_t* tok_row, int N, int K, int H,
                         void* out, int out_dtype, hipStream_t s);

}  // namespace smoe
