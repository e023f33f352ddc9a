// C ABI of libsmoe.so (declared in include/smoe.h).
//
// smoe_block_forward enqueues, per loop, on the caller's stream:
//   1  logits GEMM        h . W_r^T + loop_bias[r]            (model.py:255)
//   2  route_topk         softmax / top-k / renorm            (model.py:256-258)
//   3  plan (experts)     stable (expert, token) order        (dispatch.py:56-115)
//   4  edge-logit GEMM    per source expert: W_g[s] h + bias  (model.py:261-264)
//   5  edge_topm          top-m, softmax, dest. coefficients  (model.py:265-288)
//   6  plan (dests)       stable (destination, token) order
//   7  edge GEMM          c * W_edge[d] h per (token, d)      (model.py:271-272)
//   8  msg combine        sum over the token's destinations   (model.py:288)
//   9  up GEMM            act(W_up msg + b_up)                (sparse_experts.py:60-61)
//   10 down GEMM          w * (W_down act + b_down)           (sparse_experts.py:62-63)
//   11 epilogue           LN(h + a*sum_e y + b*x0)            (model.py:317)
// No step reads routing back to the host; grids are sized for the worst case.
#include <mutex>
#include <string>
#include <type_traits>
#include <vector>

#include "smoe_common.hpp"
#include "smoe_internal.hpp"

using namespace smoe;

namespace {

thread_local std::string g_err;

int fail(int rc, const char* what) {
  g_err = what;
  return rc;
}

int hip_rc(int rc, const char* what) {
  if (rc == SMOE_EHIP) {
    g_err = std::string(what) + ": " + hipGetErrorString(hipGetLastError());
  } else if (rc != SMOE_OK) {
    g_err = std::string(what) + ": rc " + std::to_string(rc);
  }
  return rc;
}

// ---- stage profiling (diagnostics) ----
// Per calling thread: smoe_profile_stages arms the calls this thread makes
// afterwards, and two threads profiling their own calls do not see each
// other's events (the library keeps no other process-wide state).
thread_local uint32_t g_prof_mask = 0;
thread_local hipEvent_t* g_prof_ev = nullptr;
thread_local int g_prof_cap = 0;
thread_local int g_prof_n = 0;
thread_local std::vector<int32_t> g_prof_stage;

}  // namespace

namespace smoe {
thread_local hipEvent_t g_launch_ev[2] = {nullptr, nullptr};
thread_local unsigned long long* g_clock_ctr = nullptr;
}  // namespace smoe

namespace {

// Stages that are one GEMM launch: their events go with the launch itself
// (SMOE_LAUNCH), so the interval is the kernel's execution.  The others are
// bracketed by two recorded events.
bool one_gemm_stage(int stage) {
  return stage == SMOE_STAGE_ROUTER_GEMM || stage == SMOE_STAGE_EDGE_LOGITS ||
         stage == SMOE_STAGE_EDGE_GEMM || stage == SMOE_STAGE_UP_GEMM ||
         stage == SMOE_STAGE_DOWN_GEMM || stage == SMOE_STAGE_FRONT_GEMM;
}

struct StageScope {
  int i = -1;
  bool ext = false;
  hipStream_t s;
  StageScope(int stage, hipStream_t st) : s(st) {
    if (g_prof_ev && (g_prof_mask >> stage & 1u) && g_prof_n < g_prof_cap) {
      i = g_prof_n++;
      g_prof_stage[i] = stage;
      ext = one_gemm_stage(stage);
      if (ext) {
        g_launch_ev[0] = g_prof_ev[2 * i];
        g_launch_ev[1] = g_prof_ev[2 * i + 1];
      } else {
        (void)hipEventRecord(g_prof_ev[2 * i], s);
      }
    }
  }
  ~StageScope() {
    if (i < 0) return;
    if (!ext) {
      (void)hipEventRecord(g_prof_ev[2 * i + 1], s);
    } else if (g_launch_ev[0]) {  // nothing launched (no rows): an empty interval
      (void)hipEventRecord(g_prof_ev[2 * i], s);
      (void)hipEventRecord(g_prof_ev[2 * i + 1], s);
      g_launch_ev[0] = g_launch_ev[1] = nullptr;
    }
  }
};

#define SMOE_TRY(expr, what)            \
  do {                                  \
    const int _rc = (expr);             \
    if (_rc != SMOE_OK) return hip_rc(_rc, what); \
  } while (0)

// SMOE_TRY inside a profiling scope of stage `id`
#define STAGE(id, expr, what)           \
  do {                                  \
    StageScope _ps((id), s);            \
    SMOE_TRY(expr, what);               \
  } while (0)

size_t esize(int dtype) { return dtype == SMOE_F32 ? 4 : 2; }

size_t align_up(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

struct Bump {
  size_t off = 0;
  size_t take(size_t bytes) {
    const size_t o = off;
    off = align_up(off + bytes);
    return o;
  }
};

int ffn_dtype_of(const smoe_experts& ex) { return ex.format == SMOE_F32 ? SMOE_F32 : SMOE_BF16; }

int check_experts(const smoe_experts& ex, int H) {
  if (ex.E < 1 || ex.E > 256 || ex.H != H || H <= 0 || ex.U <= 0)
    return fail(SMOE_EINVAL, "expert shape (1 <= E <= 256)");
  if (!ex.w_up || !ex.w_down) return fail(SMOE_EINVAL, "expert weights missing");
  if (ex.w_gate) return fail(SMOE_EINVAL, "w_gate must be NULL (gate interleaved into w_up)");
  if (ex.act != SMOE_ACT_GELU && ex.act != SMOE_ACT_SWIGLU) return fail(SMOE_EINVAL, "act");
  switch (ex.format) {
    case SMOE_F32:
      if (ex.act == SMOE_ACT_SWIGLU) return fail(SMOE_EUNSUPPORTED, "SwiGLU with fp32 experts");
      break;
    case SMOE_BF16:
      break;
    case SMOE_FP8_E4M3:
      if (!ex.s_up || !ex.s_down) return fail(SMOE_EINVAL, "fp8 scales missing");
      break;
    case SMOE_INT4:
      if (!ex.s_up || !ex.s_down) return fail(SMOE_EINVAL, "int4 scales missing");
      if (ex.group_size <= 0 || ex.group_size % 8 || H % ex.group_size || ex.U % ex.group_size)
        return fail(SMOE_EINVAL, "int4 group size must divide H and U and be a multiple of 8");
      if (ex.scale_dtype != SMOE_F32 && ex.scale_dtype != SMOE_F16)
        return fail(SMOE_EUNSUPPORTED, "int4 scale dtype");
      break;
    default:
      return fail(SMOE_EUNSUPPORTED, "expert format");
  }
  // bf16 GELU experts take any H, U (the SIMT kernel for shapes off the
  // MFMA grid); SwiGLU pairs and the fp8 / int4 streams need the grid
  const bool any_shape = ex.format == SMOE_F32 || (ex.format == SMOE_BF16 && ex.act == SMOE_ACT_GELU);
  if (!any_shape) {
    if (H % 32 || ex.U % 32) return fail(SMOE_EINVAL, "fp8 / int4 / SwiGLU experts need H, U % 32 == 0");
    if (ex.act == SMOE_ACT_SWIGLU && ex.U % 64)
      return fail(SMOE_EINVAL, "SwiGLU needs U % 64 == 0");
  }
  return SMOE_OK;
}

// Experts, top-k and edges of a block or stage: E <= 256 (routing holds up to
// 4 experts per lane), K, M <= 16 (per-token slot buckets) and at most 64
// destinations per token, S = min(E, K * M) (one lane per entry in the
// message combine).
int check_ekm(int E, int K, int M) {
  if (E < 1 || E > 256) return fail(SMOE_EINVAL, "E must be in [1, 256]");
  if (K < 1 || K > E || K > 16) return fail(SMOE_EINVAL, "top_k must be in [1, min(E, 16)]");
  if (M < 1 || M > E || M > 16)
    return fail(SMOE_EINVAL, "edges_per_expert must be in [1, min(E, 16)]");
  if ((E < K * M ? E : K * M) > 64)
    return fail(SMOE_EINVAL, "min(E, top_k * edges_per_expert) must be <= 64");
  return SMOE_OK;
}

int check_block(const smoe_block* b) {
  if (!b) return fail(SMOE_EINVAL, "null block");
  if (b->act_dtype != SMOE_F32 && b->act_dtype != SMOE_BF16)
    return fail(SMOE_EUNSUPPORTED, "act_dtype");
  // H % 8: the row kernels' 8-wide vectors; GEMMs off the MFMA grid take
  // the SIMT kernel
  if (b->H <= 0 || b->H % 8 || b->H > 4096) return fail(SMOE_EINVAL, "H (H % 8 == 0, <= 4096)");
  const int rc = check_ekm(b->E, b->K, b->M);
  if (rc != SMOE_OK) return rc;
  if (b->L < 0 || b->R < 1) return fail(SMOE_EINVAL, "loops");
  if (!b->router_w || !b->loop_bias || !b->edge_gen_w || !b->edge_loop_bias || !b->edge_value_w)
    return fail(SMOE_EINVAL, "block weights missing");
  if (b->experts.E != b->E) return fail(SMOE_EINVAL, "experts.E != E");
  if (b->experts.format == SMOE_F32 && b->act_dtype != SMOE_F32)
    return fail(SMOE_EUNSUPPORTED, "fp32 experts need fp32 activations");
  return check_experts(b->experts, b->H);
}

// Small bf16 steps take the fused front: one GEMM for the router logits and
// the edge logits of every source (the E x E edge generator rows, so no
// source grouping is needed), then one workgroup for top-k, both plans and
// top-m.  Shapes follow the skinny GEMM's alignment rules.
bool front_ok(const smoe_block* b, int N) {
  const int E = b->E, S = (E < b->K * b->M) ? E : b->K * b->M;
  return b->act_dtype == SMOE_BF16 && N >= 1 && N <= kFrontMaxN && E <= 64 && b->K <= 16 &&
         b->M <= 16 && S <= 64 && b->H % 64 == 0 && (E + E * E) % 4 == 0 && E % 4 == 0 && (b->H + b->L) % 8 == 0;
}

// Prefill steps whose router and edge logits come out of one pass
// (launch_front_prefill: [router | every edge generator row], at most 272
// channels, E <= 16), routed and ranked in the same workgroups, where the
// separate stages would run the plans' three-kernel form (C * E > 512).  The
// per-source edges wait in the edge_logit region in slot order (2 M <= E:
// they fit) until the expert plan's scatter moves them.
bool prefill_front_ok(const smoe_block* b, int N) {
  const int E = b->E, S = (E < b->K * b->M) ? E : b->K * b->M;
  const int64_t C = (static_cast<int64_t>(N) + 63) / 64;
  return b->act_dtype == SMOE_BF16 && N > kFrontMaxN && C * E > 512 && E % 4 == 0 && E <= 16 &&
         b->K <= 16 && b->M <= 16 && 2 * b->M <= E && S <= 64 && b->H % 64 == 0 &&
         (b->H + b->L) % 8 == 0;
}

// Router logits (G == 0, f32 out): bf16 batches of >= 64 row tiles on the
// one-pass logits kernel (a workgroup per 64 rows and every channel, h read
// once: C3's 16384 x 1024 -> 32 logits 24 -> ~8 us), the rest on the
// grouped GEMM.
int launch_router_logits(const GemmArgs& rg, hipStream_t s) {
  auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (rg.fmt == SMOE_BF16 && rg.G == 0 && rg.single_rows >= 64 * 64 && rg.K % 64 == 0 &&
      rg.N_out % 4 == 0 && rg.ldo % 4 == 0 && rg.lda % 8 == 0 && rg.ldw % 8 == 0 && !rg.W2 &&
      a16(rg.A) && a16(rg.W) && a16(rg.out)) {
    const int rc = launch_front_logits(rg, s);
    if (rc != SMOE_EUNSUPPORTED) return rc;
  }
  return launch_grouped_gemm(rg, s);
}

// bf16 decode steps the fused decode loop takes (k_decode_front and the
// plans beside the edge projection, in place of the front GEMM, the routing
// workgroup and the previous loop's epilogue, whose early-exit gate the
// next front takes).
bool decode_ok(const smoe_block* b, int N) {
  const int E = b->E, S = (E < b->K * b->M) ? E : b->K * b->M;
  return b->act_dtype == SMOE_BF16 && b->experts.format != SMOE_F32 &&
         decode_front_fits(N, b->H, E, b->K, b->M, S, b->H + b->L);
}

void make_layout(const smoe_block* b, int N, smoe_ws_layout* l) {
  const size_t n = N > 0 ? static_cast<size_t>(N) : 1;
  const int E = b->E, K = b->K, M = b->M, H = b->H;
  const int S = E < K * M ? E : K * M;
  const int fdt = ffn_dtype_of(b->experts);
  const int U = b->experts.U;
  Bump z;
  l->logits = z.take(n * E * 4);
  l->top_idx = z.take(n * K * 4);
  l->top_w = z.take(n * K * 4);
  l->tok_e = z.take(n * K * 4);
  l->tok_ew = z.take(n * K * 4);
  l->e_cnt = z.take(E * 4);
  l->e_acnt = z.take(E * 4);
  l->e_off = z.take((E + 1) * 4);
  l->e_rows = z.take(n * K * 4);
  l->e_roww = z.take(n * K * 4);
  l->e_tokrow = z.take(n * K * 4);
  l->edge_logit = z.take(n * K * E * 4);
  l->edge_idx = z.take(n * K * M * 4);
  l->edge_w = z.take(n * K * M * 4);
  l->tok_d = z.take(n * S * 4);
  l->tok_dc = z.take(n * S * 4);
  l->d_cnt = z.take(E * 4);
  l->d_acnt = z.take(E * 4);
  l->d_off = z.take((E + 1) * 4);
  l->d_rows = z.take(n * S * 4);
  l->d_roww = z.take(n * S * 4);
  l->d_tokrow = z.take(n * S * 4);
  // decode loops: the edge projection's rows at d * N + t (launch_decode_edge)
  l->proj = z.take(n * (decode_ok(b, N) ? E : S) * H * esize(b->act_dtype));
  l->msg = z.take(n * H * esize(fdt));
  // act: plan rows, row-major or in the row-tile layout (run_experts)
  l->act = z.take(row_tile_elems(n * K, U) * esize(fdt));
  l->y = z.take(n * K * H * esize(fdt));
  l->h_tmp = z.take(n * H * esize(b->act_dtype));
  const bool pf = prefill_front_ok(b, N);
  l->scratch = z.take(plan_scratch_bytes(N, E) * (pf ? 2 : 1));  // the prefill front: both plans'
  l->front = z.take(front_ok(b, N) ? n * (E + E * E) * 4 : 0);
  const bool dec = decode_ok(b, N);
  l->sel_idx = z.take(dec ? n * K * M * 4 : 0);
  l->sel_w = z.take(dec ? n * K * M * 4 : 0);
  l->h_tmp2 = z.take(dec ? n * H * esize(b->act_dtype) : 0);
  l->total = z.off;
  l->S = S;
  l->ffn_dtype = fdt;
}

template <typename T>
T* at(void* ws, size_t off) {
  return reinterpret_cast<T*>(reinterpret_cast<char*>(ws) + off);
}

// The expert up / down GEMMs' arguments over a plan of max_rows rows
// (msg rows gathered through `rows`, act and y in plan order).
void expert_gemms(const smoe_experts& ex, const void* msg, const int32_t* off, const int32_t* rows,
                  const float* roww, int max_rows, void* act, void* y, GemmArgs& up, GemmArgs& dn) {
  const int H = ex.H, U = ex.U, E = ex.E;
  const int fdt = ffn_dtype_of(ex);
  const int nup = ex.act == SMOE_ACT_SWIGLU ? 2 * U : U;
  up.fmt = ex.format;
  up.epi = ex.act == SMOE_ACT_SWIGLU ? EPI_SWIGLU : EPI_GELU;
  up.A = msg;
  up.lda = H;
  up.a_rows = rows;
  up.W = ex.w_up;
  up.Wt = ex.w_up_tiles;  // int4: its int4 tile copy (smoe_pack_int4_qtiles)
  up.w_gstride = static_cast<int64_t>(nup) * H;
  up.ldw = H;
  up.S = ex.s_up;
  up.s_f16 = ex.scale_dtype == SMOE_F16;
  up.group_size = ex.group_size;
  up.s_gstride = ex.format == SMOE_INT4 ? static_cast<int64_t>(nup) * (H / ex.group_size) : nup;
  up.K = H;
  up.N_out = nup;
  up.grp_off = off;
  up.G = E;
  up.max_rows = max_rows;
  up.out = act;
  up.ldo = U;
  up.out_dtype = fdt;
  up.bias = ex.b_up;
  up.bias_gstride = U;
  dn.fmt = ex.format;
  dn.epi = EPI_DOWN;
  dn.A = act;
  dn.lda = U;
  dn.a_rows = nullptr;  // act rows are already in plan order
  dn.W = ex.w_down;
  dn.Wt = ex.w_down_tiles;
  dn.w_gstride = static_cast<int64_t>(H) * U;
  dn.ldw = U;
  dn.S = ex.s_down;
  dn.s_f16 = ex.scale_dtype == SMOE_F16;
  dn.group_size = ex.group_size;
  dn.s_gstride = ex.format == SMOE_INT4 ? static_cast<int64_t>(H) * (U / ex.group_size) : H;
  dn.K = U;
  dn.N_out = H;
  dn.grp_off = off;
  dn.G = E;
  dn.max_rows = max_rows;
  dn.out = y;
  dn.ldo = H;
  dn.out_dtype = fdt;
  dn.bias = ex.b_down;
  dn.bias_gstride = H;
  dn.row_scale = roww;
}

// Expert up + down GEMMs over a plan.  When both run on the ping-pong
// kernels, act goes between them in the row-tile layout: the down GEMM's A
// operand DMA then reads contiguous 1 KB blocks, not 64-byte pieces of 16
// rows (C1 down GEMM 1.031 -> 0.941 ms per step).  The messages stay
// row-major: a row-tile copy of them (one per plan row, written by the
// message combine) made the up GEMM 3.5% faster but its scattered 16-byte
// writes cost the combine 0.3 ms per C1 step.
int run_experts(const smoe_experts& ex, const void* msg, const int32_t* off, const int32_t* rows,
                const float* roww, int max_rows, void* act, void* y, hipStream_t s) {
  GemmArgs up, dn;
  expert_gemms(ex, msg, off, rows, roww, max_rows, act, y, up, dn);
  if (gemm_takes_row_tiles(up) && gemm_takes_row_tiles(dn)) {
    up.out_tiles = 1;
    dn.At = act;
    dn.A = nullptr;
  }
  STAGE(SMOE_STAGE_UP_GEMM, launch_grouped_gemm(up, s), "expert up GEMM");
  STAGE(SMOE_STAGE_DOWN_GEMM, launch_grouped_gemm(dn, s), "expert down GEMM");
  return SMOE_OK;
}

}  // namespace

extern "C" {

SMOE_API int smoe_abi_version(void) { return SMOE_ABI_VERSION; }
SMOE_API const char* smoe_backend_name(void) { return "hip-gfx950"; }
SMOE_API uint32_t smoe_backend_caps(void) {
  return (1u << SMOE_F32) | (1u << SMOE_BF16) | (1u << SMOE_FP8_E4M3) | (1u << SMOE_INT4);
}
SMOE_API const char* smoe_last_error(void) { return g_err.c_str(); }

SMOE_API size_t smoe_block_workspace_bytes(const smoe_block* blk, int N) {
  if (check_block(blk) != SMOE_OK || N < 0) return 0;
  smoe_ws_layout l;
  make_layout(blk, N, &l);
  return l.total;
}

SMOE_API int smoe_block_workspace_layout(const smoe_block* blk, int N, smoe_ws_layout* out) {
  const int rc = check_block(blk);
  if (rc != SMOE_OK) return rc;
  if (!out || N < 0) return fail(SMOE_EINVAL, "layout args");
  make_layout(blk, N, out);
  return SMOE_OK;
}

SMOE_API int smoe_edge_loop_bias(const void* edge_gen_w, int act_dtype, const float* edge_gen_b,
                                 const float* loop_emb, int E, int H, int L, int R, float* out,
                                 void* stream) {
  if (!edge_gen_w || !out || (L > 0 && !loop_emb) || E < 1 || H < 1 || L < 0 || R < 1)
    return fail(SMOE_EINVAL, "edge_loop_bias args");
  if (act_dtype != SMOE_F32 && act_dtype != SMOE_BF16) return fail(SMOE_EUNSUPPORTED, "dtype");
  SMOE_TRY(launch_edge_loop_bias(edge_gen_w, act_dtype, edge_gen_b, loop_emb, E, H, L, R, out,
                                 static_cast<hipStream_t>(stream)),
           "edge_loop_bias");
  return SMOE_OK;
}

namespace {
// Loops [loop_begin, loop_begin + num_loops) of the block; gate (or null)
// is the exit gate of the early-exit decode: routing skips tokens whose
// gate->active entry is 0 and the epilogue passes their h through.
int block_forward(const smoe_block* b, const void* h_in, const void* x0, void* h_out, int N,
                  int loop_begin, int num_loops, const ExitGate* gate, void* ws, size_t ws_bytes,
                  void* stream) {
  int rc = check_block(b);
  if (rc != SMOE_OK) return rc;
  if (N < 0 || loop_begin < 0 || num_loops < 0 || loop_begin + num_loops > b->R)
    return fail(SMOE_EINVAL, "N / loop range");
  if (N == 0) return SMOE_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (num_loops == 0) {  // no loop: h_out = h_in (the reference returns h unchanged)
    if (!h_in || !h_out) return fail(SMOE_EINVAL, "null buffer");
    if (h_out != h_in &&
        hipMemcpyAsync(h_out, h_in, static_cast<size_t>(N) * b->H * esize(b->act_dtype),
                       hipMemcpyDeviceToDevice, s) != hipSuccess)
      return fail(SMOE_EHIP, "hipMemcpyAsync");
    return SMOE_OK;
  }
  if (!h_in || !x0 || !h_out || !ws) return fail(SMOE_EINVAL, "null buffer");
  smoe_ws_layout l;
  make_layout(b, N, &l);
  if (ws_bytes < l.total) return fail(SMOE_ECAPACITY, "workspace too small");
  const int H = b->H, E = b->E, K = b->K, M = b->M, L = b->L, S = l.S;
  const int adt = b->act_dtype, fdt = l.ffn_dtype;
  const int gfmt = adt == SMOE_F32 ? SMOE_F32 : SMOE_BF16;  // router / edge weights

  const bool dec = decode_ok(b, N);
  const bool front = front_ok(b, N);
  const bool pfront = !dec && !front && prefill_front_ok(b, N);
  const int32_t* active = gate ? gate->active : nullptr;
  const void* cur = h_in;
  for (int i = 0; i < num_loops; ++i) {
    const int r = loop_begin + i;
    void* dst = ((num_loops - 1 - i) % 2 == 0) ? h_out : at<void>(ws, l.h_tmp);
    if (dec) {
      // the loop's input: h_in, or the previous loop's LayerNorm, computed by
      // this loop's front and kept in h_tmp / h_tmp2 (never the buffer the
      // previous input is read from)
      void* in_r = i == 0 ? const_cast<void*>(h_in) : at<void>(ws, (i % 2) ? l.h_tmp : l.h_tmp2);
      DecFront fa;
      fa.h = cur;
      fa.x0 = x0;
      if (i > 0) {
        fa.y = at<void>(ws, l.y);
        fa.tok_e = at<int32_t>(ws, l.tok_e);
        fa.tok_ew = at<float>(ws, l.tok_ew);
        fa.e_tokrow = at<int32_t>(ws, l.e_tokrow);
        fa.ln_w = b->ln_w;
        fa.ln_b = b->ln_b;
        fa.alpha = b->alpha;
        fa.beta = b->beta;
        fa.eps = b->eps;
        fa.h_out = in_r;
      }
      fa.router_w = b->router_w;
      fa.router_bias = b->loop_bias + static_cast<int64_t>(r) * E;
      fa.edge_w = b->edge_gen_w;
      fa.ldw = H + L;
      fa.edge_bias = b->edge_loop_bias + static_cast<int64_t>(r) * E * E;
      fa.N = N;
      fa.H = H;
      fa.E = E;
      fa.K = K;
      fa.M = M;
      fa.logits = at<float>(ws, l.logits);
      fa.top_idx = at<int32_t>(ws, l.top_idx);
      fa.top_w = at<float>(ws, l.top_w);
      fa.sel_idx = at<int32_t>(ws, l.sel_idx);
      fa.sel_w = at<float>(ws, l.sel_w);
      if (gate) {  // the previous loop's exit decision, in this loop's front
        fa.active = gate->active;
        fa.loops = gate->loops;
        fa.exit_wb = gate->exit_wb;
        fa.threshold = gate->threshold;
      }
      STAGE(SMOE_STAGE_FRONT_GEMM, launch_decode_front(fa, s), "decode front");
      cur = in_r;
      DecPlan dp;
      dp.top_idx = at<int32_t>(ws, l.top_idx);
      dp.top_w = at<float>(ws, l.top_w);
      dp.sel_idx = at<int32_t>(ws, l.sel_idx);
      dp.sel_w = at<float>(ws, l.sel_w);
      dp.N = N;
      dp.E = E;
      dp.K = K;
      dp.M = M;
      dp.S = S;
      dp.tok_e = at<int32_t>(ws, l.tok_e);
      dp.tok_ew = at<float>(ws, l.tok_ew);
      dp.e_cnt = at<int32_t>(ws, l.e_cnt);
      dp.e_acnt = at<int32_t>(ws, l.e_acnt);
      dp.e_off = at<int32_t>(ws, l.e_off);
      dp.e_rows = at<int32_t>(ws, l.e_rows);
      dp.e_roww = at<float>(ws, l.e_roww);
      dp.e_tokrow = at<int32_t>(ws, l.e_tokrow);
      dp.edge_idx = at<int32_t>(ws, l.edge_idx);
      dp.edge_w = at<float>(ws, l.edge_w);
      dp.tok_d = at<int32_t>(ws, l.tok_d);
      dp.tok_dc = at<float>(ws, l.tok_dc);
      dp.d_cnt = at<int32_t>(ws, l.d_cnt);
      dp.d_acnt = at<int32_t>(ws, l.d_acnt);
      dp.d_off = at<int32_t>(ws, l.d_off);
      dp.d_rows = at<int32_t>(ws, l.d_rows);
      dp.d_roww = at<float>(ws, l.d_roww);
      dp.d_tokrow = at<int32_t>(ws, l.d_tokrow);
      dp.active = active;
      // the edge projection with the plans beside it (one launch), where
      // its kernel takes the shape
      GemmArgs pg;
      pg.fmt = SMOE_BF16;
      pg.epi = EPI_ROWSCALE;
      pg.A = cur;
      pg.lda = H;
      pg.W = b->edge_value_w;
      pg.Wt = b->edge_value_w_tiles;
      pg.w_gstride = static_cast<int64_t>(H) * H;
      pg.ldw = H;
      pg.K = H;
      pg.N_out = H;
      pg.G = E;
      pg.max_rows = N * S;
      pg.out = at<void>(ws, l.proj);
      pg.ldo = H;
      pg.out_dtype = adt;
      pg.sel_idx = dp.sel_idx;
      pg.sel_w = dp.sel_w;
      pg.sel_km = K * M;
      pg.sel_n = N;
      int erc = SMOE_EUNSUPPORTED;
      if (b->edge_value_w_tiles) {
        STAGE(SMOE_STAGE_EDGE_GEMM, (erc = launch_decode_edge(pg, dp, s)) == SMOE_EUNSUPPORTED ? SMOE_OK : erc,
              "decode edge projection");
      }
      if (erc == SMOE_OK) {
        STAGE(SMOE_STAGE_MSG_COMBINE,
              launch_msg_combine(at<void>(ws, l.proj), adt, at<int32_t>(ws, l.tok_d),
                                 at<int32_t>(ws, l.d_tokrow), N, S, H, at<void>(ws, l.msg), fdt, s,
                                 N),
              "msg combine");
        rc = run_experts(b->experts, at<void>(ws, l.msg), at<int32_t>(ws, l.e_off),
                         at<int32_t>(ws, l.e_rows), at<float>(ws, l.e_roww), N * K,
                         at<void>(ws, l.act), at<void>(ws, l.y), s);
        if (rc != SMOE_OK) return rc;
        if (i + 1 < num_loops) continue;  // the epilogue: in the next loop's front
        STAGE(SMOE_STAGE_EPILOGUE,
              launch_epilogue(cur, x0, adt, at<void>(ws, l.y), fdt, at<int32_t>(ws, l.tok_e),
                              at<float>(ws, l.tok_ew), at<int32_t>(ws, l.e_tokrow), N, K, H,
                              b->alpha, b->beta, b->ln_w, b->ln_b, b->eps, h_out, gate, s),
              "epilogue");
        cur = h_out;
        continue;
      }
      STAGE(SMOE_STAGE_FRONT_ROUTE, launch_decode_plan(dp, s), "decode plans");
    } else if (front) {
      // 1-6 fused: [router | all edge generator rows] logits, then routing
      const int ldf = E + E * E;
      GemmArgs fg;
      fg.fmt = SMOE_BF16;
      fg.epi = EPI_F32_BIAS;
      fg.A = cur;
      fg.lda = H;
      fg.W = b->router_w;
      fg.ldw = H;
      fg.K = H;
      fg.N_out = ldf;
      fg.G = 0;
      fg.single_rows = N;
      fg.out = at<float>(ws, l.front);
      fg.ldo = ldf;
      fg.bias = b->loop_bias + static_cast<int64_t>(r) * E;
      fg.W2 = b->edge_gen_w;
      fg.ldw2 = H + L;
      fg.n_split = E;
      fg.bias2 = b->edge_loop_bias + static_cast<int64_t>(r) * E * E;
      STAGE(SMOE_STAGE_FRONT_GEMM, launch_front_gemm(fg, s), "front GEMM");
      STAGE(SMOE_STAGE_FRONT_ROUTE,
            launch_front_route(at<float>(ws, l.front), ldf, N, E, K, M, S, at<float>(ws, l.logits),
                               at<int32_t>(ws, l.top_idx), at<float>(ws, l.top_w),
                               at<int32_t>(ws, l.tok_e), at<float>(ws, l.tok_ew),
                               at<int32_t>(ws, l.e_cnt), at<int32_t>(ws, l.e_acnt),
                               at<int32_t>(ws, l.e_off), at<int32_t>(ws, l.e_rows),
                               at<float>(ws, l.e_roww), at<int32_t>(ws, l.e_tokrow),
                               at<float>(ws, l.edge_logit), at<int32_t>(ws, l.edge_idx),
                               at<float>(ws, l.edge_w), at<int32_t>(ws, l.tok_d),
                               at<float>(ws, l.tok_dc), at<int32_t>(ws, l.d_cnt),
                               at<int32_t>(ws, l.d_acnt), at<int32_t>(ws, l.d_off),
                               at<int32_t>(ws, l.d_rows), at<float>(ws, l.d_roww),
                               at<int32_t>(ws, l.d_tokrow), active, s),
            "front routing");
    } else if (pfront) {
      // 1-6 in one launch per 64-token chunk (logits of the router and every
      // edge generator row, top-k, per-source top-m, destination
      // coefficients, both plans' chunk ranks), then the plans' scan and
      // scatter, which also moves the per-source edges (slot order, in the
      // edge_logit region meanwhile) to their expert-plan rows
      GemmArgs fg;
      fg.fmt = SMOE_BF16;
      fg.epi = EPI_F32_BIAS;
      fg.A = cur;
      fg.lda = H;
      fg.W = b->router_w;
      fg.ldw = H;
      fg.K = H;
      fg.N_out = E + E * E;
      fg.G = 0;
      fg.single_rows = N;
      fg.bias = b->loop_bias + static_cast<int64_t>(r) * E;
      fg.W2 = b->edge_gen_w;
      fg.ldw2 = H + L;
      fg.n_split = E;
      fg.bias2 = b->edge_loop_bias + static_cast<int64_t>(r) * E * E;
      const int C = (N + 63) / 64;
      int32_t* ccnt = at<int32_t>(ws, l.scratch);  // expert plan [E, C] x 2, then destination
      FrontPrefill fp;
      fp.N = N;
      fp.E = E;
      fp.K = K;
      fp.M = M;
      fp.S = S;
      fp.C = C;
      fp.logits = at<float>(ws, l.logits);
      fp.top_idx = at<int32_t>(ws, l.top_idx);
      fp.top_w = at<float>(ws, l.top_w);
      fp.tok_e = at<int32_t>(ws, l.tok_e);
      fp.tok_ew = at<float>(ws, l.tok_ew);
      fp.slot_idx = at<int32_t>(ws, l.edge_logit);
      fp.slot_w = reinterpret_cast<float*>(fp.slot_idx + static_cast<int64_t>(N) * K * M);
      fp.tok_d = at<int32_t>(ws, l.tok_d);
      fp.tok_dc = at<float>(ws, l.tok_dc);
      fp.e_tokrow = at<int32_t>(ws, l.e_tokrow);
      fp.d_tokrow = at<int32_t>(ws, l.d_tokrow);
      fp.e_ccnt = ccnt;
      fp.e_cacnt = ccnt + static_cast<int64_t>(C) * E;
      fp.d_ccnt = ccnt + 2 * static_cast<int64_t>(C) * E;
      fp.d_cacnt = ccnt + 3 * static_cast<int64_t>(C) * E;
      fp.active = active;
      STAGE(SMOE_STAGE_FRONT_GEMM, launch_front_prefill(fg, fp, s), "prefill front");
      PlanSpec pe, pd;
      pe.tok_g = fp.tok_e;
      pe.tok_w = fp.tok_ew;
      pe.S = K;
      pe.G = E;
      pe.drop = 0;
      pe.cnt = at<int32_t>(ws, l.e_cnt);
      pe.acnt = at<int32_t>(ws, l.e_acnt);
      pe.off = at<int32_t>(ws, l.e_off);
      pe.rows = at<int32_t>(ws, l.e_rows);
      pe.roww = at<float>(ws, l.e_roww);
      pe.tokrow = fp.e_tokrow;
      pe.pay_idx = fp.slot_idx;
      pe.pay_w = fp.slot_w;
      pe.out_idx = at<int32_t>(ws, l.edge_idx);
      pe.out_w = at<float>(ws, l.edge_w);
      pe.pay_m = M;
      pd.tok_g = fp.tok_d;
      pd.tok_w = fp.tok_dc;
      pd.S = S;
      pd.G = E;
      pd.drop = 1;
      pd.cnt = at<int32_t>(ws, l.d_cnt);
      pd.acnt = at<int32_t>(ws, l.d_acnt);
      pd.off = at<int32_t>(ws, l.d_off);
      pd.rows = at<int32_t>(ws, l.d_rows);
      pd.roww = at<float>(ws, l.d_roww);
      pd.tokrow = fp.d_tokrow;
      STAGE(SMOE_STAGE_EXPERT_PLAN, launch_plan2_finish(pe, pd, N, ccnt, s),
            "expert + destination plans");
    } else {

    // 1 router logits (+ loop bias)
    GemmArgs rg;
    rg.fmt = gfmt;
    rg.epi = EPI_F32_BIAS;
    rg.A = cur;
    rg.lda = H;
    rg.W = b->router_w;
    rg.ldw = H;
    rg.K = H;
    rg.N_out = E;
    rg.G = 0;
    rg.single_rows = N;
    rg.out = at<float>(ws, l.logits);
    rg.ldo = E;
    rg.bias = b->loop_bias + static_cast<int64_t>(r) * E;
    rg.bias_gstride = 0;
    STAGE(SMOE_STAGE_ROUTER_GEMM, launch_router_logits(rg, s), "router logits");
    // 2 top-k
    STAGE(SMOE_STAGE_ROUTE_TOPK, launch_route_topk(at<float>(ws, l.logits), N, E, K, at<int32_t>(ws, l.top_idx),
                               at<float>(ws, l.top_w), at<int32_t>(ws, l.tok_e),
                               at<float>(ws, l.tok_ew), active, s),
             "route_topk");
    // 3 expert / source plan (keeps every selected source; the FFN combine
    //   skips weights <= 0)
    STAGE(SMOE_STAGE_EXPERT_PLAN, launch_plan(at<int32_t>(ws, l.tok_e), at<float>(ws, l.tok_ew), N, K, E, 0,
                         at<int32_t>(ws, l.e_cnt), at<int32_t>(ws, l.e_acnt),
                         at<int32_t>(ws, l.e_off), at<int32_t>(ws, l.e_rows),
                         at<float>(ws, l.e_roww), at<int32_t>(ws, l.e_tokrow),
                         at<void>(ws, l.scratch), s),
             "expert plan");
    // 4 edge logits of each (token, selected source) row
    GemmArgs eg;
    eg.fmt = gfmt;
    eg.epi = EPI_F32_BIAS;
    eg.A = cur;
    eg.lda = H;
    eg.a_rows = at<int32_t>(ws, l.e_rows);
    eg.W = b->edge_gen_w;
    eg.w_gstride = static_cast<int64_t>(E) * (H + L);
    eg.ldw = H + L;
    eg.K = H;
    eg.N_out = E;
    eg.grp_off = at<int32_t>(ws, l.e_off);
    eg.G = E;
    eg.max_rows = N * K;
    eg.out = at<float>(ws, l.edge_logit);
    eg.ldo = E;
    eg.bias = b->edge_loop_bias + static_cast<int64_t>(r) * E * E;
    eg.bias_gstride = E;
    STAGE(SMOE_STAGE_EDGE_LOGITS, launch_grouped_gemm(eg, s), "edge-logit GEMM");
    // 5 top-m + destination coefficients
    STAGE(SMOE_STAGE_EDGE_TOPM, launch_edge_topm(at<float>(ws, l.edge_logit), at<int32_t>(ws, l.tok_e),
                              at<int32_t>(ws, l.e_tokrow), N, E, K, M, S,
                              at<int32_t>(ws, l.edge_idx), at<float>(ws, l.edge_w),
                              at<int32_t>(ws, l.tok_d), at<float>(ws, l.tok_dc), s),
             "edge_topm");
    // 6 destination plan
    STAGE(SMOE_STAGE_DEST_PLAN, launch_plan(at<int32_t>(ws, l.tok_d), at<float>(ws, l.tok_dc), N, S, E, 1,
                         at<int32_t>(ws, l.d_cnt), at<int32_t>(ws, l.d_acnt),
                         at<int32_t>(ws, l.d_off), at<int32_t>(ws, l.d_rows),
                         at<float>(ws, l.d_roww), at<int32_t>(ws, l.d_tokrow),
                         at<void>(ws, l.scratch), s),
             "destination plan");
    }
    // 7 edge projections c * W_edge[d] h
    GemmArgs pg;
    pg.fmt = gfmt;
    pg.epi = EPI_ROWSCALE;
    pg.A = cur;
    pg.lda = H;
    pg.a_rows = at<int32_t>(ws, l.d_rows);
    pg.W = b->edge_value_w;
    pg.Wt = b->act_dtype == SMOE_BF16 ? b->edge_value_w_tiles : nullptr;
    pg.w_gstride = static_cast<int64_t>(H) * H;
    pg.ldw = H;
    pg.K = H;
    pg.N_out = H;
    pg.grp_off = at<int32_t>(ws, l.d_off);
    pg.G = E;
    pg.max_rows = N * S;
    pg.out = at<void>(ws, l.proj);
    pg.ldo = H;
    pg.out_dtype = adt;
    pg.row_scale = at<float>(ws, l.d_roww);
    STAGE(SMOE_STAGE_EDGE_GEMM, launch_grouped_gemm(pg, s), "edge GEMM");
    // 8 messages
    STAGE(SMOE_STAGE_MSG_COMBINE, launch_msg_combine(at<void>(ws, l.proj), adt, at<int32_t>(ws, l.tok_d),
                                at<int32_t>(ws, l.d_tokrow), N, S, H, at<void>(ws, l.msg), fdt, s),
             "msg combine");
    // 9, 10 experts
    rc = run_experts(b->experts, at<void>(ws, l.msg), at<int32_t>(ws, l.e_off),
                     at<int32_t>(ws, l.e_rows), at<float>(ws, l.e_roww), N * K,
                     at<void>(ws, l.act), at<void>(ws, l.y), s);
    if (rc != SMOE_OK) return rc;
    // 11 combine + residual + LayerNorm (the decode loop: in the next loop's
    // front, and after the last loop)
    if (dec && i + 1 < num_loops) continue;
    void* out_r = dec ? h_out : dst;
    STAGE(SMOE_STAGE_EPILOGUE, launch_epilogue(cur, x0, adt, at<void>(ws, l.y), fdt, at<int32_t>(ws, l.tok_e),
                             at<float>(ws, l.tok_ew), at<int32_t>(ws, l.e_tokrow), N, K, H,
                             b->alpha, b->beta, b->ln_w, b->ln_b, b->eps, out_r, gate, s),
             "epilogue");
    cur = out_r;
  }
  return SMOE_OK;
}
}  // namespace

SMOE_API int smoe_block_forward(const smoe_block* b, const void* h_in, const void* x0,
                                void* h_out, int N, int loop_begin, int num_loops, void* ws,
                                size_t ws_bytes, void* stream) {
  return block_forward(b, h_in, x0, h_out, N, loop_begin, num_loops, nullptr, ws, ws_bytes,
                       stream);
}

SMOE_API int smoe_block_forward_exit(const smoe_block* b, const void* h_in, const void* x0,
                                     void* h_out, int N, int loop_begin, int num_loops,
                                     const float* exit_wb, float threshold, int32_t* active,
                                     int32_t* loops, void* ws, size_t ws_bytes, void* stream) {
  if (!exit_wb || !active) return fail(SMOE_EINVAL, "exit gate buffers");
  // NaN test on the bits: fast-math builds fold a self-comparison away
  const uint32_t tb = __builtin_bit_cast(uint32_t, threshold);
  if ((tb & 0x7fffffffu) > 0x7f800000u) return fail(SMOE_EINVAL, "threshold is NaN");
  const ExitGate gate{exit_wb, threshold, active, loops};
  return block_forward(b, h_in, x0, h_out, N, loop_begin, num_loops, &gate, ws, ws_bytes, stream);
}

// ---- smoe_block_forward_scratch: the block workspace in a static device
// array instead of a caller's buffer ----
namespace {
// `scratch` is a host-side stand-in for the device array: host code never
// passes it (or takes its address) directly.  The device address is read
// once per device with hipGetSymbolAddress, with that device current, and
// every later use (the kernels' workspace argument) goes through it.
__device__ __align__(256) unsigned char scratch[SMOE_SCRATCH_BYTES];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;  // held from the overlap check to the last launch
void* g_scratch_ptr[kMaxDevices] = {};
// Per device: an event recorded after the last scratch call's launches, on
// its stream (made once, at the device's first call), and that stream.
hipEvent_t g_scratch_done[kMaxDevices] = {};
hipStream_t g_scratch_stream[kMaxDevices] = {};

// Device address of the current device's scratch array (the caller holds
// g_scratch_mu), and that device's id.
int scratch_address(hipStream_t s, void** out, int* dev_out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(SMOE_EHIP, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(SMOE_EINVAL, "device id beyond 64");
  if (s) {  // the stream must belong to the current device (its array is used)
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice(s, &sdev) != hipSuccess) return fail(SMOE_EHIP, "hipStreamGetDevice");
    if (sdev != dev) return fail(SMOE_EINVAL, "stream is not on the current device");
  }
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(SMOE_EHIP, (std::string("hipGetSymbolAddress(scratch): ") +
                              hipGetErrorString(e)).c_str());
    hipEvent_t ev = nullptr;
    if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess)
      return fail(SMOE_EHIP, "hipEventCreateWithFlags(scratch)");
    g_scratch_done[dev] = ev;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  *dev_out = dev;
  return SMOE_OK;
}
}  // namespace

SMOE_API int smoe_block_forward_scratch(const smoe_block* b, const void* h_in, const void* x0,
                                        void* h_out, int N, int loop_begin, int num_loops,
                                        void* stream) {
  const int rc = check_block(b);
  if (rc != SMOE_OK) return rc;
  if (N < 0) return fail(SMOE_EINVAL, "N");
  smoe_ws_layout l;
  make_layout(b, N, &l);
  if (l.total > static_cast<size_t>(SMOE_SCRATCH_BYTES))
    return fail(SMOE_ECAPACITY, ("workspace of " + std::to_string(l.total) +
                                 " bytes exceeds the static scratch of " +
                                 std::to_string(SMOE_SCRATCH_BYTES) + " bytes")
                                    .c_str());
  hipStream_t s = static_cast<hipStream_t>(stream);
  void* ws = nullptr;
  int dev = 0;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  const int arc = scratch_address(s, &ws, &dev);
  if (arc != SMOE_OK) return arc;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cap) != hipSuccess) return fail(SMOE_EHIP, "hipStreamIsCapturing");
  const bool captured = cap != hipStreamCaptureStatusNone;
  if (!captured && g_scratch_stream[dev] != s) {
    const hipError_t q = hipEventQuery(g_scratch_done[dev]);
    if (q == hipErrorNotReady)
      return fail(SMOE_EBUSY, "the previous smoe_block_forward_scratch call on this GPU is still "
                              "running on another stream");
    if (q != hipSuccess) return fail(SMOE_EHIP, "hipEventQuery(scratch)");
  }
  const int rc2 = block_forward(b, h_in, x0, h_out, N, loop_begin, num_loops, nullptr, ws,
                                SMOE_SCRATCH_BYTES, stream);
  if (rc2 != SMOE_OK || captured) return rc2;
  if (hipEventRecord(g_scratch_done[dev], s) != hipSuccess)
    return fail(SMOE_EHIP, "hipEventRecord(scratch)");
  g_scratch_stream[dev] = s;
  return SMOE_OK;
}

SMOE_API int smoe_pack_weight_tiles(const void* w, int format, int G, int N, int K, void* out,
                                    void* stream) {
  return hip_rc(launch_pack_weight_tiles(w, format, G, N, K, out, static_cast<hipStream_t>(stream)),
                "smoe_pack_weight_tiles");
}

SMOE_API int smoe_pack_int4_qtiles(const void* packed, int G, int N, int K, void* out,
                                   void* stream) {
  return hip_rc(launch_pack_int4_qtiles(packed, G, N, K, out, static_cast<hipStream_t>(stream)),
                "smoe_pack_int4_qtiles");
}

SMOE_API int smoe_profile_stages(uint32_t stage_mask, void** events, int capacity) {
  if (events && capacity < 0) return fail(SMOE_EINVAL, "capacity");
  g_prof_mask = stage_mask;
  g_prof_ev = reinterpret_cast<hipEvent_t*>(events);
  g_prof_cap = events ? capacity : 0;
  g_prof_n = 0;
  g_prof_stage.assign(static_cast<size_t>(g_prof_cap), 0);
  return SMOE_OK;
}

SMOE_API int smoe_profile_clock(void* counters) {
  g_clock_ctr = static_cast<unsigned long long*>(counters);
  return SMOE_OK;
}

SMOE_API int smoe_profile_count(int32_t* stage_of, int capacity) {
  const int n = g_prof_n;
  if (stage_of)
    for (int i = 0; i < n && i < capacity; ++i) stage_of[i] = g_prof_stage[i];
  g_prof_n = 0;
  return n;
}

SMOE_API int smoe_events_create(int n, void** events) {
  if (n < 0 || (n && !events)) return fail(SMOE_EINVAL, "events");
  for (int i = 0; i < n; ++i) {
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) return fail(SMOE_EHIP, "hipEventCreate");
    events[i] = e;
  }
  return SMOE_OK;
}

SMOE_API int smoe_events_destroy(int n, void** events) {
  for (int i = 0; i < n; ++i)
    if (events[i]) (void)hipEventDestroy(static_cast<hipEvent_t>(events[i]));
  return SMOE_OK;
}

SMOE_API int smoe_events_elapsed(int pairs, void** events, float* ms) {
  if (pairs < 0 || (pairs && (!events || !ms))) return fail(SMOE_EINVAL, "events");
  for (int i = 0; i < pairs; ++i) {
    hipEvent_t b = static_cast<hipEvent_t>(events[2 * i]);
    hipEvent_t e = static_cast<hipEvent_t>(events[2 * i + 1]);
    if (hipEventSynchronize(e) != hipSuccess) return fail(SMOE_EHIP, "hipEventSynchronize");
    if (hipEventElapsedTime(&ms[i], b, e) != hipSuccess) return fail(SMOE_EHIP, "hipEventElapsedTime");
  }
  return SMOE_OK;
}

SMOE_API size_t smoe_router_workspace_bytes(int N, int E) {
  const size_t n = N > 0 ? N : 1;
  return align_up(n * E * 4) + 2 * align_up(n * 16 * 4);
}

SMOE_API int smoe_router_topk(const void* x, int act_dtype, int N, int H, const void* router_w,
                              const float* loop_bias_row, int E, int K, float* logits,
                              float* top_w, int32_t* top_idx, void* ws, size_t ws_bytes,
                              void* stream) {
  if (act_dtype != SMOE_F32 && act_dtype != SMOE_BF16) return fail(SMOE_EUNSUPPORTED, "dtype");
  if (N < 0 || H <= 0 || E < 1 || E > 256 || K < 1 || K > E || K > 16)
    return fail(SMOE_EINVAL, "router shape");
  if (N == 0) return SMOE_OK;
  if (!x || !router_w || !top_w || !top_idx || !ws) return fail(SMOE_EINVAL, "null buffer");
  if (ws_bytes < smoe_router_workspace_bytes(N, E)) return fail(SMOE_ECAPACITY, "workspace");
  hipStream_t s = static_cast<hipStream_t>(stream);
  Bump z;
  float* lg = logits ? logits : at<float>(ws, z.take(static_cast<size_t>(N) * E * 4));
  if (logits) z.take(static_cast<size_t>(N) * E * 4);
  int32_t* te = at<int32_t>(ws, z.take(static_cast<size_t>(N) * 16 * 4));
  float* tw = at<float>(ws, z.take(static_cast<size_t>(N) * 16 * 4));
  GemmArgs rg;
  rg.fmt = act_dtype == SMOE_F32 ? SMOE_F32 : SMOE_BF16;
  rg.epi = EPI_F32_BIAS;
  rg.A = x;
  rg.lda = H;
  rg.W = router_w;
  rg.ldw = H;
  rg.K = H;
  rg.N_out = E;
  rg.single_rows = N;
  rg.out = lg;
  rg.ldo = E;
  rg.bias = loop_bias_row;
  SMOE_TRY(launch_router_logits(rg, s), "router logits");
  SMOE_TRY(launch_route_topk(lg, N, E, K, top_idx, top_w, te, tw, nullptr, s), "route_topk");
  return SMOE_OK;
}

SMOE_API size_t smoe_dispatch_workspace_bytes(int N, int K, int E) {
  const size_t n = N > 0 ? N : 1;
  return 2 * align_up(n * K * 4) + align_up(E * 4) + align_up(plan_scratch_bytes(N, E));
}

SMOE_API int smoe_dispatch_plan(const int32_t* idx, const float* w, int N, int K, int E,
                                int32_t* counts, int32_t* offsets, int32_t* rows, float* row_w,
                                int32_t* tok_row, void* ws, size_t ws_bytes, void* stream) {
  if (N < 0 || K < 1 || K > 256 || E < 1 || E > 256) return fail(SMOE_EINVAL, "plan shape");
  if (!counts || !offsets) return fail(SMOE_EINVAL, "null buffer");
  if (N > 0 && (!idx || !w || !rows || !row_w || !tok_row || !ws))
    return fail(SMOE_EINVAL, "null buffer");
  if (ws_bytes < smoe_dispatch_workspace_bytes(N, K, E)) return fail(SMOE_ECAPACITY, "workspace");
  hipStream_t s = static_cast<hipStream_t>(stream);
  Bump z;
  int32_t* tg = at<int32_t>(ws, z.take(static_cast<size_t>(N) * K * 4));
  float* tw = at<float>(ws, z.take(static_cast<size_t>(N) * K * 4));
  int32_t* acnt = at<int32_t>(ws, z.take(E * 4));
  void* scratch = at<void>(ws, z.take(plan_scratch_bytes(N, E)));
  SMOE_TRY(launch_merge_slots(idx, w, N, K, E, 1, tg, tw, s), "merge slots");
  SMOE_TRY(launch_plan(tg, tw, N, K, E, 1, counts, acnt, offsets, rows, row_w, tok_row, scratch, s),
           "plan");
  return SMOE_OK;
}

SMOE_API size_t smoe_expert_delta_workspace_bytes(const smoe_experts* ex, int N, int K) {
  if (!ex || check_experts(*ex, ex->H) != SMOE_OK) return 0;
  const size_t n = N > 0 ? N : 1;
  const size_t es = esize(ffn_dtype_of(*ex));
  return smoe_dispatch_workspace_bytes(N, K, ex->E) + align_up((ex->E + 1) * 4) +
         align_up(ex->E * 4) + 3 * align_up(n * K * 4) +
         align_up(row_tile_elems(static_cast<int64_t>(n) * K, ex->U) * es) +
         align_up(n * K * ex->H * es);
}

SMOE_API int smoe_expert_delta(const smoe_experts* ex, const void* msg, const int32_t* idx,
                               const float* w, int N, int K, void* delta, int out_dtype,
                               void* ws, size_t ws_bytes, void* stream) {
  if (!ex) return fail(SMOE_EINVAL, "null experts");
  int rc = check_experts(*ex, ex->H);
  if (rc != SMOE_OK) return rc;
  if (N < 0 || K < 1 || K > 64) return fail(SMOE_EINVAL, "shape (1 <= top_k <= 64)");
  if (out_dtype != SMOE_F32 && out_dtype != SMOE_BF16) return fail(SMOE_EUNSUPPORTED, "out dtype");
  if (N == 0) return SMOE_OK;
  if (!msg || !idx || !w || !delta || !ws) return fail(SMOE_EINVAL, "null buffer");
  if (ws_bytes < smoe_expert_delta_workspace_bytes(ex, N, K))
    return fail(SMOE_ECAPACITY, "workspace");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int E = ex->E;
  const size_t es = esize(ffn_dtype_of(*ex));
  Bump z;
  void* pws = at<void>(ws, z.take(smoe_dispatch_workspace_bytes(N, K, E)));
  int32_t* off = at<int32_t>(ws, z.take((E + 1) * 4));
  int32_t* cnt = at<int32_t>(ws, z.take(E * 4));
  int32_t* rows = at<int32_t>(ws, z.take(static_cast<size_t>(N) * K * 4));
  float* roww = at<float>(ws, z.take(static_cast<size_t>(N) * K * 4));
  int32_t* tokrow = at<int32_t>(ws, z.take(static_cast<size_t>(N) * K * 4));
  void* act = at<void>(ws, z.take(row_tile_elems(static_cast<int64_t>(N) * K, ex->U) * es));
  void* y = at<void>(ws, z.take(static_cast<size_t>(N) * K * ex->H * es));
  rc = smoe_dispatch_plan(idx, w, N, K, E, cnt, off, rows, roww, tokrow, pws,
                          smoe_dispatch_workspace_bytes(N, K, E), stream);
  if (rc != SMOE_OK) return rc;
  rc = run_experts(*ex, msg, off, rows, roww, N * K, act, y, s);
  if (rc != SMOE_OK) return rc;
  SMOE_TRY(launch_delta_combine(y, ffn_dtype_of(*ex), tokrow, N, K, ex->H, delta, out_dtype, s),
           "delta combine");
  return SMOE_OK;
}

// ------------------------------------------------ stage entry points ----
namespace {

int check_act(int adt, int H) {
  if (adt != SMOE_F32 && adt != SMOE_BF16) return fail(SMOE_EUNSUPPORTED, "act_dtype");
  if (H <= 0 || H % 8 || H > 4096) return fail(SMOE_EINVAL, "H (H % 8 == 0, <= 4096)");
  return SMOE_OK;
}



// workspace of smoe_edge_topm
struct TopmWs {
  size_t tok_e, tok_ew, cnt, acnt, off, rows, roww, tokrow, scratch, logit, eidx, ew, tok_d, tok_dc;
  size_t total;
};
TopmWs topm_ws(int N, int K, int E, int M) {
  const size_t n = N > 0 ? static_cast<size_t>(N) : 1;
  const int S = E < K * M ? E : K * M;
  TopmWs w;
  Bump z;
  w.tok_e = z.take(n * K * 4);
  w.tok_ew = z.take(n * K * 4);
  w.cnt = z.take(E * 4);
  w.acnt = z.take(E * 4);
  w.off = z.take((E + 1) * 4);
  w.rows = z.take(n * K * 4);
  w.roww = z.take(n * K * 4);
  w.tokrow = z.take(n * K * 4);
  w.scratch = z.take(plan_scratch_bytes(N, E));
  w.logit = z.take(n * K * E * 4);
  w.eidx = z.take(n * K * M * 4);
  w.ew = z.take(n * K * M * 4);
  w.tok_d = z.take(n * S * 4);
  w.tok_dc = z.take(n * S * 4);
  w.total = z.off;
  return w;
}

// workspace of smoe_edge_message
struct MsgWs {
  size_t tok_d, tok_dc, cnt, acnt, off, rows, roww, tokrow, scratch, proj, total;
};
MsgWs msg_ws(int N, int H, int E, int K, int M, int adt) {
  const size_t n = N > 0 ? static_cast<size_t>(N) : 1;
  const int S = E < K * M ? E : K * M;
  MsgWs w;
  Bump z;
  w.tok_d = z.take(n * S * 4);
  w.tok_dc = z.take(n * S * 4);
  w.cnt = z.take(E * 4);
  w.acnt = z.take(E * 4);
  w.off = z.take((E + 1) * 4);
  w.rows = z.take(n * S * 4);
  w.roww = z.take(n * S * 4);
  w.tokrow = z.take(n * S * 4);
  w.scratch = z.take(plan_scratch_bytes(N, E));
  w.proj = z.take(n * S * H * esize(adt));
  w.total = z.off;
  return w;
}

}  // namespace

SMOE_API size_t smoe_edge_topm_workspace_bytes(int N, int K, int E, int M) {
  if (N < 0 || check_ekm(E, K, M) != SMOE_OK) return 0;
  return topm_ws(N, K, E, M).total;
}

SMOE_API int smoe_edge_topm(const void* x, int act_dtype, int N, int H, const void* edge_gen_w,
                            int ldw, const float* edge_bias, int E, int K, int M,
                            const int32_t* src_idx, int32_t* out_eidx, float* out_ew, void* ws,
                            size_t ws_bytes, void* stream) {
  int rc = check_act(act_dtype, H);
  if (rc != SMOE_OK) return rc;
  rc = check_ekm(E, K, M);
  if (rc != SMOE_OK) return rc;
  if (N < 0 || ldw < H || ldw % 8) return fail(SMOE_EINVAL, "shape (ldw >= H, ldw % 8 == 0)");
  if (N == 0) return SMOE_OK;
  if (!x || !edge_gen_w || !edge_bias || !src_idx || !out_eidx || !out_ew || !ws)
    return fail(SMOE_EINVAL, "null buffer");
  const TopmWs l = topm_ws(N, K, E, M);
  if (ws_bytes < l.total) return fail(SMOE_ECAPACITY, "workspace");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int S = E < K * M ? E : K * M;
  // the token's sources: distinct, ascending, each weighing 1 (the edges of
  // a source do not depend on its router weight)
  SMOE_TRY(launch_merge_slots(src_idx, nullptr, N, K, E, 0, at<int32_t>(ws, l.tok_e),
                              at<float>(ws, l.tok_ew), s),
           "source slots");
  SMOE_TRY(launch_plan(at<int32_t>(ws, l.tok_e), at<float>(ws, l.tok_ew), N, K, E, 0,
                       at<int32_t>(ws, l.cnt), at<int32_t>(ws, l.acnt), at<int32_t>(ws, l.off),
                       at<int32_t>(ws, l.rows), at<float>(ws, l.roww), at<int32_t>(ws, l.tokrow),
                       at<void>(ws, l.scratch), s),
           "source plan");
  GemmArgs eg;
  eg.fmt = act_dtype == SMOE_F32 ? SMOE_F32 : SMOE_BF16;
  eg.epi = EPI_F32_BIAS;
  eg.A = x;
  eg.lda = H;
  eg.a_rows = at<int32_t>(ws, l.rows);
  eg.W = edge_gen_w;
  eg.w_gstride = static_cast<int64_t>(E) * ldw;
  eg.ldw = ldw;
  eg.K = H;
  eg.N_out = E;
  eg.grp_off = at<int32_t>(ws, l.off);
  eg.G = E;
  eg.max_rows = N * K;
  eg.out = at<float>(ws, l.logit);
  eg.ldo = E;
  eg.bias = edge_bias;
  eg.bias_gstride = E;
  SMOE_TRY(launch_grouped_gemm(eg, s), "edge-logit GEMM");
  SMOE_TRY(launch_edge_topm(at<float>(ws, l.logit), at<int32_t>(ws, l.tok_e), at<int32_t>(ws, l.tokrow),
                            N, E, K, M, S, at<int32_t>(ws, l.eidx), at<float>(ws, l.ew),
                            at<int32_t>(ws, l.tok_d), at<float>(ws, l.tok_dc), s),
           "edge top-m");
  SMOE_TRY(launch_gather_topm(src_idx, at<int32_t>(ws, l.tok_e), at<int32_t>(ws, l.tokrow),
                              at<int32_t>(ws, l.eidx), at<float>(ws, l.ew), N, K, M, out_eidx,
                              out_ew, s),
           "top-m gather");
  return SMOE_OK;
}

SMOE_API size_t smoe_edge_message_workspace_bytes(int N, int H, int E, int K, int M,
                                                  int act_dtype) {
  if (N < 0 || H <= 0 || check_ekm(E, K, M) != SMOE_OK) return 0;
  if (act_dtype != SMOE_F32 && act_dtype != SMOE_BF16) return 0;
  return msg_ws(N, H, E, K, M, act_dtype).total;
}

SMOE_API int smoe_edge_message(const void* x, int act_dtype, int N, int H,
                               const void* edge_value_w, const void* edge_value_w_tiles, int E,
                               int K, int M, const int32_t* src_idx, const int32_t* eidx,
                               const float* ew, void* msg, int msg_dtype, void* ws,
                               size_t ws_bytes, void* stream) {
  int rc = check_act(act_dtype, H);
  if (rc != SMOE_OK) return rc;
  rc = check_ekm(E, K, M);
  if (rc != SMOE_OK) return rc;
  if (msg_dtype != SMOE_F32 && msg_dtype != SMOE_BF16) return fail(SMOE_EUNSUPPORTED, "msg dtype");
  if (N < 0) return fail(SMOE_EINVAL, "N");
  if (N == 0) return SMOE_OK;
  if (!x || !edge_value_w || !src_idx || !eidx || !ew || !msg || !ws)
    return fail(SMOE_EINVAL, "null buffer");
  const MsgWs l = msg_ws(N, H, E, K, M, act_dtype);
  if (ws_bytes < l.total) return fail(SMOE_ECAPACITY, "workspace");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int S = E < K * M ? E : K * M;
  SMOE_TRY(launch_dest_coeffs(src_idx, eidx, ew, N, K, M, E, S, at<int32_t>(ws, l.tok_d),
                              at<float>(ws, l.tok_dc), s),
           "destination coefficients");
  SMOE_TRY(launch_plan(at<int32_t>(ws, l.tok_d), at<float>(ws, l.tok_dc), N, S, E, 1,
                       at<int32_t>(ws, l.cnt), at<int32_t>(ws, l.acnt), at<int32_t>(ws, l.off),
                       at<int32_t>(ws, l.rows), at<float>(ws, l.roww), at<int32_t>(ws, l.tokrow),
                       at<void>(ws, l.scratch), s),
           "destination plan");
  GemmArgs pg;
  pg.fmt = act_dtype == SMOE_F32 ? SMOE_F32 : SMOE_BF16;
  pg.epi = EPI_ROWSCALE;
  pg.A = x;
  pg.lda = H;
  pg.a_rows = at<int32_t>(ws, l.rows);
  pg.W = edge_value_w;
  pg.Wt = act_dtype == SMOE_BF16 ? edge_value_w_tiles : nullptr;
  pg.w_gstride = static_cast<int64_t>(H) * H;
  pg.ldw = H;
  pg.K = H;
  pg.N_out = H;
  pg.grp_off = at<int32_t>(ws, l.off);
  pg.G = E;
  pg.max_rows = N * S;
  pg.out = at<void>(ws, l.proj);
  pg.ldo = H;
  pg.out_dtype = act_dtype;
  pg.row_scale = at<float>(ws, l.roww);
  SMOE_TRY(launch_grouped_gemm(pg, s), "edge GEMM");
  SMOE_TRY(launch_msg_combine(at<void>(ws, l.proj), act_dtype, at<int32_t>(ws, l.tok_d),
                              at<int32_t>(ws, l.tokrow), N, S, H, msg, msg_dtype, s),
           "message combine");
  return SMOE_OK;
}

SMOE_API int smoe_select_topk(const float* logits, int N, int E, int K, int mode, float* top_w,
                              int32_t* top_idx, void* stream) {
  if (N < 0 || E < 1 || E > 256 || K < 1 || K > E || K > 64)
    return fail(SMOE_EINVAL, "select shape (1 <= K <= min(E, 64), E <= 256)");
  if (mode != SMOE_SELECT_ROUTER && mode != SMOE_SELECT_TOPK_SOFTMAX)
    return fail(SMOE_EINVAL, "select mode");
  if (N == 0) return SMOE_OK;
  if (!logits || !top_w || !top_idx) return fail(SMOE_EINVAL, "null buffer");
  SMOE_TRY(launch_select_topk(logits, N, E, K, mode, top_w, top_idx,
                              static_cast<hipStream_t>(stream)),
           "select top-k");
  return SMOE_OK;
}

SMOE_API int smoe_linear(const void* x, int N, int K, const void* w, int w_format,
                         const float* w_scale, const float* bias, int N_out, int act, void* out,
                         int out_dtype, void* stream) {
  if (N < 0 || K <= 0 || N_out <= 0) return fail(SMOE_EINVAL, "linear shape");
  if (w_format != SMOE_F32 && w_format != SMOE_BF16 && w_format != SMOE_FP8_E4M3)
    return fail(SMOE_EUNSUPPORTED, "linear weight format");
  if (act != SMOE_LINEAR_NONE && act != SMOE_LINEAR_GELU) return fail(SMOE_EINVAL, "act");
  if (out_dtype != SMOE_F32 && out_dtype != SMOE_BF16) return fail(SMOE_EUNSUPPORTED, "out dtype");
  if (act == SMOE_LINEAR_NONE && out_dtype != SMOE_F32)
    return fail(SMOE_EUNSUPPORTED, "a linear without activation writes f32");
  if (w_format == SMOE_F32 && out_dtype != SMOE_F32) return fail(SMOE_EINVAL, "f32 linear: f32 out");
  if (w_format == SMOE_FP8_E4M3 && K % 32) return fail(SMOE_EINVAL, "fp8 linear: K % 32 == 0");
  if (w_format == SMOE_FP8_E4M3 && !w_scale) return fail(SMOE_EINVAL, "fp8 weights need a scale");
  if (N == 0) return SMOE_OK;
  if (!x || !w || !out) return fail(SMOE_EINVAL, "null buffer");
  GemmArgs g;
  g.fmt = w_format;
  g.epi = act == SMOE_LINEAR_GELU ? EPI_GELU : EPI_F32_BIAS;
  g.A = x;
  g.lda = K;
  g.W = w;
  g.ldw = K;
  g.S = w_scale;
  g.K = K;
  g.N_out = N_out;
  g.G = 0;
  g.single_rows = N;
  g.out = out;
  g.ldo = N_out;
  g.out_dtype = out_dtype;
  g.bias = bias;
  SMOE_TRY(launch_grouped_gemm(g, static_cast<hipStream_t>(stream)), "linear GEMM");
  return SMOE_OK;
}

SMOE_API size_t smoe_quantize_fp8_workspace_bytes(void) { return quantize_fp8_workspace_bytes(); }

SMOE_API int smoe_quantize_fp8_tensor(const void* x, int x_dtype, int rows, int cols, int ld_out,
                                      int per_row, uint8_t* codes, float* scale, void* workspace,
                                      size_t workspace_bytes, void* stream) {
  if (rows < 0 || cols < 1 || ld_out < cols || ld_out % 4)
    return fail(SMOE_EINVAL, "quantize shape (cols >= 1, ld_out >= cols, ld_out % 4 == 0)");
  if (x_dtype != SMOE_F32 && x_dtype != SMOE_BF16 && x_dtype != SMOE_F16)
    return fail(SMOE_EUNSUPPORTED, "quantize input dtype");
  if (rows == 0) return SMOE_OK;
  if (!x || !codes || !scale || (!per_row && !workspace)) return fail(SMOE_EINVAL, "null buffer");
  if (!per_row && workspace_bytes < quantize_fp8_workspace_bytes())
    return fail(SMOE_ECAPACITY, "workspace");
  SMOE_TRY(launch_quantize_fp8(x, x_dtype, rows, cols, ld_out, per_row, codes, scale, workspace,
                               static_cast<hipStream_t>(stream)),
           "quantize fp8");
  return SMOE_OK;
}

SMOE_API int smoe_linear_fp8fp8(const uint8_t* xq, const float* x_scale, int N, int K,
                                const uint8_t* wq, const float* w_scale, const float* bias,
                                int N_out, int act, void* out, int out_dtype, void* stream) {
  if (N < 0 || K <= 0 || K % 256 || N_out <= 0)
    return fail(SMOE_EINVAL, "fp8 x fp8 linear shape (K % 256 == 0: zero-padded codes)");
  if (act != SMOE_LINEAR_NONE && act != SMOE_LINEAR_GELU) return fail(SMOE_EINVAL, "act");
  if (out_dtype != SMOE_F32 && out_dtype != SMOE_BF16) return fail(SMOE_EUNSUPPORTED, "out dtype");
  if (N == 0) return SMOE_OK;
  if (!xq || !wq || !x_scale || !w_scale || !out) return fail(SMOE_EINVAL, "null buffer");
  SMOE_TRY(launch_gemm_f8f8(xq, K, x_scale, wq, K, w_scale, bias, N, K, N_out,
                            act == SMOE_LINEAR_GELU, out, out_dtype, N_out,
                            static_cast<hipStream_t>(stream)),
           "fp8 x fp8 GEMM");
  return SMOE_OK;
}

SMOE_API int smoe_combine_rows(const void* y, int y_dtype, const float* row_w,
                               const int32_t* tok_row, int N, int K, int H, void* out,
                               int out_dtype, void* stream) {
  if (N < 0 || K < 1 || K > 64 || H <= 0 || H % 8 || H > 4096)
    return fail(SMOE_EINVAL, "combine shape (1 <= K <= 64, H % 8 == 0, H <= 4096)");
  if ((y_dtype != SMOE_F32 && y_dtype != SMOE_BF16) || (out_dtype != SMOE_F32 && out_dtype != SMOE_BF16))
    return fail(SMOE_EUNSUPPORTED, "combine dtype");
  if (N == 0) return SMOE_OK;
  if (!y || !tok_row || !out) return fail(SMOE_EINVAL, "null buffer");
  SMOE_TRY(launch_combine_rows(y, y_dtype, row_w, tok_row, N, K, H, out, out_dtype,
                               static_cast<hipStream_t>(stream)),
           "combine rows");
  return SMOE_OK;
}

SMOE_API int smoe_remap_ids(const int32_t* ids, int64_t n, const int32_t* map, int E,
                            int32_t* out, void* stream) {
  if (n < 0 || E < 0) return fail(SMOE_EINVAL, "remap shape");
  if (n == 0) return SMOE_OK;
  if (!ids || !out || (E > 0 && !map)) return fail(SMOE_EINVAL, "null buffer");
  SMOE_TRY(launch_remap_ids(ids, n, map, E, out, static_cast<hipStream_t>(stream)), "remap ids");
  return SMOE_OK;
}

SMOE_API int smoe_combine_epilogue(const void* h, const void* x0, int act_dtype, const void* delta,
                                   int delta_dtype, int N, int H, float alpha, float beta,
                                   const float* ln_w, const float* ln_b, float eps, void* out,
                                   void* stream) {
  int rc = check_act(act_dtype, H);
  if (rc != SMOE_OK) return rc;
  if (delta_dtype != SMOE_F32 && delta_dtype != SMOE_BF16)
    return fail(SMOE_EUNSUPPORTED, "delta dtype");
  if (N < 0) return fail(SMOE_EINVAL, "N");
  if (N == 0) return SMOE_OK;
  if (!h || !x0 || !delta || !out) return fail(SMOE_EINVAL, "null buffer");
  SMOE_TRY(launch_epilogue(h, x0, act_dtype, delta, delta_dtype, nullptr, nullptr, nullptr, N, 1, H,
                           alpha, beta, ln_w, ln_b, eps, out, nullptr,
                           static_cast<hipStream_t>(stream)),
           "epilogue");
  return SMOE_OK;
}

}  // extern "C"
