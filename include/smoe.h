/*
 * smoe.h — C ABI of libsmoe.so, the gfx950 (MI355X) Spider-MoE block.
 *
 * One loop of the recurrent block (spider_moe/model.py:240-317 of the
 * reference, run num_loops times by model.py:445-448):
 *   router top-k  ->  edge generator top-m  ->  destination-grouped edge
 *   projection + message combine  ->  dispatch by expert  ->  grouped expert
 *   FFN (f32 / bf16 / fp8-e4m3 / int4 weights)  ->  weighted combine +
 *   residual + LayerNorm.
 *
 * Conventions follow the reference's native ABI (kernels/include/
 * spider_kernels.h:26-149, spider_cuda.h:8-60):
 *   - every entry point returns int: 0 ok, 1 invalid argument, 2 index out of
 *     range, 3 capacity (workspace too small), -2 unsupported dtype/format,
 *     4 HIP runtime error (the HIP error string is kept for smoe_last_error);
 *   - the caller owns every buffer (inputs, outputs and the workspace, whose
 *     size comes from the *_workspace_bytes queries); nothing allocates;
 *   - the stream is an opaque hipStream_t passed as void* (spider_cuda.h:8);
 *   - tensors are row-major and contiguous, indices int32;
 *   - all device pointers; calls enqueue work on `stream` and return without
 *     synchronizing.
 * Calls that share a workspace must not overlap in time.
 */
#pragma once
#include <stddef.h>
#include <stdint.h>

#if defined(_WIN32)
#define SMOE_API __declspec(dllexport)
#else
#define SMOE_API __attribute__((visibility("default")))
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define SMOE_ABI_VERSION 10

/* status codes (spider_kernels.h convention; see scalar.cpp:9,45,58) */
#define SMOE_OK 0
#define SMOE_EINVAL 1
#define SMOE_ERANGE 2
#define SMOE_ECAPACITY 3
#define SMOE_EUNSUPPORTED (-2)
#define SMOE_EHIP 4
/* smoe_block_forward_scratch only: an earlier call on this GPU, enqueued on
 * another stream, has not finished (its static workspace is in use) */
#define SMOE_EBUSY 5

/* element formats */
#define SMOE_F32 0
#define SMOE_BF16 1
#define SMOE_FP8_E4M3 2 /* OCP e4m3fn codes + per-output-channel fp32 scale  */
#define SMOE_INT4 3     /* 2 per byte, low nibble first, per-group scales     */
#define SMOE_F16 4      /* scale dtype only                                   */

/* expert activations */
#define SMOE_ACT_GELU 0   /* Linear(+b) -> GELU(erf) -> Linear(+b)  (model.py:177-183) */
#define SMOE_ACT_SWIGLU 1 /* W_down (silu(W_gate x) * (W_up x (+b_up))) (+b_down)     */

/* Expert FFN weights, stacked over experts (the reference stacks them per
 * call, model.py:305-308; here they are stacked once).
 *   f32 / bf16: w_up [E,U,H], w_down [E,H,U] elements.
 *   fp8:        codes with the same shapes; s_up f32 [E,U], s_down f32 [E,H]
 *               (per output channel; quant.py:146-169 with a per-row scale).
 *   int4:       w_up [E,U,H/2] bytes, s_up [E,U,H/g]; w_down [E,H,U/2],
 *               s_down [E,H,U/g]; scales f32 or f16 (quant.py:89-143).
 *   SwiGLU:     w_up holds the gate and up projections interleaved by
 *               blocks of 32 rows — rows [64j, 64j+32) are gate rows
 *               [32j, 32j+32) and rows [64j+32, 64j+64) are up rows
 *               [32j, 32j+32) — so w_up is [E,2U,H] (and s_up [E,2U(,..)]).
 *               w_gate must be NULL.
 *   b_up [E,U] and b_down [E,H] are fp32 or NULL.
 * Shapes: 1 <= E <= 256.  f32 experts and bf16 GELU experts take any H
 * and U (shapes off the MFMA kernels' grid run a SIMT kernel); SwiGLU,
 * fp8 and int4 experts need H, U % 32 == 0 (SwiGLU U % 64, int4 the group
 * size dividing both).  Within a block (smoe_block) and the routing stages:
 * H % 8 == 0, H <= 4096, E <= 256, 1 <= K, M <= min(E, 16) and
 * min(E, K * M) <= 64 (the destinations a token can reach, one lane each);
 * the reference takes any shape (model.py:165-185), these limits return
 * SMOE_EINVAL. */
typedef struct smoe_experts {
  int format;      /* SMOE_F32 / SMOE_BF16 / SMOE_FP8_E4M3 / SMOE_INT4 */
  int act;         /* SMOE_ACT_GELU / SMOE_ACT_SWIGLU */
  int E, H, U;
  int group_size;  /* int4 only */
  int scale_dtype; /* int4: SMOE_F32 or SMOE_F16; fp8: SMOE_F32 */
  const void* w_up;
  const void* w_gate; /* reserved, must be NULL */
  const void* w_down;
  const void* s_up;
  const void* s_down;
  const float* b_up;
  const float* b_down;
  /* optional: w_up / w_down in the weight tile layout, NULL to read the
   * row-major weights.  bf16 and fp8 (smoe_pack_weight_tiles): read instead
   * of them by the decode weight stream and the ping-pong GEMM (bit-identical
   * results for bf16).  int4 (smoe_pack_int4_qtiles): the int4 tile layout,
   * read by the ping-pong GEMM at prefill sizes (>= 256 rows per expert) in
   * place of the general int4 kernel; the decode and stream kernels keep
   * reading the packed int4. */
  const void* w_up_tiles;
  const void* w_down_tiles;
} smoe_experts;

/* One Spider-MoE block (parameters of model.py:165-185).
 * act_dtype (SMOE_F32 or SMOE_BF16) is the dtype of h, x0, the output and of
 * router_w, edge_gen_w and edge_value_w.  loop_bias [R,E] and
 * edge_loop_bias [R,E*E] are fp32; edge_loop_bias[r] = b_g + W_g[:,H:] .
 * loop_embedding[r], filled by smoe_edge_loop_bias(). */
typedef struct smoe_block {
  int act_dtype;
  int H, E, K, M, L, R; /* hidden, experts, top_k, edges_per_expert, loop_embed_size, num_loops */
  const void* router_w;       /* [E,H]      router.weight          */
  const float* loop_bias;     /* [R,E]      loop_bias              */
  const void* edge_gen_w;     /* [E*E,H+L]  edge_generator.weight  */
  const float* edge_loop_bias;/* [R,E*E]                           */
  const void* edge_value_w;   /* [E,H,H]    edge_value.{e}.weight  */
  smoe_experts experts;       /*            experts.{e}.{0,2}      */
  const float* ln_w;          /* [H]        norm.weight            */
  const float* ln_b;          /* [H]        norm.bias              */
  float alpha;                /* residual_scale  (config.py:18)    */
  float beta;                 /* re_inject_weight (config.py:19)   */
  float eps;                  /* LayerNorm eps (1e-5)              */
  const void* edge_value_w_tiles; /* optional (bf16): edge_value_w in the weight
                                     tile layout, or NULL            */
} smoe_block;

/* Byte offsets of the named regions inside a block workspace (for tests and
 * diagnostics: they hold the last loop's routing after a call). */
typedef struct smoe_ws_layout {
  size_t total;
  size_t logits;    /* f32 [N,E]      router logits (+ loop bias)                 */
  size_t top_idx;   /* i32 [N,K]      router top-k, descending probability        */
  size_t top_w;     /* f32 [N,K]      renormalized top-k weights                  */
  size_t tok_e;     /* i32 [N,K]      token's distinct experts, ascending, -1 pad  */
  size_t tok_ew;    /* f32 [N,K]      merged weight of each                        */
  size_t e_cnt;     /* i32 [E]        rows per expert (all distinct top-k pairs)  */
  size_t e_acnt;    /* i32 [E]        rows with weight > 0 (the dispatch counts)  */
  size_t e_off;     /* i32 [E+1]      row offsets                                 */
  size_t e_rows;    /* i32 [N*K]      token of each row, (expert, token) order    */
  size_t e_roww;    /* f32 [N*K]      weight of each row                          */
  size_t e_tokrow;  /* i32 [N,K]      row of each tok_e entry                     */
  size_t edge_logit;/* f32 [N*K,E]    edge logits of each source row              */
  size_t edge_idx;  /* i32 [N*K,M]    top-m destinations of each source row       */
  size_t edge_w;    /* f32 [N*K,M]    their softmax weights                       */
  size_t tok_d;     /* i32 [N,S]      token's destinations, ascending, -1 pad     */
  size_t tok_dc;    /* f32 [N,S]      destination coefficients                    */
  size_t d_cnt;     /* i32 [E]        rows per destination                        */
  size_t d_acnt;    /* i32 [E]        (same as d_cnt: zero coefficients are dropped) */
  size_t d_off;     /* i32 [E+1]                                                 */
  size_t d_rows;    /* i32 [N*S]                                                 */
  size_t d_roww;    /* f32 [N*S]                                                 */
  size_t d_tokrow;  /* i32 [N,S]                                                 */
  size_t proj;      /* act  [N*S,H]   c * W_edge[d] h per destination row         */
  size_t msg;       /* ffn  [N,H]     messages                                    */
  size_t act;       /* ffn  [N*K,U]   expert hidden activations (row-major, or in   */
                    /* 16-row bands of 1 KB lane-ordered 16x32 blocks, the weight */
                    /* tile layout, between the large-tile GEMMs; N*K rounded up  */
                    /* to 16 rows)                                                */
  size_t y;         /* ffn  [N*K,H]   weighted expert outputs                     */
  size_t h_tmp;     /* act  [N,H]     loop ping-pong buffer                       */
  size_t scratch;   /* plan scratch                                               */
  size_t front;     /* f32 [N,E+E*E]  router logits | edge logits of every source,  */
                    /*                bf16 steps of N <= 64 (else 0 bytes)          */
  size_t sel_idx;   /* i32 [N,K,M]    decode loop: the top-m of each token's sources */
  size_t sel_w;     /* f32 [N,K,M]    (ascending), their weights (else 0 bytes)     */
  size_t h_tmp2;    /* act [N,H]      decode loop: second loop-input buffer         */
  int S;            /* destinations per token: min(E, K*M)                        */
  int ffn_dtype;    /* SMOE_F32 or SMOE_BF16                                      */
} smoe_ws_layout;

SMOE_API int smoe_abi_version(void);
/* spider_backend_name / spider_backend_caps (spider_kernels.h:148-149) */
SMOE_API const char* smoe_backend_name(void);
SMOE_API uint32_t smoe_backend_caps(void); /* bit i set = format i supported */
SMOE_API const char* smoe_last_error(void);

/* Workspace for smoe_block_forward over N tokens, and its layout. */
SMOE_API size_t smoe_block_workspace_bytes(const smoe_block* blk, int N);
SMOE_API int smoe_block_workspace_layout(const smoe_block* blk, int N, smoe_ws_layout* out);

/* edge_loop_bias[r, o] = b_g[o] + sum_l W_g[o, H+l] * loop_emb[r, l]
 * (the loop-embedding half of edge_generator, model.py:261-263).
 * W_g in act_dtype [E*E, H+L]; b_g f32 [E*E] or NULL; loop_emb f32 [R,L]. */
SMOE_API int smoe_edge_loop_bias(const void* edge_gen_w, int act_dtype, const float* edge_gen_b,
                                 const float* loop_emb, int E, int H, int L, int R,
                                 float* out, void* stream);

/* SpiderMoELayer.forward (model.py:240-317) for loops
 * [loop_begin, loop_begin + num_loops), back to back on `stream`, no host
 * synchronization; with num_loops > 1 it is SpiderWebLM._run_recurrent_full
 * (model.py:445-448).  h_in, x0, h_out: [N,H] in act_dtype; h_out may alias
 * h_in.  Replaces the reference's fused step spider_moe_loop_step_f32
 * (spider_kernels.h:113-121) and the declared-only
 * spider_cuda_moe_loop_step_f32 (spider_cuda.h:35-44). */
SMOE_API int smoe_block_forward(const smoe_block* blk, const void* h_in, const void* x0,
                                void* h_out, int N, int loop_begin, int num_loops,
                                void* workspace, size_t workspace_bytes, void* stream);

/* Early-exit decode (SpiderWebLM._run_recurrent_decode with early_exit,
 * model.py:450-473, and the early_exit branch of SpiderWebLM.forward,
 * model.py:683-698; the ActiveSet compaction of spider_moe/active_set.py:14-64
 * kept on the device): smoe_block_forward over the tokens still in orbit.
 * active i32 [N] in/out: nonzero = in orbit.  Per loop, tokens with
 * active[t] == 0 get no routing (no expert or edge work) and keep their h;
 * every other token gets h' and leaves the orbit (active[t] := 0) when
 * sigmoid(exit_wb[0:H] . h' + exit_wb[H]) > threshold, computed in fp32 over
 * h' as stored (exit_head, model.py:185,467).  loops i32 [N] in/out or NULL:
 * incremented for each loop a token runs.  No host synchronization: a
 * fixed-R decode step with early exit can be captured in one HIP graph.
 * Replaces spider_early_exit_f32 (spider_kernels.h:109-111) and the exit
 * mask of spider_moe_loop_step_f32 (spider_kernels.h:113-121), fused into
 * the block's epilogue. */
SMOE_API int smoe_block_forward_exit(const smoe_block* blk, const void* h_in, const void* x0,
                                     void* h_out, int N, int loop_begin, int num_loops,
                                     const float* exit_wb, float threshold, int32_t* active,
                                     int32_t* loops, void* workspace, size_t workspace_bytes,
                                     void* stream);

/* Allocation-free smoe_block_forward.  No counterpart in the reference: it
 * is for callers that cannot allocate device memory or pass a workspace
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The block workspace is a static device array of
 * SMOE_SCRATCH_BYTES inside libsmoe.so, one per GPU, held until the process
 * ends; a call whose workspace (smoe_block_workspace_bytes(blk, N)) exceeds
 * it fails with SMOE_ECAPACITY and launches nothing.  The limit admits
 * decode-size steps: 64 tokens of the H 1024, E 16, U 2816 block need about
 * 2 MiB.  Every call on a GPU shares that GPU's array (the kernels write
 * every workspace byte they read, so nothing is cleared between calls):
 * calls that overlap in time on one GPU would race, so they are detected:
 * a call on a stream other than the previous call's, made while that call
 * is still running on the GPU, returns SMOE_EBUSY and launches nothing
 * (host threads are serialized around the check and the enqueue).  Calls
 * on one stream never overlap.  Under HIP graph capture the check is
 * skipped: the captured graph orders its own nodes.  The call runs on the
 * current device and `stream` must belong to it.  Arguments and results as
 * smoe_block_forward, bit for bit; no hipMalloc / hipFree or other
 * allocating routine is called. */
#define SMOE_SCRATCH_BYTES (8u << 20)
SMOE_API int smoe_block_forward_scratch(const smoe_block* blk, const void* h_in, const void* x0,
                                        void* h_out, int N, int loop_begin, int num_loops,
                                        void* stream);

/* Router stage alone (model.py:255-258; spider_router_f32,
 * spider_kernels.h:26-28, with the logits GEMM of model.py:255 fused in):
 * x [N,H] act_dtype, router_w [E,H] act_dtype, loop_bias_row f32 [E] or NULL
 * -> logits f32 [N,E] (may be NULL), top_w f32 [N,K], top_idx i32 [N,K].
 * 1 <= K <= min(E, 16), E <= 256. */
SMOE_API size_t smoe_router_workspace_bytes(int N, int E);
SMOE_API int smoe_router_topk(const void* x, int act_dtype, int N, int H, const void* router_w,
                              const float* loop_bias_row, int E, int K, float* logits,
                              float* top_w, int32_t* top_idx, void* workspace,
                              size_t workspace_bytes, void* stream);

/* Dispatch plan (spider_infer/forge/ep/dispatch.py:56-115 build_dispatch_plan,
 * sparse_experts.py:51-56): idx/w [N,K] -> per expert ascending, the tokens
 * whose merged weight is > 0, ascending.  counts [E], offsets [E+1],
 * rows [N*K] (token per row; entries past offsets[E] are unspecified),
 * row_w [N*K], tok_row [N,K] (row of each distinct positive (token, expert),
 * in ascending expert order, -1 padded).  Expert ids outside [0, E) match
 * no expert and are dropped, as the reference's per-expert masks drop them.
 * 1 <= K <= 256, 1 <= E <= 256. */
SMOE_API size_t smoe_dispatch_workspace_bytes(int N, int K, int E);
SMOE_API int smoe_dispatch_plan(const int32_t* idx, const float* w, int N, int K, int E,
                                int32_t* counts, int32_t* offsets, int32_t* rows, float* row_w,
                                int32_t* tok_row, void* workspace, size_t workspace_bytes,
                                void* stream);

/* sparse_expert_delta (sparse_experts.py:11-68; dispatch_expert_ffn
 * forge/ep/dispatch.py:145-185; spider_expert_grouped_gemm_f32
 * spider_kernels.h:89-92): msg [N,H] in ffn dtype (f32 for f32 experts,
 * bf16 otherwise), idx i32 / w f32 [N,K] -> delta [N,H] in out_dtype
 * (SMOE_F32 or SMOE_BF16).  1 <= K <= 64. */
SMOE_API size_t smoe_expert_delta_workspace_bytes(const smoe_experts* ex, int N, int K);
SMOE_API int smoe_expert_delta(const smoe_experts* ex, const void* msg, const int32_t* idx,
                               const float* w, int N, int K, void* delta, int out_dtype,
                               void* workspace, size_t workspace_bytes, void* stream);

/* Edge generator and per-source top-m (model.py:261-266) for the K selected
 * sources of each token: x [N,H] act_dtype, edge_gen_w [E*E, ldw] act_dtype
 * (its first H columns; ldw = H + L for the reference's [h; e_loop] input,
 * ldw % 8 == 0), edge_bias f32 [E*E] = the loop's row of
 * smoe_edge_loop_bias (b_g plus the loop-embedding half), src_idx i32
 * [N,K] (a source listed twice is one source; ids outside [0, E): none)
 * -> out_eidx i32 [N,K,M] (destinations by descending logit, ties to the
 * lower index) and out_ew f32 [N,K,M] (their softmax weights), slot for
 * slot with src_idx; -1 / 0 for slots without a source.  The same
 * kernels as smoe_block_forward's stages 3-5. */
SMOE_API size_t smoe_edge_topm_workspace_bytes(int N, int K, int E, int M);
SMOE_API int smoe_edge_topm(const void* x, int act_dtype, int N, int H, const void* edge_gen_w,
                            int ldw, const float* edge_bias, int E, int K, int M,
                            const int32_t* src_idx, int32_t* out_eidx, float* out_ew,
                            void* workspace, size_t workspace_bytes, void* stream);

/* Destination projections and message aggregation (model.py:271-288):
 * msg[t] = sum over the token's distinct sources s in src_idx [N,K] and
 * their edges j < M of ew[t,s,j] * edge_value_w[eidx[t,s,j]] x[t], with
 * the weights of each destination added first (in ascending source order)
 * so each (token, destination) projection is computed once.  x [N,H] and
 * edge_value_w [E,H,H] act_dtype (edge_value_w_tiles: optional bf16 copy in
 * the weight tile layout, or NULL), eidx i32 / ew f32 [N,K,M] as
 * smoe_edge_topm writes them -> msg [N,H] in msg_dtype (SMOE_F32 or
 * SMOE_BF16).  The same kernels as smoe_block_forward's stages 6-8. */
SMOE_API size_t smoe_edge_message_workspace_bytes(int N, int H, int E, int K, int M,
                                                  int act_dtype);
SMOE_API int smoe_edge_message(const void* x, int act_dtype, int N, int H,
                               const void* edge_value_w, const void* edge_value_w_tiles, int E,
                               int K, int M, const int32_t* src_idx, const int32_t* eidx,
                               const float* ew, void* msg, int msg_dtype, void* workspace,
                               size_t workspace_bytes, void* stream);

/* Residual, re-injection and LayerNorm (model.py:317):
 * out = LayerNorm(h + alpha * delta + beta * x0) over H (eps; ln_w / ln_b
 * f32 [H] or NULL for 1 / 0).  h, x0, out [N,H] act_dtype; delta [N,H] in
 * delta_dtype (SMOE_F32 or SMOE_BF16).  No workspace. */
SMOE_API int smoe_combine_epilogue(const void* h, const void* x0, int act_dtype,
                                   const void* delta, int delta_dtype, int N, int H, float alpha,
                                   float beta, const float* ln_w, const float* ln_b, float eps,
                                   void* out, void* stream);

/* ---- Forge surfaces (spider_infer/forge) on the same kernels ---- */

/* Top-k selection over f32 logits [N,E] (1 <= K <= min(E, 64), E <= 256) -> top_w f32
 * [N,K], top_idx i32 [N,K], descending.
 *   SMOE_SELECT_ROUTER: the block's router (model.py:256-258): softmax over
 *     the E logits, top-k, weights renormalised by max(sum, 1e-9);
 *   SMOE_SELECT_TOPK_SOFTMAX: ForgeSelect.route (forge/select/api.py:28-40):
 *     top-k on the logits, softmax over the k values.
 * Ties go to the lower index.  No workspace. */
#define SMOE_SELECT_ROUTER 0
#define SMOE_SELECT_TOPK_SOFTMAX 1
SMOE_API int smoe_select_topk(const float* logits, int N, int E, int K, int mode, float* top_w,
                              int32_t* top_idx, void* stream);

/* out [N, N_out] = act(x [N,K] . W^T * scale + bias): ForgeGEMM.linear /
 * linear_fp8 / the two halves of expert_ffn (forge/gemm/api.py:34-58,
 * fp8.py:22-78, triton_kernels.py:65-123) on the block's GEMM kernels.
 * x: f32 (w_format SMOE_F32) or bf16 (SMOE_BF16, SMOE_FP8_E4M3); W
 * [N_out, K] row-major (e4m3 codes for SMOE_FP8_E4M3, whose scale f32
 * [N_out] is required: a per-tensor scale is that value in every entry);
 * bias f32 [N_out] or NULL; act SMOE_LINEAR_NONE (out f32) or
 * SMOE_LINEAR_GELU (erf GELU; out f32 or bf16).  Any K (fp8: K % 32 == 0). */
#define SMOE_LINEAR_NONE 0
#define SMOE_LINEAR_GELU 1
SMOE_API int smoe_linear(const void* x, int N, int K, const void* w, int w_format,
                         const float* w_scale, const float* bias, int N_out, int act, void* out,
                         int out_dtype, void* stream);

/* e4m3 quantization on the device: per tensor, the activation side of
 * fp8_linear(quantize_input=True) (forge/gemm/fp8.py:49-52; quantize_fp8 /
 * compute_fp8_scale, spider_moe/quant.py:30-56) and its weights, or per row
 * (per_row = 1: the per-output-channel scales of the block's fp8 experts,
 * quant.py:146-169 with a row amax): scale = max(amax|x| / 448, 1e-12) in f32
 * (a NaN in x gives a NaN scale), codes = e4m3fn(x / scale) rounded to
 * nearest even, not saturating (|x / scale| > 464 -> NaN code).  Both
 * divisions are IEEE, so the codes and scales are the bits torch gives on the
 * CPU (torch's GPU kernels divide by a reciprocal, which moves the scale by
 * an ulp and, rarely, a code by one step).  x [rows, cols] contiguous, f32 /
 * bf16 / f16 -> codes [rows, ld_out] (ld_out >= cols, ld_out % 4 == 0;
 * columns cols .. ld_out-1 get code 0) and scale f32 [1] or [rows] (device).
 * Per tensor, the workspace (smoe_quantize_fp8_workspace_bytes) holds
 * partial maxima; per row it is unused (may be NULL). */
SMOE_API size_t smoe_quantize_fp8_workspace_bytes(void);
SMOE_API int smoe_quantize_fp8_tensor(const void* x, int x_dtype, int rows, int cols, int ld_out,
                                      int per_row, uint8_t* codes, float* scale, void* workspace,
                                      size_t workspace_bytes, void* stream);

/* out [N, N_out] = act(x_scale * w_scale * (xq [N,K] . wq^T) + bias) with
 * both operands e4m3fn codes (per-tensor scales: device f32 [1] each):
 * the fp8 x fp8 GEMM of fp8_linear(quantize_input=True)
 * (forge/gemm/fp8.py:22-62), which the reference runs as a dequantize +
 * F.linear.  v_mfma_f32_16x16x128_f8f6f4 multiplies the codes exactly and
 * sums each block of 128 products below f32 precision (measured: within
 * 2^-14 of the block's largest product), the blocks in f32; the scales and
 * bias are applied in f32.
 * K % 256 == 0 (pad both operands' rows with code 0: smoe_quantize_fp8_tensor
 * with ld_out = K); bias f32 [N_out] or NULL; act SMOE_LINEAR_NONE / GELU
 * (erf); out f32 or bf16, row-major [N, N_out]. */
SMOE_API int smoe_linear_fp8fp8(const uint8_t* xq, const float* x_scale, int N, int K,
                                const uint8_t* wq, const float* w_scale, const float* bias,
                                int N_out, int act, void* out, int out_dtype, void* stream);

/* out [N,H] = per token, the sum over its rows tok_row [N,K] (-1: none;
 * distinct rows, added in ascending row order) of y [R,H] times row_w [R]
 * (NULL: 1; cast to y's dtype first), each product rounded to y's dtype and
 * each partial sum to out's (SMOE_F32 / SMOE_BF16): the combine of
 * dispatch_expert_ffn (forge/ep/dispatch.py:127-134, 176-180), a
 * scatter-add of weighted expert outputs in ascending expert order (plan
 * rows are grouped by ascending expert). */
SMOE_API int smoe_combine_rows(const void* y, int y_dtype, const float* row_w,
                               const int32_t* tok_row, int N, int K, int H, void* out,
                               int out_dtype, void* stream);

/* ---- Dobu expert residency (spider_moe/expert_store.py:121-166) ----
 * out[i] = map[ids[i]] for ids in [0, E), else -1: routed expert ids ->
 * slots of the device-resident expert slab (map[e] = -1 for experts not in
 * the slab), so smoe_expert_delta runs over the slab as E' = slot count
 * experts.  n >= 0; no workspace. */
SMOE_API int smoe_remap_ids(const int32_t* ids, int64_t n, const int32_t* map, int E,
                            int32_t* out, void* stream);

/* ---- diagnostics (no counterpart in the reference; used by bench.py) ----
 * Stage ids of smoe_block_forward, in launch order within a loop. */
#define SMOE_STAGE_ROUTER_GEMM 0
#define SMOE_STAGE_ROUTE_TOPK 1
#define SMOE_STAGE_EXPERT_PLAN 2
#define SMOE_STAGE_EDGE_LOGITS 3
#define SMOE_STAGE_EDGE_TOPM 4
#define SMOE_STAGE_DEST_PLAN 5
#define SMOE_STAGE_EDGE_GEMM 6
#define SMOE_STAGE_MSG_COMBINE 7
#define SMOE_STAGE_UP_GEMM 8
#define SMOE_STAGE_DOWN_GEMM 9
#define SMOE_STAGE_EPILOGUE 10
/* bf16 steps of N <= 64 run stages 0-5 as these two launches; decode loops
 * (H <= 1024) as FRONT_GEMM alone (k_decode_front), their plans running
 * inside the EDGE_GEMM launch */
#define SMOE_STAGE_FRONT_GEMM 11  /* router + all edge-generator logits, one GEMM */
#define SMOE_STAGE_FRONT_ROUTE 12 /* top-k, expert plan, top-m, destination plan */
#define SMOE_NUM_STAGES 13

/* Weight tile layout of weights w [G,N,K] (format SMOE_BF16 or
 * SMOE_FP8_E4M3 codes; N % 16 == 0, K % 64 == 0), same size.  Rows are cut
 * into 64-byte pieces; for group g, 16-row tile t, piece c and lane
 * l = 16q + r, the 16 bytes j at
 *   out_bytes[(((g*(N/16) + t)*C + c)*64 + l)*16 + j]
 *     = row_bytes(w[g][16t + r])[64c + 16q + j],      C = K x elt size / 64.
 * In elements, bf16:  out[((((g*(N/16) + t)*(K/64) + s)*2 + h)*64 + l)*8 + e]
 *                       = w[g][16t + r][64s + 32h + 8q + e];
 *              fp8:   out[(((g*(N/16) + t)*(K/64) + s)*64 + l)*16 + e]
 *                       = w[g][16t + r][64s + 16q + e].
 * Each 16-row x 64-byte block is 1 KB holding, lane by lane, the 16-byte
 * MFMA fragments a wave loads, and a tile's blocks follow one another along
 * K.  The decode weight stream reads a block with one contiguous 1 KB load
 * instead of sixteen 64-byte row pieces a row pitch apart, and the
 * ping-pong GEMM copies bf16 blocks into LDS as they are (its fragment
 * reads need no swizzle).  Measured (bf16): C2 0.390 -> 0.377 ms per step,
 * C1 5.25 -> 5.09, C3 4.00 -> 3.93, C4 1.90 -> 1.80 (C4's 537 MB edge
 * projection 178 -> 156 us).  No counterpart in the reference (its weights
 * stay nn.Linear row-major); the row-major weights remain the format every
 * other kernel reads.  Returns -2 for other formats. */
SMOE_API int smoe_pack_weight_tiles(const void* w, int format, int G, int N, int K, void* out,
                                    void* stream);

/* int4 weights (packed [G,N,K/2] as quant.py:119-143 packs them: element
 * 2i in the low nibble of byte i) -> the same bytes in the int4 tile layout
 * the ping-pong GEMM reads, out [G*N*K/2] bytes: per group, 64-row quad Q
 * and 32-k stage st, a 1 KB block at ((g*N/64 + Q)*K/32 + st)*1024 of four
 * 16-row tiles (256 B each), lane l of tile t holding the 4 bytes of row
 * 64Q + 16t + l%16 with k = 32st + 8(l/16) .. +7.  For the smoe_experts
 * w_up_tiles / w_down_tiles of int4 experts: prefill-size expert GEMMs
 * (>= 256 rows per expert, N_out % 256 == 0, 32 | group_size, K/group_size
 * <= 32) then run on the ping-pong kernel, which widens the nibbles to bf16
 * (q * s) in registers, with no memory beyond the int4 bytes.  N % 64,
 * K % 32.  No counterpart in the reference (it dequantizes per call,
 * model.py:299-303). */
SMOE_API int smoe_pack_int4_qtiles(const void* packed, int G, int N, int K, void* out,
                                   void* stream);

/* When `events` is not NULL, every later smoe_block_forward records
 * events[2*i] before and events[2*i+1] after the i-th launch of a stage in
 * `stage_mask` (bit s = stage s), for i < capacity, on the call's stream.
 * The setting belongs to the calling thread: it arms that thread's later
 * calls only, and each thread counts its own pairs.  Pass NULL to stop.
 * smoe_profile_count returns how many pairs this thread recorded and resets
 * its counter; stage_of[i] (may be NULL) receives the stage of pair i. */
SMOE_API int smoe_profile_stages(uint32_t stage_mask, void** events, int capacity);
/* When `counters` (device memory, 2 x uint64, zeroed by the caller) is not
 * NULL, every profiled launch of a single-GEMM stage that runs on the
 * 256-column ping-pong GEMM adds its workgroups' shader-clock cycles to
 * counters[0] and their 100 MHz wall-clock ticks to counters[1]:
 * counters[0] / counters[1] * 100 is the MHz those tiles ran at.  Per
 * calling thread; NULL stops it.  Diagnostics; no counterpart in the
 * reference. */
SMOE_API int smoe_profile_clock(void* counters);
SMOE_API int smoe_profile_count(int32_t* stage_of, int capacity);
/* hipEvent helpers for callers without a HIP binding. */
SMOE_API int smoe_events_create(int n, void** events);
SMOE_API int smoe_events_destroy(int n, void** events);
/* ms[i] = elapsed time between events[2*i] and events[2*i+1] (synchronizes). */
SMOE_API int smoe_events_elapsed(int pairs, void** events, float* ms);

#ifdef __cplusplus
}
#endif
