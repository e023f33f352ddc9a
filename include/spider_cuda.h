/*
 * spider_cuda.h — the reference's device ABI for the torch-free loop,
 * exported by libsmoe.so over gfx950 HIP kernels.
 *
 * The names, argument lists and semantics follow the reference's CUDA
 * header kernels/include/spider_cuda.h:8-44 and its kernels
 * kernels/cuda/spider_kernels.cu:8-117 and spider_expert_v2.cu:13-85, so a
 * caller written for that header (spider_infer/orbit/native_backend.py's
 * loop, kernels/python/spider_native.py's bindings) links against
 * libsmoe.so unchanged.  These are the reference's fp32 "native" semantics,
 * which differ from the PyTorch block's (include/smoe.h):
 *   - router logits are given (or, in the loop step, h . router_w with
 *     router_w [H, E]); top-k over the softmax probabilities, lowest index
 *     on ties, renormalised by max(sum, 1e-20);
 *   - the message pass is the static CSR graph of the reference (v1: each
 *     edge of a selected source adds edge_w * route_w * h; col_idx unused);
 *   - the expert FFN is tanh-GELU with no biases, W_up [E, H, U] and
 *     W_down [E, U, H] (input-major);
 *   - the epilogue is LayerNorm(h + alpha d + beta x0) with double-precision
 *     statistics (the reference's Welford pass);
 *   - exit: sigmoid(h . exit_proj) > threshold, one byte per row.
 * All pointers are device pointers; every call enqueues on `stream` (a
 * hipStream_t passed as void*) and returns 0, 1 for invalid arguments, or
 * the HIP error code.  Results are deterministic: every sum runs in a fixed
 * order (no atomics), unlike the reference's atomicAdd down projection.
 * Limits of this build: E <= 256 for the router (E <= 64 in the loop
 * step); H <= 8192 and U <= 16384 for the expert FFN (H + U <= 16384
 * without a workspace).  The workspace of spider_cuda_expert_grouped_gemm_v2_f32
 * holds the hidden activations [B, K, U] as in the reference.
 */
#pragma once
#include <stddef.h>
#include <stdint.h>

#if defined(_WIN32)
#define SPIDER_CUDA_API __declspec(dllexport)
#else
#define SPIDER_CUDA_API __attribute__((visibility("default")))
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* logits [B,E] + loop_bias[loop_idx] ([R,E]) -> out_w [B,K], out_idx [B,K]
 * (spider_cuda.h:8-9, spider_kernels.cu:8-26) */
SPIDER_CUDA_API int spider_cuda_router_f32(const float* logits, const float* loop_bias, int B,
                                           int E, int K, int loop_idx, float* out_w,
                                           int32_t* out_idx, void* stream);

/* messages[b] = h[b] * sum over slots k with a valid source s = assign[b,k]
 * and edges e in [row_ptr[s], row_ptr[s+1]) (e < nnz) of
 * edge_w[loop_idx * nnz + e] * route_w[b,k]   (spider_cuda.h:11-14,
 * spider_kernels.cu:28-40) */
SPIDER_CUDA_API int spider_cuda_graph_message_passing_f32(
    const float* h, int B, int H, int E, int K, const int32_t* row_ptr, const int32_t* col_idx,
    const float* edge_w, int nnz, int loop_idx, const int32_t* assign, const float* route_w,
    float* messages, void* stream);

/* out[b] = sum_k route_w[b,k] * W_down[e] . gelu_tanh(W_up[e] . x[b]),
 * e = assign[b,k] (slots with e outside [0, E) skipped)  (spider_cuda.h:16-18,
 * spider_kernels.cu:42-60) */
SPIDER_CUDA_API int spider_cuda_expert_grouped_gemm_f32(const float* x, int B, int H, int U,
                                                        int E, int K, const int32_t* assign,
                                                        const float* route_w, const float* W_up,
                                                        const float* W_down, float* out,
                                                        void* stream);

/* B * K * U * 4 bytes (spider_cuda.h:20, spider_expert_v2.cu:61-64) */
SPIDER_CUDA_API size_t spider_cuda_expert_workspace_bytes(int B, int K, int U);

/* the same FFN with the hidden activations in `workspace` [B,K,U]
 * (spider_cuda.h:22-26, spider_expert_v2.cu:66-85) */
SPIDER_CUDA_API int spider_cuda_expert_grouped_gemm_v2_f32(
    const float* x, int B, int H, int U, int E, int K, const int32_t* assign,
    const float* route_w, const float* W_up, const float* W_down, float* out, float* workspace,
    void* stream);

/* out = LayerNorm(h + alpha d + beta x0) with gamma / beta_ln [H]
 * (spider_cuda.h:28-30, spider_kernels.cu:62-82) */
SPIDER_CUDA_API int spider_cuda_loop_epilogue_f32(const float* h, const float* d,
                                                  const float* x0, int B, int H, float alpha,
                                                  float beta, const float* gamma,
                                                  const float* beta_ln, float eps, float* out,
                                                  void* stream);

/* mask[b] = sigmoid(h[b] . proj) > threshold  (spider_cuda.h:32-33,
 * spider_kernels.cu:84-88) */
SPIDER_CUDA_API int spider_cuda_early_exit_f32(const float* h, const float* proj, int B, int H,
                                               float threshold, uint8_t* mask, void* stream);

/* One loop of the torch-free block, declared by the reference
 * (spider_cuda.h:35-44) without a definition; composed here as the
 * reference's scalar step (scalar_phase1_1.cpp:62-121) with the device
 * ABI's static graph: logits = h . router_w ([H,E]), router (loop_bias
 * [R,E]) -> tmp_assign / tmp_route [B,K]; messages (tmp_messages [B,H]) =
 * the CSR message pass when row_ptr, col_idx and edge_w are given, else h;
 * h_next = epilogue(h, expert FFN(messages), x0); exit_mask [B] (or NULL)
 * from exit_proj [H] (NULL: all zero). */
SPIDER_CUDA_API int spider_cuda_moe_loop_step_f32(
    const float* h, const float* x0, int B, int H, int E, int K, int U, int loop_idx,
    const float* router_w, const float* loop_bias, const int32_t* row_ptr,
    const int32_t* col_idx, const float* edge_w, int nnz, const float* W_up,
    const float* W_down, const float* ln_weight, const float* ln_bias, float alpha, float beta,
    float eps, const float* exit_proj, float exit_threshold, float* h_next, uint8_t* exit_mask,
    int32_t* tmp_assign, float* tmp_route, float* tmp_messages, void* stream);

/* ---- Device-pointer forms of the reference's dynamic-edge host functions
 * (kernels/include/spider_kernels.h:48-86).  The reference's CUDA header
 * has no counterpart; these carry the scalar library's semantics
 * (scalar_phase1_1.cpp:17-60, scalar_phase1_2.cpp:11-72,
 * scalar_phase1_3.cpp:14-42) for the host entry points of spider_kernels.h
 * and for GPU callers.  Sources or destinations outside [0, E) are skipped
 * here; the host entry points reject them first. */

/* out_proj [B,E,H]: out_proj[b,e,j] = sum_i h[b,i] W_edge[e][j][i], double
 * sums in i order (W_edge [E,H,H]) */
SPIDER_CUDA_API int spider_cuda_edge_project_f32(const float* h, int B, int H, int E,
                                                 const float* W_edge, float* out_proj,
                                                 void* stream);

/* messages [B,H] = sum over selected sources (assign [B,K]) and their CSR
 * edges of edge_w[loop_idx * nnz + edge] * projected[b, col_idx[edge], :] */
SPIDER_CUDA_API int spider_cuda_graph_message_passing_v2_f32(
    const float* projected, int B, int H, int E, int K, const int32_t* row_ptr,
    const int32_t* col_idx, const float* edge_w, int nnz, int loop_idx, const int32_t* assign,
    float* messages, void* stream);

/* edge_logits [B,E,E] -> per (b, src) row the M largest (first index on
 * ties; no candidate left: index -1) and a softmax over them:
 * edge_idx [B,E,M], edge_w [B,E,M]; E <= 256 */
SPIDER_CUDA_API int spider_cuda_edge_topk_f32(const float* edge_logits, int B, int E, int M,
                                              int32_t* edge_idx, float* edge_w, void* stream);

/* messages [B,H] = sum over selected sources and their M picks of
 * edge_w[b,src,m] * projected[b, edge_idx[b,src,m], :] */
SPIDER_CUDA_API int spider_cuda_graph_message_passing_dynamic_f32(
    const float* projected, int B, int H, int E, int K, int M, const int32_t* edge_idx,
    const float* edge_w, const int32_t* assign, float* messages, void* stream);

/* out_logits [B,E*E] = [h, loop_emb] . W_gen^T (W_gen [E*E, H + D]),
 * double sums in input order, no bias */
SPIDER_CUDA_API int spider_cuda_edge_generator_f32(const float* h, int B, int H, int E,
                                                   const float* loop_emb, int loop_emb_dim,
                                                   const float* W_gen, float* out_logits,
                                                   void* stream);

#ifdef __cplusplus
}
#endif
