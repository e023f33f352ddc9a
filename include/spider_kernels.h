/*
 * spider_kernels.h — the reference's host C ABI for the torch-free loop
 * (kernels/include/spider_kernels.h:26-121, the MoE-loop entries), exported
 * by libsmoe.so and computed on the GPU.
 *
 * Same names, argument lists, layouts and return codes as the reference's
 * CPU library (its scalar implementation, kernels/scalar/scalar.cpp and
 * scalar_phase1_{1,2,3}.cpp, behind kernels/src/dispatch.cpp), so the
 * reference's ctypes binding (kernels/python/spider_native.py) and
 * native_backend.py's loop call it unchanged: all pointers are HOST
 * pointers; each call copies its inputs to the current HIP device, runs the
 * spider_cuda_* kernels of include/spider_cuda.h on a stream of its own,
 * copies the outputs back and returns when they are in place.
 *
 * Return codes: 0 ok; 1 invalid arguments (null pointers, sizes, a CSR
 * whose row_ptr[0] != 0 or row_ptr[E] != nnz) or beyond this build's
 * limits; 2 a selected source or an edge destination outside [0, E) (as the
 * scalar library reports them; checked before any device work, here over
 * every edge of a selected source); 3 a HIP error (device memory, launch);
 * -2 for the f16 entries, which the reference's library stubs out the same
 * way (kernels/src/phase1_api_ext.cpp:4-15).
 *
 * Numerics follow the scalar library operation by operation: float sums in
 * its order, double sums where it uses double (router logits of the loop
 * step, edge projection, edge generator, LayerNorm statistics, exit dot);
 * exp / tanh come from the device's math library, so router and edge
 * weights and the GELU differ from the CPU's in the last bits.
 * Limits: E <= 256 (router, edge top-m), E <= 64 in the loop step,
 * H <= 8192 for the expert FFN and the epilogue.  The staging buffer of a
 * device is reused across calls (grown on demand); calls on one device are
 * serialised.
 */
#pragma once
#include <stddef.h>
#include <stdint.h>

#if defined(_WIN32)
#define SPIDER_API __declspec(dllexport)
#else
#define SPIDER_API __attribute__((visibility("default")))
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* spider_kernels.h:26-28, scalar.cpp:7-34 */
SPIDER_API int spider_router_f32(const float* logits, const float* loop_bias, int B, int E, int K,
                                 int loop_idx, float* out_weights, int32_t* out_indices);
/* spider_kernels.h:30-32 (stub in the reference: -2) */
SPIDER_API int spider_router_f16(const uint16_t* logits, const uint16_t* loop_bias, int B, int E,
                                 int K, int loop_idx, float* out_weights, int32_t* out_indices);

/* spider_kernels.h:34-39, scalar.cpp:36-53 (static CSR, route-weighted) */
SPIDER_API int spider_graph_message_passing_f32(const float* hidden, int B, int H, int E, int K,
                                                const int32_t* adj_row_ptr,
                                                const int32_t* adj_col_idx,
                                                const float* edge_weights, int nnz, int loop_idx,
                                                const int32_t* expert_assign,
                                                const float* route_weights, float* messages);
/* spider_kernels.h:41-46 (stub in the reference: -2) */
SPIDER_API int spider_graph_message_passing_f16(const uint16_t* hidden, int B, int H, int E, int K,
                                                const int32_t* adj_row_ptr,
                                                const int32_t* adj_col_idx,
                                                const float* edge_weights, int nnz, int loop_idx,
                                                const int32_t* expert_assign,
                                                const float* route_weights, float* messages);

/* spider_kernels.h:48-50, scalar_phase1_1.cpp:17-32 */
SPIDER_API int spider_edge_project_f32(const float* hidden, int B, int H, int E,
                                       const float* W_edge, float* out_proj);
/* spider_kernels.h:52-56, scalar_phase1_1.cpp:34-60 */
SPIDER_API int spider_graph_message_passing_v2_f32(const float* projected, int B, int H, int E,
                                                   int K, const int32_t* row_ptr,
                                                   const int32_t* col_idx,
                                                   const float* edge_weights, int nnz,
                                                   int loop_idx, const int32_t* assign,
                                                   float* messages);
/* spider_kernels.h:58-60, scalar_phase1_2.cpp:11-47 */
SPIDER_API int spider_edge_topk_f32(const float* edge_logits, int B, int E, int M,
                                    int32_t* edge_indices, float* edge_weights);
/* spider_kernels.h:62-65, scalar_phase1_2.cpp:49-72 */
SPIDER_API int spider_graph_message_passing_dynamic_f32(const float* projected, int B, int H,
                                                        int E, int K, int M,
                                                        const int32_t* edge_indices,
                                                        const float* edge_weights,
                                                        const int32_t* assign, float* messages);
/* spider_kernels.h:67-71, scalar_phase1_2.cpp:74-86 */
SPIDER_API int spider_graph_dynamic_with_edge_value_f32(const float* hidden, int B, int H, int E,
                                                        int K, int M, const float* W_edge,
                                                        const int32_t* edge_indices,
                                                        const float* edge_weights,
                                                        const int32_t* assign, float* messages,
                                                        float* tmp_projected);
/* spider_kernels.h:73-76, scalar_phase1_3.cpp:14-42 */
SPIDER_API int spider_edge_generator_f32(const float* hidden, int B, int H, int E,
                                         const float* loop_emb, int loop_emb_dim,
                                         const float* W_gen, float* out_logits);
/* spider_kernels.h:78-81, scalar_phase1_3.cpp:44-52 */
SPIDER_API int spider_edge_generator_topk_f32(const float* hidden, int B, int H, int E, int M,
                                              const float* loop_emb, int loop_emb_dim,
                                              const float* W_gen, int32_t* edge_indices,
                                              float* edge_weights, float* tmp_logits);
/* spider_kernels.h:83-87, scalar_phase1_3.cpp:54-70 */
SPIDER_API int spider_graph_from_generator_f32(const float* hidden, int B, int H, int E, int K,
                                               int M, const float* loop_emb, int loop_emb_dim,
                                               const float* W_gen, const float* W_edge,
                                               const int32_t* assign, float* messages,
                                               float* tmp_logits, int32_t* tmp_edge_idx,
                                               float* tmp_edge_w, float* tmp_projected);

/* spider_kernels.h:89-92, scalar.cpp:55-73 (tanh-GELU, no biases) */
SPIDER_API int spider_expert_grouped_gemm_f32(const float* tokens, int B, int H, int H_up, int E,
                                              int K, const int32_t* expert_assign,
                                              const float* route_weights, const float* W_up,
                                              const float* W_down, float* output);
/* spider_kernels.h:94-97 (stub in the reference: -2) */
SPIDER_API int spider_expert_grouped_gemm_f16(const float* tokens, int B, int H, int H_up, int E,
                                              int K, const int32_t* expert_assign,
                                              const float* route_weights, const uint16_t* W_up,
                                              const uint16_t* W_down, float* output);

/* spider_kernels.h:99-102, scalar.cpp:75-92 */
SPIDER_API int spider_loop_epilogue_f32(const float* h, const float* delta,
                                        const float* input_embed, int B, int H, float alpha,
                                        float beta, const float* ln_weight, const float* ln_bias,
                                        float eps, float* h_next);
/* spider_kernels.h:104-107 (stub in the reference: -2) */
SPIDER_API int spider_loop_epilogue_f16(const float* h, const float* delta,
                                        const float* input_embed, int B, int H, float alpha,
                                        float beta, const float* ln_weight, const float* ln_bias,
                                        float eps, float* h_next);

/* spider_kernels.h:109-111, scalar.cpp:94-104 */
SPIDER_API int spider_early_exit_f32(const float* h, const float* exit_proj, int B, int H,
                                     float threshold, uint8_t* should_exit);

/* spider_kernels.h:113-121, scalar_phase1_1.cpp:62-121: router on
 * h . router_w, messages = the projected CSR pass when W_edge and the CSR
 * are given (else h), tanh-GELU experts, epilogue, exit mask */
SPIDER_API int spider_moe_loop_step_f32(
    const float* h, const float* x0, int B, int H, int E, int K, int U, int loop_idx,
    const float* router_w, const float* loop_bias, const int32_t* row_ptr,
    const int32_t* col_idx, const float* edge_w, int nnz, const float* W_edge,
    const float* W_up, const float* W_down, const float* ln_weight, const float* ln_bias,
    float alpha, float beta, float eps, const float* exit_proj, float exit_threshold,
    float* h_next, uint8_t* exit_mask, int32_t* tmp_assign, float* tmp_route,
    float* tmp_messages);

/* spider_kernels.h:148-149: "hip-gfx950"; caps bit 0 f32, bit 1 device */
SPIDER_API const char* spider_backend_name(void);
SPIDER_API uint32_t spider_backend_caps(void);

#ifdef __cplusplus
}
#endif
