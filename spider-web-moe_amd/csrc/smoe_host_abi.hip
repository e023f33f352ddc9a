// The reference's host C ABI (include/spider_kernels.h) on the GPU: each
// entry point checks its arguments as the reference's scalar library does,
// copies its host inputs into a per-device staging buffer, runs the
// spider_cuda_* kernels (smoe_compat.hip) on the device's staging stream,
// copies the outputs back and synchronises.  No arithmetic happens on the
// host.
#include <hip/hip_runtime.h>

#include <cstring>
#include <mutex>
#include <vector>

#include "smoe_internal.hpp"
#include "spider_cuda.h"
#include "spider_kernels.h"

namespace smoe {
namespace {

constexpr int kMaxDevices = 64;
constexpr int kDeviceError = 3;
constexpr size_t kAlign = 256;

// One device's staging state: a grow-only buffer and a stream of default
// priority, created on first use; the mutex serialises calls on the device.
struct Stage {
  std::mutex mu;
  char* buf = nullptr;
  size_t cap = 0;
  hipStream_t stream = nullptr;
};

Stage& stage_of(int dev) {
  static Stage stages[kMaxDevices];
  return stages[dev];
}

// The buffers of one call: inputs (copied in), outputs (copied back) and
// device-only scratch, each at its own 256-byte aligned offset.
class Staging {
 public:
  int in(const void* host, size_t bytes) { return add(host, nullptr, bytes); }
  int out(void* host, size_t bytes) { return add(nullptr, host, bytes); }
  int tmp(size_t bytes) { return add(nullptr, nullptr, bytes); }

  template <typename T>
  T* dev(int h) const {
    return reinterpret_cast<T*>(base_ + slots_[h].off);
  }
  float* f(int h) const { return dev<float>(h); }
  int32_t* i(int h) const { return dev<int32_t>(h); }

  // Copies in, launch(stream) (its return code: 0 or an error), copies out.
  template <typename F>
  int run(F&& launch) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return kDeviceError;
    Stage& st = stage_of(dev);
    std::lock_guard<std::mutex> lock(st.mu);
    if (!st.stream && hipStreamCreateWithFlags(&st.stream, hipStreamNonBlocking) != hipSuccess) {
      st.stream = nullptr;
      return kDeviceError;
    }
    const size_t need = total_ < kAlign ? kAlign : total_;
    if (need > st.cap) {
      if (st.buf) (void)hipFree(st.buf);
      st.buf = nullptr;
      st.cap = 0;
      if (hipMalloc(reinterpret_cast<void**>(&st.buf), need) != hipSuccess) return kDeviceError;
      st.cap = need;
    }
    base_ = st.buf;
    for (const Slot& s : slots_)
      if (s.src && s.bytes &&
          hipMemcpyAsync(base_ + s.off, s.src, s.bytes, hipMemcpyHostToDevice, st.stream) !=
              hipSuccess)
        return finish(st, kDeviceError);
    const int rc = launch(st.stream);
    if (rc != 0) return finish(st, rc == 1 ? 1 : kDeviceError);
    for (const Slot& s : slots_)
      if (s.dst && s.bytes &&
          hipMemcpyAsync(s.dst, base_ + s.off, s.bytes, hipMemcpyDeviceToHost, st.stream) !=
              hipSuccess)
        return finish(st, kDeviceError);
    return finish(st, 0);
  }

 private:
  struct Slot {
    const void* src;
    void* dst;
    size_t bytes;
    size_t off;
  };
  int add(const void* src, void* dst, size_t bytes) {
    slots_.push_back(Slot{src, dst, bytes, total_});
    total_ += (bytes + kAlign - 1) / kAlign * kAlign;
    if (bytes == 0) total_ += kAlign;  // a distinct, valid address
    return static_cast<int>(slots_.size()) - 1;
  }
  static int finish(Stage& st, int rc) {
    const hipError_t e = hipStreamSynchronize(st.stream);
    if (rc == 0 && e != hipSuccess) return kDeviceError;
    return rc;
  }
  std::vector<Slot> slots_;
  size_t total_ = 0;
  char* base_ = nullptr;
};

size_t fbytes(int64_t n) { return static_cast<size_t>(n) * sizeof(float); }
size_t ibytes(int64_t n) { return static_cast<size_t>(n) * sizeof(int32_t); }

// scalar.cpp:40 / scalar_phase1_1.cpp:39-41: a CSR must start at 0 and end at nnz.
bool csr_ok(const int32_t* rp, int E, int nnz) { return rp[0] == 0 && rp[E] == nnz; }

// The index checks the scalar library makes while it walks the graph
// (scalar.cpp:45-48, scalar_phase1_1.cpp:47-52): 2 for a selected source
// >= E or a destination of its edges outside [0, E); 1 for a row of the
// CSR that points outside [0, nnz) (which the scalar loop would read past).
int check_csr_sources(const int32_t* assign, int B, int K, int E, const int32_t* rp,
                      const int32_t* ci, int nnz) {
  for (int64_t t = 0; t < static_cast<int64_t>(B) * K; ++t) {
    const int src = assign[t];
    if (src < 0) continue;
    if (src >= E) return 2;
    if (rp[src] < 0 || rp[src + 1] > nnz) return 1;
    for (int e = rp[src]; e < rp[src + 1]; ++e)
      if (ci[e] < 0 || ci[e] >= E) return 2;
  }
  return 0;
}

// scalar_phase1_2.cpp:58-66: the same over the picks of each selected source.
int check_dynamic_sources(const int32_t* assign, int B, int K, int E, int M,
                          const int32_t* eidx) {
  for (int b = 0; b < B; ++b)
    for (int k = 0; k < K; ++k) {
      const int src = assign[static_cast<int64_t>(b) * K + k];
      if (src < 0) continue;
      if (src >= E) return 2;
      const int32_t* row = eidx + (static_cast<int64_t>(b) * E + src) * M;
      for (int m = 0; m < M; ++m)
        if (row[m] < 0 || row[m] >= E) return 2;
    }
  return 0;
}

// scalar.cpp:62: an assigned expert >= E is an error, a negative one a gap.
int check_experts(const int32_t* assign, int B, int K, int E) {
  for (int64_t t = 0; t < static_cast<int64_t>(B) * K; ++t)
    if (assign[t] >= E) return 2;
  return 0;
}

}  // namespace
}  // namespace smoe

using namespace smoe;

extern "C" {

SPIDER_API int spider_router_f32(const float* logits, const float* loop_bias, int B, int E, int K,
                                 int loop_idx, float* out_w, int32_t* out_idx) {
  if (!logits || !loop_bias || !out_w || !out_idx || B <= 0 || E <= 0 || K <= 0 || K > E ||
      loop_idx < 0 || E > 256)
    return 1;
  Staging st;
  const int hl = st.in(logits, fbytes(int64_t(B) * E));
  const int hb = st.in(loop_bias + static_cast<int64_t>(loop_idx) * E, fbytes(E));
  const int hw = st.out(out_w, fbytes(int64_t(B) * K));
  const int hi = st.out(out_idx, ibytes(int64_t(B) * K));
  return st.run([&](hipStream_t s) {
    return spider_cuda_router_f32(st.f(hl), st.f(hb), B, E, K, 0, st.f(hw), st.i(hi), s);
  });
}

SPIDER_API int spider_router_f16(const uint16_t*, const uint16_t*, int, int, int, int, float*,
                                 int32_t*) {
  return -2;
}

SPIDER_API int spider_graph_message_passing_f32(const float* hidden, int B, int H, int E, int K,
                                                const int32_t* row_ptr, const int32_t* col_idx,
                                                const float* edge_w, int nnz, int loop_idx,
                                                const int32_t* assign, const float* route_w,
                                                float* messages) {
  if (!hidden || !row_ptr || !col_idx || !edge_w || !assign || !route_w || !messages || B <= 0 ||
      H <= 0 || E <= 0 || K <= 0 || nnz < 0 || loop_idx < 0 || !csr_ok(row_ptr, E, nnz))
    return 1;
  const int bad = check_csr_sources(assign, B, K, E, row_ptr, col_idx, nnz);
  if (bad) return bad;
  Staging st;
  const int hh = st.in(hidden, fbytes(int64_t(B) * H));
  const int hr = st.in(row_ptr, ibytes(E + 1));
  const int hc = st.in(col_idx, ibytes(nnz));
  const int he = st.in(edge_w + static_cast<int64_t>(loop_idx) * nnz, fbytes(nnz));
  const int ha = st.in(assign, ibytes(int64_t(B) * K));
  const int hw = st.in(route_w, fbytes(int64_t(B) * K));
  const int hm = st.out(messages, fbytes(int64_t(B) * H));
  return st.run([&](hipStream_t s) {
    return spider_cuda_graph_message_passing_f32(st.f(hh), B, H, E, K, st.i(hr), st.i(hc),
                                                 st.f(he), nnz, 0, st.i(ha), st.f(hw), st.f(hm),
                                                 s);
  });
}

SPIDER_API int spider_graph_message_passing_f16(const uint16_t*, int, int, int, int,
                                                const int32_t*, const int32_t*, const float*, int,
                                                int, const int32_t*, const float*, float*) {
  return -2;
}

SPIDER_API int spider_edge_project_f32(const float* hidden, int B, int H, int E,
                                       const float* W_edge, float* out_proj) {
  if (!hidden || !W_edge || !out_proj || B <= 0 || H <= 0 || E <= 0) return 1;
  Staging st;
  const int hh = st.in(hidden, fbytes(int64_t(B) * H));
  const int hw = st.in(W_edge, fbytes(int64_t(E) * H * H));
  const int ho = st.out(out_proj, fbytes(int64_t(B) * E * H));
  return st.run([&](hipStream_t s) {
    return spider_cuda_edge_project_f32(st.f(hh), B, H, E, st.f(hw), st.f(ho), s);
  });
}

SPIDER_API int spider_graph_message_passing_v2_f32(const float* projected, int B, int H, int E,
                                                   int K, const int32_t* row_ptr,
                                                   const int32_t* col_idx, const float* edge_w,
                                                   int nnz, int loop_idx, const int32_t* assign,
                                                   float* messages) {
  if (!projected || !row_ptr || !col_idx || !edge_w || !assign || !messages || B <= 0 || H <= 0 ||
      E <= 0 || K <= 0 || nnz < 0 || loop_idx < 0 || !csr_ok(row_ptr, E, nnz))
    return 1;
  const int bad = check_csr_sources(assign, B, K, E, row_ptr, col_idx, nnz);
  if (bad) return bad;
  Staging st;
  const int hp = st.in(projected, fbytes(int64_t(B) * E * H));
  const int hr = st.in(row_ptr, ibytes(E + 1));
  const int hc = st.in(col_idx, ibytes(nnz));
  const int he = st.in(edge_w + static_cast<int64_t>(loop_idx) * nnz, fbytes(nnz));
  const int ha = st.in(assign, ibytes(int64_t(B) * K));
  const int hm = st.out(messages, fbytes(int64_t(B) * H));
  return st.run([&](hipStream_t s) {
    return spider_cuda_graph_message_passing_v2_f32(st.f(hp), B, H, E, K, st.i(hr), st.i(hc),
                                                    st.f(he), nnz, 0, st.i(ha), st.f(hm), s);
  });
}

SPIDER_API int spider_edge_topk_f32(const float* edge_logits, int B, int E, int M,
                                    int32_t* edge_idx, float* edge_w) {
  if (!edge_logits || !edge_idx || !edge_w || B <= 0 || E <= 0 || M <= 0 || M > E || E > 256)
    return 1;
  Staging st;
  const int hl = st.in(edge_logits, fbytes(int64_t(B) * E * E));
  const int hi = st.out(edge_idx, ibytes(int64_t(B) * E * M));
  const int hw = st.out(edge_w, fbytes(int64_t(B) * E * M));
  return st.run([&](hipStream_t s) {
    return spider_cuda_edge_topk_f32(st.f(hl), B, E, M, st.i(hi), st.f(hw), s);
  });
}

SPIDER_API int spider_graph_message_passing_dynamic_f32(const float* projected, int B, int H,
                                                        int E, int K, int M,
                                                        const int32_t* edge_idx,
                                                        const float* edge_w,
                                                        const int32_t* assign, float* messages) {
  if (!projected || !edge_idx || !edge_w || !assign || !messages || B <= 0 || H <= 0 || E <= 0 ||
      K <= 0 || M <= 0)
    return 1;
  const int bad = check_dynamic_sources(assign, B, K, E, M, edge_idx);
  if (bad) return bad;
  Staging st;
  const int hp = st.in(projected, fbytes(int64_t(B) * E * H));
  const int hi = st.in(edge_idx, ibytes(int64_t(B) * E * M));
  const int hw = st.in(edge_w, fbytes(int64_t(B) * E * M));
  const int ha = st.in(assign, ibytes(int64_t(B) * K));
  const int hm = st.out(messages, fbytes(int64_t(B) * H));
  return st.run([&](hipStream_t s) {
    return spider_cuda_graph_message_passing_dynamic_f32(st.f(hp), B, H, E, K, M, st.i(hi),
                                                         st.f(hw), st.i(ha), st.f(hm), s);
  });
}

SPIDER_API int spider_graph_dynamic_with_edge_value_f32(const float* hidden, int B, int H, int E,
                                                        int K, int M, const float* W_edge,
                                                        const int32_t* edge_idx,
                                                        const float* edge_w,
                                                        const int32_t* assign, float* messages,
                                                        float* tmp_projected) {
  if (!hidden || !W_edge || !edge_idx || !edge_w || !assign || !messages || !tmp_projected ||
      B <= 0 || H <= 0 || E <= 0 || K <= 0 || M <= 0)
    return 1;
  const int bad = check_dynamic_sources(assign, B, K, E, M, edge_idx);
  if (bad) return bad;
  Staging st;
  const int hh = st.in(hidden, fbytes(int64_t(B) * H));
  const int hwe = st.in(W_edge, fbytes(int64_t(E) * H * H));
  const int hi = st.in(edge_idx, ibytes(int64_t(B) * E * M));
  const int hw = st.in(edge_w, fbytes(int64_t(B) * E * M));
  const int ha = st.in(assign, ibytes(int64_t(B) * K));
  const int hm = st.out(messages, fbytes(int64_t(B) * H));
  const int hp = st.out(tmp_projected, fbytes(int64_t(B) * E * H));
  return st.run([&](hipStream_t s) {
    int rc = spider_cuda_edge_project_f32(st.f(hh), B, H, E, st.f(hwe), st.f(hp), s);
    if (rc) return rc;
    return spider_cuda_graph_message_passing_dynamic_f32(st.f(hp), B, H, E, K, M, st.i(hi),
                                                         st.f(hw), st.i(ha), st.f(hm), s);
  });
}

SPIDER_API int spider_edge_generator_f32(const float* hidden, int B, int H, int E,
                                         const float* loop_emb, int loop_emb_dim,
                                         const float* W_gen, float* out_logits) {
  if (!hidden || !loop_emb || !W_gen || !out_logits || B <= 0 || H <= 0 || E <= 0 ||
      loop_emb_dim < 0)
    return 1;
  const int64_t n_in = int64_t(H) + loop_emb_dim;
  Staging st;
  const int hh = st.in(hidden, fbytes(int64_t(B) * H));
  const int he = st.in(loop_emb, fbytes(loop_emb_dim));
  const int hw = st.in(W_gen, fbytes(int64_t(E) * E * n_in));
  const int ho = st.out(out_logits, fbytes(int64_t(B) * E * E));
  return st.run([&](hipStream_t s) {
    return spider_cuda_edge_generator_f32(st.f(hh), B, H, E, st.f(he), loop_emb_dim, st.f(hw),
                                          st.f(ho), s);
  });
}

SPIDER_API int spider_edge_generator_topk_f32(const float* hidden, int B, int H, int E, int M,
                                              const float* loop_emb, int loop_emb_dim,
                                              const float* W_gen, int32_t* edge_idx,
                                              float* edge_w, float* tmp_logits) {
  if (!tmp_logits || !hidden || !loop_emb || !W_gen || !edge_idx || !edge_w || B <= 0 || H <= 0 ||
      E <= 0 || loop_emb_dim < 0 || M <= 0 || M > E || E > 256)
    return 1;
  const int64_t n_in = int64_t(H) + loop_emb_dim;
  Staging st;
  const int hh = st.in(hidden, fbytes(int64_t(B) * H));
  const int he = st.in(loop_emb, fbytes(loop_emb_dim));
  const int hw = st.in(W_gen, fbytes(int64_t(E) * E * n_in));
  const int hl = st.out(tmp_logits, fbytes(int64_t(B) * E * E));
  const int hi = st.out(edge_idx, ibytes(int64_t(B) * E * M));
  const int hv = st.out(edge_w, fbytes(int64_t(B) * E * M));
  return st.run([&](hipStream_t s) {
    int rc = spider_cuda_edge_generator_f32(st.f(hh), B, H, E, st.f(he), loop_emb_dim, st.f(hw),
                                            st.f(hl), s);
    if (rc) return rc;
    return spider_cuda_edge_topk_f32(st.f(hl), B, E, M, st.i(hi), st.f(hv), s);
  });
}

SPIDER_API int spider_graph_from_generator_f32(const float* hidden, int B, int H, int E, int K,
                                               int M, const float* loop_emb, int loop_emb_dim,
                                               const float* W_gen, const float* W_edge,
                                               const int32_t* assign, float* messages,
                                               float* tmp_logits, int32_t* tmp_edge_idx,
                                               float* tmp_edge_w, float* tmp_projected) {
  if (!hidden || !W_gen || !W_edge || !assign || !messages || !tmp_logits || !tmp_edge_idx ||
      !tmp_edge_w || !tmp_projected || !loop_emb || B <= 0 || H <= 0 || E <= 0 || K <= 0 ||
      M <= 0 || M > E || E > 256 || loop_emb_dim < 0)
    return 1;
  for (int64_t t = 0; t < int64_t(B) * K; ++t)
    if (assign[t] >= E) return 2;
  const int64_t n_in = int64_t(H) + loop_emb_dim;
  Staging st;
  const int hh = st.in(hidden, fbytes(int64_t(B) * H));
  const int he = st.in(loop_emb, fbytes(loop_emb_dim));
  const int hg = st.in(W_gen, fbytes(int64_t(E) * E * n_in));
  const int hwe = st.in(W_edge, fbytes(int64_t(E) * H * H));
  const int ha = st.in(assign, ibytes(int64_t(B) * K));
  const int hm = st.out(messages, fbytes(int64_t(B) * H));
  const int hl = st.out(tmp_logits, fbytes(int64_t(B) * E * E));
  const int hi = st.out(tmp_edge_idx, ibytes(int64_t(B) * E * M));
  const int hv = st.out(tmp_edge_w, fbytes(int64_t(B) * E * M));
  const int hp = st.out(tmp_projected, fbytes(int64_t(B) * E * H));
  const int rc = st.run([&](hipStream_t s) {
    int r = spider_cuda_edge_generator_f32(st.f(hh), B, H, E, st.f(he), loop_emb_dim, st.f(hg),
                                           st.f(hl), s);
    if (!r) r = spider_cuda_edge_topk_f32(st.f(hl), B, E, M, st.i(hi), st.f(hv), s);
    if (!r) r = spider_cuda_edge_project_f32(st.f(hh), B, H, E, st.f(hwe), st.f(hp), s);
    if (!r)
      r = spider_cuda_graph_message_passing_dynamic_f32(st.f(hp), B, H, E, K, M, st.i(hi),
                                                        st.f(hv), st.i(ha), st.f(hm), s);
    return r;
  });
  if (rc) return rc;
  // a pick with no candidate (all logits -inf / NaN) has index -1, which the
  // scalar message pass reports as 2 when its source is selected
  return check_dynamic_sources(assign, B, K, E, M, tmp_edge_idx);
}

SPIDER_API int spider_expert_grouped_gemm_f32(const float* tokens, int B, int H, int U, int E,
                                              int K, const int32_t* assign, const float* route_w,
                                              const float* W_up, const float* W_down,
                                              float* output) {
  if (!tokens || !assign || !route_w || !W_up || !W_down || !output || B <= 0 || H <= 0 ||
      U <= 0 || E <= 0 || K <= 0 || H > 8192)
    return 1;
  const int bad = check_experts(assign, B, K, E);
  if (bad) return bad;
  Staging st;
  const int hx = st.in(tokens, fbytes(int64_t(B) * H));
  const int ha = st.in(assign, ibytes(int64_t(B) * K));
  const int hr = st.in(route_w, fbytes(int64_t(B) * K));
  const int hu = st.in(W_up, fbytes(int64_t(E) * H * U));
  const int hd = st.in(W_down, fbytes(int64_t(E) * U * H));
  const int hw = st.tmp(spider_cuda_expert_workspace_bytes(B, K, U));
  const int ho = st.out(output, fbytes(int64_t(B) * H));
  return st.run([&](hipStream_t s) {
    return spider_cuda_expert_grouped_gemm_v2_f32(st.f(hx), B, H, U, E, K, st.i(ha), st.f(hr),
                                                  st.f(hu), st.f(hd), st.f(ho), st.f(hw), s);
  });
}

SPIDER_API int spider_expert_grouped_gemm_f16(const float*, int, int, int, int, int,
                                              const int32_t*, const float*, const uint16_t*,
                                              const uint16_t*, float*) {
  return -2;
}

SPIDER_API int spider_loop_epilogue_f32(const float* h, const float* delta, const float* x0, int B,
                                        int H, float alpha, float beta, const float* ln_w,
                                        const float* ln_b, float eps, float* h_next) {
  if (!h || !delta || !x0 || !ln_w || !ln_b || !h_next || B <= 0 || H <= 0 || !(eps > 0.f) ||
      H > 8192)
    return 1;
  Staging st;
  const int hh = st.in(h, fbytes(int64_t(B) * H));
  const int hd = st.in(delta, fbytes(int64_t(B) * H));
  const int hx = st.in(x0, fbytes(int64_t(B) * H));
  const int hg = st.in(ln_w, fbytes(H));
  const int hb = st.in(ln_b, fbytes(H));
  const int ho = st.out(h_next, fbytes(int64_t(B) * H));
  return st.run([&](hipStream_t s) {
    return spider_cuda_loop_epilogue_f32(st.f(hh), st.f(hd), st.f(hx), B, H, alpha, beta,
                                         st.f(hg), st.f(hb), eps, st.f(ho), s);
  });
}

SPIDER_API int spider_loop_epilogue_f16(const float*, const float*, const float*, int, int, float,
                                        float, const float*, const float*, float, float*) {
  return -2;
}

SPIDER_API int spider_early_exit_f32(const float* h, const float* proj, int B, int H,
                                     float threshold, uint8_t* should_exit) {
  if (!h || !proj || !should_exit || B <= 0 || H <= 0) return 1;
  Staging st;
  const int hh = st.in(h, fbytes(int64_t(B) * H));
  const int hp = st.in(proj, fbytes(H));
  const int hm = st.out(should_exit, static_cast<size_t>(B));
  return st.run([&](hipStream_t s) {
    return spider_cuda_early_exit_f32(st.f(hh), st.f(hp), B, H, threshold, st.dev<uint8_t>(hm),
                                      s);
  });
}

SPIDER_API int spider_moe_loop_step_f32(
    const float* h, const float* x0, int B, int H, int E, int K, int U, int loop_idx,
    const float* router_w, const float* loop_bias, const int32_t* row_ptr,
    const int32_t* col_idx, const float* edge_w, int nnz, const float* W_edge,
    const float* W_up, const float* W_down, const float* ln_w, const float* ln_b, float alpha,
    float beta, float eps, const float* exit_proj, float exit_threshold, float* h_next,
    uint8_t* exit_mask, int32_t* tmp_assign, float* tmp_route, float* tmp_messages) {
  if (!h || !x0 || !router_w || !loop_bias || !W_up || !W_down || !ln_w || !ln_b || !h_next ||
      !tmp_assign || !tmp_route || !tmp_messages || B <= 0 || H <= 0 || E <= 0 || K <= 0 ||
      U <= 0)
    return 1;
  // the router's own checks (scalar.cpp:9) and this build's limits
  if (K > E || loop_idx < 0 || E > 64 || H > 8192 || !(eps > 0.f)) return 1;
  const bool graph = W_edge && row_ptr && col_idx && edge_w && nnz >= 0;
  if (graph && !csr_ok(row_ptr, E, nnz)) return 1;
  if (graph) {  // every source may be selected: check every row and destination
    for (int e = 0; e < E; ++e)
      if (row_ptr[e] < 0 || row_ptr[e + 1] > nnz) return 1;
    for (int e = 0; e < nnz; ++e)
      if (col_idx[e] < 0 || col_idx[e] >= E) return 2;
  }
  const int64_t BH = int64_t(B) * H, BK = int64_t(B) * K;
  Staging st;
  const int hh = st.in(h, fbytes(BH));
  const int hx = st.in(x0, fbytes(BH));
  const int hrw = st.in(router_w, fbytes(int64_t(H) * E));
  const int hb = st.in(loop_bias + static_cast<int64_t>(loop_idx) * E, fbytes(E));
  const int hu = st.in(W_up, fbytes(int64_t(E) * H * U));
  const int hd = st.in(W_down, fbytes(int64_t(E) * U * H));
  const int hg = st.in(ln_w, fbytes(H));
  const int hlb = st.in(ln_b, fbytes(H));
  const int hep = exit_proj ? st.in(exit_proj, fbytes(H)) : -1;
  int hr = -1, hc = -1, hew = -1, hwe = -1, hproj = -1;
  if (graph) {
    hr = st.in(row_ptr, ibytes(E + 1));
    hc = st.in(col_idx, ibytes(nnz));
    hew = st.in(edge_w + static_cast<int64_t>(loop_idx) * nnz, fbytes(nnz));
    hwe = st.in(W_edge, fbytes(int64_t(E) * H * H));
    hproj = st.tmp(fbytes(int64_t(B) * E * H));
  }
  const int hws = st.tmp(spider_cuda_expert_workspace_bytes(B, K, U));
  const int hdelta = st.tmp(fbytes(BH));
  const int hn = st.out(h_next, fbytes(BH));
  const int hm = exit_mask && exit_proj ? st.out(exit_mask, static_cast<size_t>(B)) : -1;
  const int ha = st.out(tmp_assign, ibytes(BK));
  const int hro = st.out(tmp_route, fbytes(BK));
  const int hmsg = st.out(tmp_messages, fbytes(BH));
  const int rc = st.run([&](hipStream_t s) {
    int r = ref_logits_router(st.f(hh), st.f(hrw), st.f(hb), B, H, E, K, st.f(hro), st.i(ha), s);
    if (r) return r;
    if (graph) {
      r = spider_cuda_edge_project_f32(st.f(hh), B, H, E, st.f(hwe), st.f(hproj), s);
      if (!r)
        r = spider_cuda_graph_message_passing_v2_f32(st.f(hproj), B, H, E, K, st.i(hr), st.i(hc),
                                                     st.f(hew), nnz, 0, st.i(ha), st.f(hmsg), s);
    } else {
      r = ref_copy_f32(st.f(hh), st.f(hmsg), BH, s);
    }
    if (!r)
      r = spider_cuda_expert_grouped_gemm_v2_f32(st.f(hmsg), B, H, U, E, K, st.i(ha), st.f(hro),
                                                 st.f(hu), st.f(hd), st.f(hdelta), st.f(hws), s);
    if (!r)
      r = spider_cuda_loop_epilogue_f32(st.f(hh), st.f(hdelta), st.f(hx), B, H, alpha, beta,
                                        st.f(hg), st.f(hlb), eps, st.f(hn), s);
    if (!r && hm >= 0)
      r = spider_cuda_early_exit_f32(st.f(hn), st.f(hep), B, H, exit_threshold,
                                     st.dev<uint8_t>(hm), s);
    return r;
  });
  if (rc == 0 && exit_mask && !exit_proj) std::memset(exit_mask, 0, static_cast<size_t>(B));
  return rc;
}

SPIDER_API const char* spider_backend_name(void) { return "hip-gfx950"; }

SPIDER_API uint32_t spider_backend_caps(void) { return 0x3u; }

}  // extern "C"
