// Per-token combines of the Spider-MoE block (one wave per token row).
//
//  msg[t]  = sum over the token's destination rows (ascending destination)
//            of proj[row] (= c * W_edge[d] h, model.py:277-288)
//  h'[t]   = LayerNorm(h + alpha * delta + beta * x0)  (model.py:317), with
//            delta = sum over the token's expert rows with weight > 0
//            (ascending expert, as sparse_experts.py:51-63 accumulates) of
//            y[row] (= w * FFN_e(msg), the down-GEMM epilogue)
//
// A fixed summation order per token and no atomics make every output
// bit-reproducible run to run.  Rows are read as 16-byte vectors; H must be
// a multiple of 8.
#include "smoe_common.hpp"
#include "smoe_internal.hpp"
#include "smoe_rows.hpp"

namespace smoe {

// CPL = 8-element chunks per lane (H <= 512 * CPL)
// Lane j (< S) holds the token's j-th (destination, row) entry.  DENSE: the
// row of destination d is d * dense_n + t (the decode edge projection's
// layout), else d_tokrow's.
template <int CPL, int PDT, int MDT, bool DENSE>
__global__ __launch_bounds__(256) void k_msg_combine(const void* __restrict__ proj,
                                                     const int32_t* __restrict__ tok_d,
                                                     const int32_t* __restrict__ d_tokrow, int N,
                                                     int S, int H, void* __restrict__ msg,
                                                     int dense_n) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= N) return;
  // unconditional loads (lanes past S read entry S-1 and drop it): no
  // branch for the compiler to wait at
  const int64_t e = static_cast<int64_t>(t) * S + (lane < S ? lane : S - 1);
  const int d = tok_d[e];
  const int r = DENSE ? d * dense_n + t : d_tokrow[e];
  const int my_row = (lane < S && d >= 0) ? r : -1;  // ascending destination (tok_d is sorted)
  float acc[CPL][8];
#pragma unroll
  for (int c = 0; c < CPL; ++c)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[c][i] = 0.f;
  gather_add<CPL, PDT>(proj, H, my_row, __ballot(my_row >= 0), acc);
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int col = (lane + 64 * c) * 8;
    if (col < H) store8<MDT>(msg, static_cast<int64_t>(t) * H + col, acc[c]);
  }
}

// GATE: the exit gate of the early-exit decode (model.py:450-473).  A token
// whose active[t] is 0 left the orbit in an earlier loop: its h passes
// through unchanged.  An active token gets h' and then
// conf = sigmoid(exit_w . h' + exit_b) (fp32, over h' as stored); it leaves
// the orbit (active[t] = 0) when conf > thr, and loops[t] (if not null)
// counts the loops it ran.
template <int CPL, int ADT, int YDT, bool GATE>
__global__ __launch_bounds__(256) void k_epilogue(
    const void* __restrict__ h, const void* __restrict__ x0, const void* __restrict__ y,
    const int32_t* __restrict__ tok_e, const float* __restrict__ tok_ew,
    const int32_t* __restrict__ e_tokrow, int N, int K, int H, float alpha, float beta,
    const float* __restrict__ ln_w, const float* __restrict__ ln_b, float eps,
    void* __restrict__ out, const float* __restrict__ exit_wb, float thr,
    int32_t* __restrict__ active, int32_t* __restrict__ loops) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= N) return;
  // the token's own rows and the LayerNorm parameters do not depend on the
  // routing: their loads go out first, with the routing metadata
  float hv[CPL][8], xv[CPL][8], d[CPL][8], gw[CPL][8], gb[CPL][8], ew[CPL][8];
  ln_load<CPL, ADT>(h, x0, ln_w, ln_b, t, H, hv, xv, gw, gb);
#pragma unroll
  for (int c = 0; c < CPL; ++c)
#pragma unroll
    for (int i = 0; i < 8; ++i) d[c][i] = 0.f;
  // the loop count is read here, unconditionally (from active when loops is
  // null, value unused), so its latency hides behind the row loads; a load
  // under the final lane-0 branch would be waited for at the kernel's end
  int loops_in = 0;
  if (GATE) loops_in = (loops ? loops : active)[t];
  if (GATE && active[t] == 0) {  // wave-uniform: out of orbit, h passes through
    if (out != h)
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const int col = (lane + 64 * c) * 8;
        if (col < H) store8<ADT>(out, static_cast<int64_t>(t) * H + col, hv[c]);
      }
    return;
  }
  // lane j (< K): the token's j-th expert row if its weight is > 0 (rows
  // with weight <= 0 are dropped from the FFN, sparse_experts.py:56); lanes
  // past K read entry K-1 and drop it.  Without routing (tok_e null) y is
  // the dense delta [N, H] and lane 0 takes row t.
  int my_row = lane == 0 ? t : -1;
  if (tok_e) {
    const int64_t e = static_cast<int64_t>(t) * K + (lane < K ? lane : K - 1);
    const int te = tok_e[e];
    const float tw = tok_ew[e];
    const int tr = e_tokrow[e];
    my_row = (lane < K && te >= 0 && tw > 0.f) ? tr : -1;
  }
  gather_add<CPL, YDT>(y, H, my_row, __ballot(my_row >= 0), d);  // ascending expert order
  if (GATE)  // x0 is read by ln_row before it returns: the exit weights go elsewhere
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int col = (lane + 64 * c) * 8;
      load8<SMOE_F32>(exit_wb, col < H ? col : 0, ew[c]);
    }
  float o[CPL][8];
  ln_row<CPL>(hv, xv, gw, gb, d, H, alpha, beta, eps, o);
  float g = 0.f;  // exit-gate dot product (GATE)
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int col = (lane + 64 * c) * 8;
    if (col < H) {
      store8<ADT>(out, static_cast<int64_t>(t) * H + col, o[c]);
      if (GATE)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float stored = ADT == SMOE_BF16 ? bf2f(f2bf(o[c][i])) : o[c][i];
          g += stored * ew[c][i];
        }
    }
  }
  if (GATE) {
    // a bf16 model's exit_head is a bf16 Linear: its output (the logit) is
    // rounded to bf16 before the fp32 sigmoid (model.py:467)
    float z = wave_sum(g) + exit_wb[H];
    if (ADT == SMOE_BF16) z = bf2f(f2bf(z));
    if (lane == 0) {
      if (1.0f / (1.0f + expf(-z)) > thr) active[t] = 0;
      if (loops) loops[t] = loops_in + 1;
    }
  }
}

template <int CPL, int YDT, int ODT>
__global__ __launch_bounds__(256) void k_delta_combine(const void* __restrict__ y,
                                                       const int32_t* __restrict__ tok_row, int N,
                                                       int K, int H, void* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= N) return;
  float d[CPL][8];
#pragma unroll
  for (int c = 0; c < CPL; ++c)
#pragma unroll
    for (int i = 0; i < 8; ++i) d[c][i] = 0.f;
  const int r = tok_row[static_cast<int64_t>(t) * K + (lane < K ? lane : K - 1)];
  const int my_row = lane < K ? r : -1;
  gather_add<CPL, YDT>(y, H, my_row, __ballot(my_row >= 0), d);  // slot (= ascending expert) order
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int col = (lane + 64 * c) * 8;
    if (col < H) store8<ODT>(out, static_cast<int64_t>(t) * H + col, d[c]);
  }
}

// The same sum for rows of any width (H not a multiple of 8, or > 4096):
// one thread per (token, column), the token's rows in slot order.
template <int YDT, int ODT>
__global__ __launch_bounds__(256) void k_delta_combine_any(const void* __restrict__ y,
                                                           const int32_t* __restrict__ tok_row,
                                                           int N, int K, int H,
                                                           void* __restrict__ out) {
  const int t = blockIdx.y;
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= H) return;
  float acc = 0.f;
  for (int s = 0; s < K; ++s) {
    const int r = tok_row[static_cast<int64_t>(t) * K + s];
    if (r < 0) continue;
    const int64_t o = static_cast<int64_t>(r) * H + j;
    acc += YDT == SMOE_F32 ? reinterpret_cast<const float*>(y)[o]
                           : bf2f(reinterpret_cast<const uint16_t*>(y)[o]);
  }
  const int64_t o = static_cast<int64_t>(t) * H + j;
  if (ODT == SMOE_F32) reinterpret_cast<float*>(out)[o] = acc;
  else reinterpret_cast<uint16_t*>(out)[o] = f2bf(acc);
}

namespace {
int last_rc() { return hipGetLastError() == hipSuccess ? SMOE_OK : SMOE_EHIP; }
}  // namespace

int launch_msg_combine(const void* proj, int pdt, const int32_t* tok_d, const int32_t* d_tokrow,
                       int N, int S, int H, void* msg, int mdt, hipStream_t s, int dense_n) {
  if (S < 1 || S > 64 || dense_n < 0 || (dense_n > 0 && dense_n < N)) return SMOE_EINVAL;
  if (N <= 0) return SMOE_OK;
  return by_cpl(H, [&](auto cpl) {
    return by_dt(pdt, [&](auto pd) {
      return by_dt(mdt, [&](auto md) {
        constexpr int C = decltype(cpl)::value, P = decltype(pd)::value, Q = decltype(md)::value;
        if (dense_n > 0)
          hipLaunchKernelGGL((k_msg_combine<C, P, Q, true>), dim3((N + 3) / 4), dim3(256), 0, s,
                             proj, tok_d, d_tokrow, N, S, H, msg, dense_n);
        else
          hipLaunchKernelGGL((k_msg_combine<C, P, Q, false>), dim3((N + 3) / 4), dim3(256), 0, s,
                             proj, tok_d, d_tokrow, N, S, H, msg, 0);
        return last_rc();
      });
    });
  });
}

int launch_epilogue(const void* h, const void* x0, int adt, const void* y, int ydt,
                    const int32_t* tok_e, const float* tok_ew, const int32_t* e_tokrow, int N,
                    int K, int H, float alpha, float beta, const float* ln_w, const float* ln_b,
                    float eps, void* out, const ExitGate* gate, hipStream_t s) {
  if (K < 1 || K > 64) return SMOE_EINVAL;  // one lane per entry
  if (N <= 0) return SMOE_OK;
  if (gate && (!gate->exit_wb || !gate->active)) return SMOE_EINVAL;
  return by_cpl(H, [&](auto cpl) {
    return by_dt(adt, [&](auto ad) {
      return by_dt(ydt, [&](auto yd) {
        constexpr int C = decltype(cpl)::value, A = decltype(ad)::value, Y = decltype(yd)::value;
        if (gate)
          hipLaunchKernelGGL((k_epilogue<C, A, Y, true>), dim3((N + 3) / 4), dim3(256), 0, s, h, x0,
                             y, tok_e, tok_ew, e_tokrow, N, K, H, alpha, beta, ln_w, ln_b, eps, out,
                             gate->exit_wb, gate->threshold, gate->active, gate->loops);
        else
          hipLaunchKernelGGL((k_epilogue<C, A, Y, false>), dim3((N + 3) / 4), dim3(256), 0, s, h,
                             x0, y, tok_e, tok_ew, e_tokrow, N, K, H, alpha, beta, ln_w, ln_b, eps,
                             out, nullptr, 0.f, nullptr, nullptr);
        return last_rc();
      });
    });
  });
}

int launch_delta_combine(const void* y, int ydt, const int32_t* tok_row, int N, int K, int H,
                         void* out, int odt, hipStream_t s) {
  if (K < 1 || K > 64 || H < 1 || N > 65535 * 64) return SMOE_EINVAL;  // one lane per entry
  if (N <= 0) return SMOE_OK;
  if (H % 8 || H > 4096) {
    if (N > 65535) return SMOE_EINVAL;  // grid.y
    return by_dt(ydt, [&](auto yd) {
      return by_dt(odt, [&](auto od) {
        hipLaunchKernelGGL((k_delta_combine_any<decltype(yd)::value, decltype(od)::value>),
                           dim3((H + 255) / 256, N), dim3(256), 0, s, y, tok_row, N, K, H, out);
        return last_rc();
      });
    });
  }
  return by_cpl(H, [&](auto cpl) {
    return by_dt(ydt, [&](auto yd) {
      return by_dt(odt, [&](auto od) {
        hipLaunchKernelGGL((k_delta_combine<decltype(cpl)::value, decltype(yd)::value, decltype(od)::value>),
                           dim3((N + 3) / 4), dim3(256), 0, s, y, tok_row, N, K, H, out);
        return last_rc();
      });
    });
  });
}

}  // namespace smoe
