/* Host-side checks of the C ABI under AddressSanitizer and UBSan: the entry
 * points' argument validation, workspace layout arithmetic over a range of
 * shapes, the error strings and the reference-compatible host entry points'
 * checks, all of which run on the CPU.  Built from the library's sources
 * with the host code instrumented and no device code (build.sh); on a host
 * without a GPU, calls that pass validation stop at their first HIP call
 * with SMOE_EHIP, which exercises those error paths too.  Exit status 0 and
 * a final "host ABI checks passed" line mean every check held and no
 * sanitizer report fired. */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "smoe.h"
#include "spider_kernels.h"

static int failures = 0;
#define CHECK(cond)                                                   \
  do {                                                                \
    if (!(cond)) {                                                    \
      fprintf(stderr, "check failed at line %d: %s\n", __LINE__, #cond); \
      ++failures;                                                     \
    }                                                                 \
  } while (0)

static const void* const FAKE = (const void*)0x1000; /* never dereferenced on the host */

static smoe_block make_block(int dtype, int H, int E, int K, int M, int U, int fmt, int act) {
  smoe_block b;
  memset(&b, 0, sizeof b);
  b.act_dtype = dtype;
  b.H = H;
  b.E = E;
  b.K = K;
  b.M = M;
  b.L = 32;
  b.R = 6;
  b.router_w = b.edge_gen_w = b.edge_value_w = FAKE;
  b.loop_bias = b.edge_loop_bias = (const float*)FAKE;
  b.experts.format = fmt;
  b.experts.act = act;
  b.experts.E = E;
  b.experts.H = H;
  b.experts.U = U;
  b.experts.group_size = fmt == SMOE_INT4 ? 128 : 0;
  b.experts.scale_dtype = fmt == SMOE_INT4 ? SMOE_F16 : SMOE_F32;
  b.experts.w_up = b.experts.w_down = FAKE;
  if (fmt == SMOE_FP8_E4M3 || fmt == SMOE_INT4) b.experts.s_up = b.experts.s_down = FAKE;
  b.alpha = 0.5f;
  b.beta = 0.1f;
  b.eps = 1e-5f;
  return b;
}

/* every region of a layout lies inside total, 256-byte aligned, and the
 * regions do not overlap one another */
static void check_layout(const smoe_block* b, int N) {
  smoe_ws_layout l;
  memset(&l, 0xAB, sizeof l);
  CHECK(smoe_block_workspace_layout(b, N, &l) == SMOE_OK);
  CHECK(l.total == smoe_block_workspace_bytes(b, N));
  const size_t* f = &l.logits;
  const size_t* end = &l.h_tmp2;
  const int n = (int)(end - f) + 1;
  for (int i = 0; i < n; ++i) {
    CHECK(f[i] % 256 == 0);
    CHECK(f[i] <= l.total);
  }
  /* offsets are non-decreasing in declaration order (the layout is a bump
   * allocator), so a region ends where the next begins at the latest */
  for (int i = 0; i + 1 < n; ++i) CHECK(f[i] <= f[i + 1]);
  CHECK(l.S >= 1 && l.S <= 64);
}

int main(void) {
  CHECK(smoe_abi_version() == SMOE_ABI_VERSION);
  CHECK(strcmp(smoe_backend_name(), "hip-gfx950") == 0);
  CHECK(smoe_backend_caps() == 0xFu);
  CHECK(strcmp(spider_backend_name(), "hip-gfx950") == 0);

  /* workspace layouts over shapes the block takes */
  const int Ns[] = {0, 1, 7, 64, 65, 300, 2176, 16384, 70000};
  const int shapes[][6] = {
      /* H, E, K, M, U, fmt */
      {1024, 16, 2, 2, 2816, SMOE_BF16},  {1024, 16, 2, 2, 2816, SMOE_FP8_E4M3},
      {1024, 32, 4, 2, 1408, SMOE_BF16},  {2048, 64, 2, 4, 1408, SMOE_INT4},
      {128, 256, 2, 2, 256, SMOE_BF16},   {128, 128, 4, 4, 256, SMOE_BF16},
      {64, 4, 2, 2, 128, SMOE_F32},       {4096, 8, 2, 2, 1024, SMOE_BF16},
  };
  for (size_t s = 0; s < sizeof shapes / sizeof shapes[0]; ++s) {
    const int* p = shapes[s];
    const int dtype = p[5] == SMOE_F32 ? SMOE_F32 : SMOE_BF16;
    const int act = p[5] == SMOE_BF16 && p[4] % 64 == 0 ? SMOE_ACT_SWIGLU : SMOE_ACT_GELU;
    smoe_block b = make_block(dtype, p[0], p[1], p[2], p[3], p[4], p[5], act);
    for (size_t i = 0; i < sizeof Ns / sizeof Ns[0]; ++i) check_layout(&b, Ns[i]);
  }

  /* shapes outside the limits are refused with SMOE_EINVAL and a message */
  {
    smoe_block b = make_block(SMOE_BF16, 1024, 257, 2, 2, 2816, SMOE_BF16, SMOE_ACT_GELU);
    smoe_ws_layout l;
    CHECK(smoe_block_workspace_layout(&b, 64, &l) == SMOE_EINVAL);
    CHECK(smoe_block_workspace_bytes(&b, 64) == 0);
    CHECK(strlen(smoe_last_error()) > 0);
    b = make_block(SMOE_BF16, 1024, 16, 17, 2, 2816, SMOE_BF16, SMOE_ACT_GELU);
    CHECK(smoe_block_workspace_layout(&b, 64, &l) == SMOE_EINVAL);
    b = make_block(SMOE_BF16, 1020, 16, 2, 2, 2816, SMOE_BF16, SMOE_ACT_GELU);
    CHECK(smoe_block_workspace_layout(&b, 64, &l) == SMOE_EINVAL);
    b = make_block(SMOE_BF16, 1024, 16, 2, 2, 2816, SMOE_BF16, SMOE_ACT_GELU);
    CHECK(smoe_block_workspace_layout(NULL, 64, &l) != SMOE_OK);
    CHECK(smoe_block_workspace_layout(&b, 64, NULL) == SMOE_EINVAL);
    CHECK(smoe_block_workspace_layout(&b, -1, &l) == SMOE_EINVAL);
  }

  /* argument validation of the entry points: null buffers, bad sizes */
  {
    smoe_block b = make_block(SMOE_BF16, 1024, 16, 2, 2, 2816, SMOE_BF16, SMOE_ACT_SWIGLU);
    const size_t ws = smoe_block_workspace_bytes(&b, 64);
    CHECK(ws > 0);
    void* dev = (void*)FAKE;
    CHECK(smoe_block_forward(&b, NULL, dev, dev, 64, 0, 6, dev, ws, NULL) == SMOE_EINVAL);
    CHECK(smoe_block_forward(&b, dev, dev, dev, 64, 0, 6, dev, ws - 1, NULL) == SMOE_ECAPACITY);
    CHECK(smoe_block_forward(&b, dev, dev, dev, 64, 5, 6, dev, ws, NULL) != SMOE_OK);
    CHECK(smoe_block_forward_exit(&b, dev, dev, dev, 64, 0, 6, NULL, 0.5f, NULL, NULL, dev, ws,
                                  NULL) == SMOE_EINVAL);
    float nan_bits;
    const uint32_t qnan = 0x7fc00000u;
    memcpy(&nan_bits, &qnan, sizeof nan_bits);
    CHECK(smoe_block_forward_exit(&b, dev, dev, dev, 64, 0, 6, (const float*)FAKE, nan_bits,
                                  (int32_t*)FAKE, NULL, dev, ws, NULL) == SMOE_EINVAL);
    CHECK(smoe_router_topk(NULL, SMOE_BF16, 64, 1024, dev, NULL, 16, 2, NULL, NULL, NULL, NULL, 0,
                           NULL) != SMOE_OK);
    CHECK(smoe_dispatch_plan(NULL, NULL, 64, 2, 16, NULL, NULL, NULL, NULL, NULL, NULL, 0, NULL) !=
          SMOE_OK);
    CHECK(smoe_select_topk(NULL, 64, 16, 2, SMOE_SELECT_ROUTER, NULL, NULL, NULL) != SMOE_OK);
    CHECK(smoe_select_topk((const float*)FAKE, 64, 300, 2, SMOE_SELECT_ROUTER, (float*)FAKE,
                           (int32_t*)FAKE, NULL) != SMOE_OK);
    CHECK(smoe_linear(NULL, 4, 64, dev, SMOE_BF16, NULL, NULL, 64, SMOE_LINEAR_NONE, dev,
                      SMOE_F32, NULL) != SMOE_OK);
    CHECK(smoe_linear_fp8fp8(NULL, NULL, 4, 256, NULL, NULL, NULL, 64, SMOE_LINEAR_NONE, dev,
                             SMOE_F32, NULL) != SMOE_OK);
    CHECK(smoe_linear_fp8fp8((const uint8_t*)FAKE, (const float*)FAKE, 4, 100, (const uint8_t*)FAKE,
                             (const float*)FAKE, NULL, 64, SMOE_LINEAR_NONE, dev, SMOE_F32,
                             NULL) != SMOE_OK); /* K % 256 */
    CHECK(smoe_quantize_fp8_tensor(NULL, SMOE_BF16, 4, 64, 64, 0, NULL, NULL, NULL, 0, NULL) !=
          SMOE_OK);
    CHECK(smoe_pack_weight_tiles(NULL, SMOE_BF16, 1, 16, 64, NULL, NULL) != SMOE_OK);
    CHECK(smoe_pack_weight_tiles(dev, SMOE_BF16, 1, 15, 64, dev, NULL) != SMOE_OK); /* N % 16 */
    CHECK(smoe_pack_int4_qtiles(dev, 1, 63, 64, dev, NULL) != SMOE_OK);             /* N % 64 */
    CHECK(smoe_remap_ids(NULL, 4, NULL, 16, NULL, NULL) != SMOE_OK);
    CHECK(smoe_events_create(-1, NULL) != SMOE_OK);
  }

  /* workspace queries of the stage entry points */
  CHECK(smoe_router_workspace_bytes(16384, 16) > 0);
  CHECK(smoe_dispatch_workspace_bytes(16384, 2, 16) > 0);
  CHECK(smoe_edge_topm_workspace_bytes(16384, 2, 16, 2) > 0);
  CHECK(smoe_edge_message_workspace_bytes(16384, 1024, 16, 2, 2, SMOE_BF16) > 0);
  CHECK(smoe_quantize_fp8_workspace_bytes() > 0);

  /* the reference's host entry points: its argument checks (1) and index
   * checks (2) run before any staging */
  {
    float w[8];
    int32_t idx[8];
    const float logits[8] = {0};
    const float bias[4] = {0};
    CHECK(spider_router_f32(NULL, bias, 2, 4, 2, 0, w, idx) == 1);
    CHECK(spider_router_f32(logits, bias, 2, 4, 5, 0, w, idx) == 1); /* K > E */
    CHECK(spider_router_f16(NULL, NULL, 2, 4, 2, 0, w, idx) == -2);
    CHECK(spider_edge_topk_f32(NULL, 2, 4, 2, idx, w) == 1);
    const int32_t row_ptr[3] = {0, 1, 2};
    const int32_t col_bad[2] = {0, 7}; /* destination 7 of 2 experts */
    const float ew[2] = {1.f, 1.f};
    const int32_t assign[2] = {0, 1};
    const float rw[2] = {1.f, 1.f};
    float h[2 * 4] = {0}, msg[2 * 4];
    const int rc = spider_graph_message_passing_f32(h, 2, 4, 2, 1, row_ptr, col_bad, ew, 2, 0,
                                                    assign, rw, msg);
    CHECK(rc == 1 || rc == 2);
  }

  if (failures) {
    fprintf(stderr, "%d host ABI check(s) failed\n", failures);
    return 1;
  }
  printf("host ABI checks passed\n");
  return 0;
}
