/* The C-ABI library's host code under AddressSanitizer and
 * UndefinedBehaviorSanitizer: every entry point's argument checks, including
 * sizes at the edge of int64 that must be rejected before any size
 * arithmetic can overflow.  Every call here is answered on the host; none
 * reaches the device (the pointers are placeholders that are never
 * dereferenced), so the checker runs without a GPU. */
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "argcases.h"

static int sample_capi(const void* a, int b, int64_t c, int64_t d, int64_t e, const int32_t* f,
                       int64_t g, int64_t h, const uint32_t* i, int64_t j, const float* k,
                       const gtp_sampler_params* l, const uint8_t* m, int64_t n, int64_t* o,
                       float* p, float* q, int32_t* r, float* s, int32_t* t, int32_t* u) {
  return gtp_sample_rows(a, b, c, d, e, f, g, h, i, j, k, l, m, n, o, p, q, r, s, t, u, NULL, 0,
                         NULL);
}

static int sample_noalloc(const void* a, int b, int64_t c, int64_t d, int64_t e, const int32_t* f,
                          int64_t g, int64_t h, const uint32_t* i, int64_t j, const float* k,
                          const gtp_sampler_params* l, const uint8_t* m, int64_t n, int64_t* o,
                          float* p, float* q, int32_t* r, float* s, int32_t* t, int32_t* u) {
  return gtp_sample_rows_noalloc(a, b, c, d, e, f, g, h, i, j, k, l, m, n, o, p, q, r, s, t, u,
                                 NULL);
}

static int logprob_capi(const void* a, int b, int64_t c, int64_t d, int64_t e, const void* f,
                        int g, float* h, float* i, int32_t* j) {
  return gtp_logprob_entropy_rows(a, b, c, d, e, f, g, h, i, j, NULL);
}

int main(void) {
  const int I = GTP_ERR_INVALID_ARGUMENT, X = GTP_ERR_UNSUPPORTED, OK = GTP_OK;
  const char* w = "capi";
  sample_arg_cases(sample_capi, "capi sampler");
  sample_arg_cases(sample_noalloc, "capi sampler noalloc");
  logprob_arg_cases(logprob_capi, "capi logprob");

  const void* L = PH(const void*);
  const void* T = PH(const void*);
  const float* F = PH(const float*);
  float* o = PH(float*);
  void* g = PH(void*);
  const gtp_sampler_params topp = {0.7f, 0, 0.9f, 1.0f};

  /* the workspace query: zero for every call that cannot run */
  {
    int32_t rt = 0, sl = 0;
    EXPECT_RC(w, gtp_sample_route(1, 4, 151936, 1, 0, 0, NULL, 0, &rt, &sl), I);
    EXPECT_RC(w, gtp_sample_route(1, 4, 151936, 1, 0, 0, &topp, 0, NULL, &sl), I);
    EXPECT_RC(w, gtp_sample_route(1, 0, 151936, 1, 0, 0, &topp, 0, &rt, &sl), I);
    EXPECT_RC(w, gtp_sample_route(1, 4, 0, 1, 0, 0, &topp, 0, &rt, &sl), I);
    EXPECT_RC(w, gtp_sample_route(1, 4, 151936, 1, -1, 0, &topp, 0, &rt, &sl), I);
    EXPECT_RC(w, gtp_sample_route(7, 4, 151936, 1, 0, 0, &topp, 0, &rt, &sl), I);
    EXPECT_RC(w, gtp_sample_route(1, 4, INT64_MAX, 1, 0, 0, &topp, 0, &rt, &sl), X);
    EXPECT_RC(w, gtp_sample_route(1, INT64_MAX, 151936, 1, 0, 0, &topp, 0, &rt, &sl), X);
    EXPECT_RC(w, gtp_sample_route(1, 4, 151936, 1, 0, 0, &topp, SIZE_MAX, &rt, NULL), OK);
    EXPECT_RC(w, rt, GTP_ROUTE_TOPP_SPLIT);
  }
  EXPECT_RC(w, (int)gtp_sample_workspace_bytes(1, 4, 100, NULL), 0);
  EXPECT_RC(w, (int)gtp_sample_workspace_bytes(1, 0, 151936, &topp), 0);
  EXPECT_RC(w, (int)gtp_sample_workspace_bytes(1, 4, 0, &topp), 0);
  EXPECT_RC(w, (int)(gtp_sample_workspace_bytes(1, INT64_MAX, 151936, &topp) != 0), 0);
  EXPECT_RC(w, (int)(gtp_sample_workspace_bytes(1, 64, INT64_MAX, &topp) != 0), 0);
  /* top-p rows of a large batch (and fp32 rows): one workgroup per row, no
     workspace */
  EXPECT_RC(w, (int)gtp_sample_workspace_bytes(1, 256, 151936, &topp), 0);
  EXPECT_RC(w, (int)gtp_sample_workspace_bytes(0, 64, 151936, &topp), 0);
  /* bf16 top-p rows of a small batch, split over S = 4 workgroups per row
     (no device here: 256 CUs assumed): 16 KB of counters, 64 x 4 headers of
     64 bytes, 64 x 4 slots of 64 KB */
  EXPECT_RC(w, (int)gtp_sample_workspace_bytes(1, 64, 151936, &topp), 16384 + 16384 + 64 * 4 * 65536);
  /* the library's own workspace is bounded: 8192 fp32 rows of 2^18 with
     top-k 128 merge more candidate lists than it holds */
  {
    const gtp_sampler_params topk = {1.0f, 128, 1.0f, 1.0f};
    EXPECT_RC(w, (int)(gtp_sample_workspace_bytes(0, 8192, 1 << 18, &topk) > GTP_NOALLOC_SCRATCH_BYTES), 1);
    EXPECT_RC(w, gtp_sample_rows_noalloc(L, 0, 8192, 1 << 18, 1 << 18, NULL, 0, 0, NULL, 0, F, &topk,
                                         NULL, 0, PH(int64_t*), NULL, NULL, NULL, NULL, NULL, NULL,
                                         NULL),
              X);
  }

  EXPECT_RC(w, gtp_lse_partial_rows(L, 1, -1, 10, 10, 0, T, 0, o, 0, NULL), I);
  EXPECT_RC(w, gtp_lse_partial_rows(L, 1, 4, 0, 10, 0, T, 0, o, 0, NULL), I);
  EXPECT_RC(w, gtp_lse_partial_rows(L, 1, 4, 10, 9, 0, T, 0, o, 0, NULL), I);
  EXPECT_RC(w, gtp_lse_partial_rows(L, 1, 4, 10, 10, -1, T, 0, o, 0, NULL), I);
  EXPECT_RC(w, gtp_lse_partial_rows(NULL, 1, 4, 10, 10, 0, T, 0, o, 0, NULL), I);
  EXPECT_RC(w, gtp_lse_partial_rows(L, 1, 4, 10, 10, 0, T, 0, NULL, 0, NULL), I);
  EXPECT_RC(w, gtp_lse_partial_rows(L, 7, 4, 10, 10, 0, T, 0, o, 0, NULL), I);
  EXPECT_RC(w, gtp_lse_partial_rows(L, 1, INT64_MAX, 10, 10, 0, T, 0, o, 0, NULL), X);
  EXPECT_RC(w, gtp_lse_partial_rows(NULL, 1, 0, 10, 10, 0, NULL, 0, NULL, 0, NULL), OK);

  EXPECT_RC(w, gtp_lse_finalize_rows(F, -1, o, NULL, NULL), I);
  EXPECT_RC(w, gtp_lse_finalize_rows(NULL, 4, o, NULL, NULL), I);
  EXPECT_RC(w, gtp_lse_finalize_rows(F, INT64_MAX, o, NULL, NULL), X);
  EXPECT_RC(w, gtp_lse_finalize_rows(NULL, 0, NULL, NULL, NULL), OK);

  EXPECT_RC(w, gtp_logprob_backward_rows(L, 1, -1, 10, 10, 0, T, 0, F, F, g, 10, NULL), I);
  EXPECT_RC(w, gtp_logprob_backward_rows(L, 1, 4, 10, 10, 0, T, 0, F, F, g, 9, NULL), I);
  EXPECT_RC(w, gtp_logprob_backward_rows(L, 1, 4, 10, 10, 0, T, 0, F, NULL, g, 10, NULL), I);
  EXPECT_RC(w, gtp_logprob_backward_rows(L, 1, 4, 10, 10, 0, T, 0, F, F, NULL, 10, NULL), I);
  EXPECT_RC(w, gtp_logprob_backward_rows(L, 8, 4, 10, 10, 0, T, 0, F, F, g, 10, NULL), I);
  EXPECT_RC(w, gtp_logprob_backward_rows(L, 1, INT64_MAX, 10, 10, 0, T, 0, F, F, g, 10, NULL), X);
  EXPECT_RC(w, gtp_logprob_backward_rows(NULL, 1, 0, 10, 10, 0, NULL, 0, NULL, NULL, NULL, 10,
                                         NULL),
            OK);

  uint16_t* h = PH(uint16_t*);
  EXPECT_RC(w, gtp_logprob_backward_split_rows(F, -1, 10, 10, 0, T, 0, F, F, h, h, 10, NULL), I);
  EXPECT_RC(w, gtp_logprob_backward_split_rows(F, 4, 10, 10, 0, T, 0, F, F, h, NULL, 10, NULL), I);
  EXPECT_RC(w, gtp_logprob_backward_split_rows(F, 4, 10, 10, 0, T, 0, F, F, h, h, 3, NULL), I);
  EXPECT_RC(w, gtp_logprob_backward_split_rows(F, INT64_MAX, 10, 10, 0, T, 0, F, F, h, h, 10,
                                               NULL),
            X);

  EXPECT_RC(w, gtp_graspo_loss_forward(F, F, F, NULL, 0, 0, 8, 0.8f, 1.2f, o, o, o, NULL), I);
  EXPECT_RC(w, gtp_graspo_loss_forward(F, F, F, NULL, 0, 4, 0, 0.8f, 1.2f, o, o, o, NULL), I);
  EXPECT_RC(w, gtp_graspo_loss_forward(F, NULL, F, NULL, 0, 4, 8, 0.8f, 1.2f, o, o, o, NULL), I);
  EXPECT_RC(w, gtp_graspo_loss_forward(F, F, F, NULL, 0, (int64_t)1 << 31, 8, 0.8f, 1.2f, o, o, o,
                                       NULL),
            X);
  EXPECT_RC(w, gtp_graspo_loss_backward(F, F, F, NULL, 0, F, F, -4, 8, 0.8f, 1.2f, o, NULL), I);
  EXPECT_RC(w, gtp_graspo_loss_backward(F, F, F, NULL, 0, NULL, F, 4, 8, 0.8f, 1.2f, o, NULL), I);
  /* B * T beyond int64, and beyond the launch grid */
  EXPECT_RC(w, gtp_graspo_loss_backward(F, F, F, NULL, 0, F, F, (int64_t)1 << 40, (int64_t)1 << 40,
                                        0.8f, 1.2f, o, NULL),
            X);
  EXPECT_RC(w, gtp_graspo_loss_backward(F, F, F, NULL, 0, F, F, 1, (int64_t)1 << 40, 0.8f, 1.2f,
                                        o, NULL),
            X);

  int64_t* ids = PH(int64_t*);
  uint8_t* fin = PH(uint8_t*);
  int32_t* flags = PH(int32_t*);
  EXPECT_RC(w, gtp_decode_update_rows(ids, NULL, -1, 2, 0, fin, NULL, 0, NULL, 0, 0, flags, NULL),
            I);
  EXPECT_RC(w, gtp_decode_update_rows(ids, NULL, 4, 2, 0, fin, NULL, 0, NULL, 0, -1, flags, NULL),
            I);
  EXPECT_RC(w, gtp_decode_update_rows(ids, NULL, 4, 2, 0, fin, NULL, 0, NULL, 0, 0, NULL, NULL),
            I);
  EXPECT_RC(w, gtp_decode_update_rows(NULL, NULL, 4, 2, 0, fin, NULL, 0, NULL, 0, 0, flags, NULL),
            I);
  EXPECT_RC(w, gtp_decode_update_rows(ids, NULL, 4, 2, 0, fin, ids, 5, NULL, 0, 5, flags, NULL),
            I);
  EXPECT_RC(w, gtp_decode_update_rows(ids, NULL, 4, 2, 0, fin, NULL, 0, fin, 3, 5, flags, NULL),
            I);
  EXPECT_RC(w, gtp_decode_update_rows(ids, NULL, INT64_MAX, 2, 0, fin, NULL, 0, NULL, 0, 0, flags,
                                      NULL),
            X);

  uint32_t* inexact = PH(uint32_t*);
  EXPECT_RC(w, gtp_f32_to_bf16_exact(F, -1, h, inexact, NULL), I);
  EXPECT_RC(w, gtp_f32_to_bf16_exact(F, 10, h, NULL, NULL), I);
  EXPECT_RC(w, gtp_f32_to_bf16_exact(NULL, 10, h, inexact, NULL), I);
  EXPECT_RC(w, gtp_f32_to_bf16_exact((const float*)(uintptr_t)0x14, INT64_MAX, h, inexact, NULL),
            X);
  EXPECT_RC(w, gtp_f32_to_bf16_exact(NULL, 0, NULL, inexact, NULL), OK);

  EXPECT_RC(w, gtp_time_next_launch(NULL, g), I);
  EXPECT_RC(w, gtp_time_next_launch(g, NULL), I);

  uint32_t* out = PH(uint32_t*);
  const void* A = (const void*)(uintptr_t)0x100;
  EXPECT_RC(w, gtp_stream_read_rows(A, -1, 16, 16, out, NULL), I);
  EXPECT_RC(w, gtp_stream_read_rows(A, 4, -16, 16, out, NULL), I);
  EXPECT_RC(w, gtp_stream_read_rows(A, 4, 32, 16, out, NULL), I);
  EXPECT_RC(w, gtp_stream_read_rows(A, 4, 32, 32, NULL, NULL), I);
  EXPECT_RC(w, gtp_stream_read_rows((const void*)(uintptr_t)0x104, 4, 32, 32, out, NULL), X);
  EXPECT_RC(w, gtp_stream_read_rows(A, 4, 24, 32, out, NULL), X);
  EXPECT_RC(w, gtp_stream_read_rows(A, INT64_MAX, 32, 32, out, NULL), X);
  EXPECT_RC(w, gtp_stream_read_rows(NULL, 0, 32, 32, NULL, NULL), OK);

  const uint16_t* HB = PH(const uint16_t*);
  const uint16_t* WB = (const uint16_t*)(uintptr_t)0x1000;
  void* wsp = PH(void*);
  const size_t wsz = gtp_lm_head_workspace_bytes(256, 1000);
  EXPECT_RC(w, wsz > 0, 1);
  EXPECT_RC(w, (int)gtp_lm_head_workspace_bytes(0, 1000), 0);
  EXPECT_RC(w, (int)gtp_lm_head_workspace_bytes(256, 0), 0);
  EXPECT_RC(w, (int)gtp_lm_head_workspace_bytes(INT64_MAX, 1000), 0);
  EXPECT_RC(w, gtp_lm_head_logprob_rows(HB, -1, 128, 128, WB, 1000, 128, T, 0, o, NULL, NULL, NULL,
                                        wsp, wsz, NULL), I);
  EXPECT_RC(w, gtp_lm_head_logprob_rows(HB, 256, 128, 128, WB, 0, 128, T, 0, o, NULL, NULL, NULL,
                                        wsp, wsz, NULL), I);
  EXPECT_RC(w, gtp_lm_head_logprob_rows(HB, 256, 0, 128, WB, 1000, 128, T, 0, o, NULL, NULL, NULL,
                                        wsp, wsz, NULL), I);
  EXPECT_RC(w, gtp_lm_head_logprob_rows(HB, 256, 128, 120, WB, 1000, 128, T, 0, o, NULL, NULL,
                                        NULL, wsp, wsz, NULL), I);
  EXPECT_RC(w, gtp_lm_head_logprob_rows(NULL, 256, 128, 128, WB, 1000, 128, T, 0, o, NULL, NULL,
                                        NULL, wsp, wsz, NULL), I);
  EXPECT_RC(w, gtp_lm_head_logprob_rows(HB, 256, 128, 128, WB, 1000, 128, NULL, 0, o, NULL, NULL,
                                        NULL, wsp, wsz, NULL), I);
  EXPECT_RC(w, gtp_lm_head_logprob_rows(HB, 256, 128, 128, WB, 1000, 128, T, 0, o, NULL, NULL,
                                        NULL, NULL, wsz, NULL), I);
  EXPECT_RC(w, gtp_lm_head_logprob_rows(HB, 256, 128, 128, WB, 1000, 128, T, 0, o, NULL, NULL,
                                        NULL, wsp, wsz - 1, NULL), I);
  EXPECT_RC(w, gtp_lm_head_logprob_rows(HB, 256, 192, 192, WB, 1000, 192, T, 0, o, NULL, NULL,
                                        NULL, wsp, wsz, NULL), X);  /* K % 128 */
  EXPECT_RC(w, gtp_lm_head_logprob_rows((const uint16_t*)(uintptr_t)0x18, 256, 128, 128, WB, 1000,
                                        128, T, 0, o, NULL, NULL, NULL, wsp, wsz, NULL), X);
  EXPECT_RC(w, gtp_lm_head_logprob_rows(HB, 256, 128, 1 << 22, WB, 1000, 128, T, 0, o, NULL, NULL,
                                        NULL, wsp, wsz, NULL), X);
  EXPECT_RC(w, gtp_lm_head_logprob_rows(HB, INT64_MAX, 128, 128, WB, 1000, 128, T, 0, o, NULL,
                                        NULL, NULL, wsp, wsz, NULL), X);
  EXPECT_RC(w, gtp_lm_head_logprob_rows(NULL, 0, 128, 128, NULL, 1000, 128, NULL, 0, NULL, NULL,
                                        NULL, NULL, NULL, 0, NULL), OK);

  float* LG = PH(float*);
  EXPECT_RC(w, gtp_lm_head_logprob_save_rows(HB, 256, 128, 128, WB, 1000, 128, T, 0, o, NULL,
                                             NULL, NULL, NULL, 256, wsp, wsz, NULL), I);
  EXPECT_RC(w, gtp_lm_head_logprob_save_rows(HB, 256, 128, 128, WB, 1000, 128, T, 0, o, NULL,
                                             NULL, NULL, LG, 255, wsp, wsz, NULL), I);
  EXPECT_RC(w, gtp_lm_head_logprob_save_rows(HB, 256, 128, 128, WB, 1000, 128, T, 0, o, NULL,
                                             NULL, NULL, (float*)(uintptr_t)0x1002, 256, wsp,
                                             wsz, NULL), X);
  EXPECT_RC(w, gtp_lm_head_logprob_save_rows(HB, 256, 128, 128, WB, 1000, 128, T, 0, o, NULL,
                                             NULL, NULL, LG, (int64_t)1 << 40, wsp, wsz, NULL), X);
  EXPECT_RC(w, gtp_lm_head_logprob_save_rows(HB, 256, 192, 192, WB, 1000, 192, T, 0, o, NULL,
                                             NULL, NULL, LG, 256, wsp, wsz, NULL), X);
  EXPECT_RC(w, gtp_lm_head_logprob_save_rows(HB, 256, 128, 128, WB, 1000, 128, T, 0, o, NULL,
                                             NULL, NULL, LG, 256, wsp, wsz - 1, NULL), I);
  EXPECT_RC(w, gtp_lm_head_logprob_save_rows(NULL, 0, 128, 128, NULL, 1000, 128, NULL, 0, NULL,
                                             NULL, NULL, NULL, NULL, 0, NULL, 0, NULL), OK);

  EXPECT_RC(w, gtp_softmax_grad_bf16_cols(F, 10, -1, 10, F, F, h, 10, NULL, 0, NULL), I);
  EXPECT_RC(w, gtp_softmax_grad_bf16_cols(F, 10, 4, 3, F, F, h, 10, NULL, 0, NULL), I);
  EXPECT_RC(w, gtp_softmax_grad_bf16_cols(F, 10, 4, 4, F, F, h, 3, NULL, 0, NULL), I);
  EXPECT_RC(w, gtp_softmax_grad_bf16_cols(F, 0, 4, 4, F, F, h, 4, NULL, 0, NULL), I);
  EXPECT_RC(w, gtp_softmax_grad_bf16_cols(F, 10, 4, 4, NULL, F, h, 4, NULL, 0, NULL), I);
  EXPECT_RC(w, gtp_softmax_grad_bf16_cols(F, 10, 4, 4, F, F, NULL, 4, NULL, 0, NULL), I);
  EXPECT_RC(w, gtp_softmax_grad_bf16_cols(F, 10, INT64_MAX, INT64_MAX, F, F, h, INT64_MAX, NULL, 0, NULL),
            X);
  EXPECT_RC(w, gtp_softmax_grad_bf16_cols(F, INT64_MAX, 4, 4, F, F, h, 4, NULL, 0, NULL), X);
  EXPECT_RC(w, gtp_softmax_grad_bf16_cols(NULL, 10, 0, 0, NULL, NULL, NULL, 0, NULL, 0, NULL), OK);
  /* the token-major output: its stride must hold V, and bound N * stride */
  EXPECT_RC(w, gtp_softmax_grad_bf16_cols(F, 10, 4, 4, F, F, NULL, 0, h, 9, NULL), I);
  EXPECT_RC(w, gtp_softmax_grad_bf16_cols(F, 10, 4, 4, F, F, h, 4, h, 9, NULL), I);
  EXPECT_RC(w, gtp_softmax_grad_bf16_cols(F, 10, 4, 4, F, F, NULL, 0, h, INT64_MAX, NULL), X);

  EXPECT_RC(w, strstr(gtp_version(), "gfx950") != NULL, 1);

  printf("C-ABI sanitizer checks: %d run, %d failed\n", g_checks, g_fails);
  return g_fails ? 1 : 0;
}
