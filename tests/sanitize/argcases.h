/* Argument checks shared by the oracle's and the C-ABI library's sampler and
 * logprob entry points: every call here must be answered on the host, before
 * any memory behind a pointer is touched, with the same return code on both
 * sides (the pointers are placeholders that are never dereferenced). */
#ifndef GTP_SANITIZE_ARGCASES_H
#define GTP_SANITIZE_ARGCASES_H

#include <math.h>
#include <stdint.h>
#include <stdio.h>

#include "graspo_tokpath.h"

typedef int (*sample_fn)(const void* logits, int dtype, int64_t B, int64_t V, int64_t row_stride,
                         const int32_t* history, int64_t hist_len, int64_t hist_stride,
                         const uint32_t* allow_mask, int64_t mask_stride, const float* uniforms,
                         const gtp_sampler_params* params, const uint8_t* finished,
                         int64_t pad_token_id, int64_t* out_ids, float* out_logprob,
                         float* out_sampled_logprob, int32_t* out_kept, float* out_thresh_value,
                         int32_t* out_thresh_id, int32_t* out_status);

typedef int (*logprob_fn)(const void* logits, int dtype, int64_t N, int64_t V, int64_t row_stride,
                          const void* targets, int targets_int64, float* out_logprob,
                          float* out_entropy, int32_t* out_status);

static int g_checks = 0, g_fails = 0;

#define EXPECT_RC(who, call, want)                                                        \
  do {                                                                                    \
    const int got_ = (call);                                                              \
    ++g_checks;                                                                           \
    if (got_ != (want)) {                                                                 \
      fprintf(stderr, "%s:%d: [%s] %s returned %d, expected %d\n", __FILE__, __LINE__, who, \
              #call, got_, (int)(want));                                                  \
      ++g_fails;                                                                          \
    }                                                                                     \
  } while (0)

/* A non-null placeholder; a check that dereferenced it would crash. */
#define PH(T) ((T)(uintptr_t)0x10)

static void sample_arg_cases(sample_fn f, const char* who) {
  const gtp_sampler_params ok = {0.7f, 0, 0.9f, 1.0f};
  gtp_sampler_params p;
  const void* L = PH(const void*);
  int64_t* ids = PH(int64_t*);
  const float* U = PH(const float*);
  const uint32_t* M = PH(const uint32_t*);
  const int32_t* H = PH(const int32_t*);
  const int I = GTP_ERR_INVALID_ARGUMENT, X = GTP_ERR_UNSUPPORTED;
#define S(dt, B, V, rs, h, hl, hs, m, ms, u, pp, lg, oi) \
  f(lg, dt, B, V, rs, h, hl, hs, m, ms, u, pp, NULL, 0, oi, NULL, NULL, NULL, NULL, NULL, NULL)
  EXPECT_RC(who, S(1, 2, 100, 100, NULL, 0, 0, NULL, 0, U, NULL, L, ids), I);    /* no params */
  EXPECT_RC(who, S(1, -1, 100, 100, NULL, 0, 0, NULL, 0, U, &ok, L, ids), I);    /* B < 0 */
  EXPECT_RC(who, S(1, 2, 0, 0, NULL, 0, 0, NULL, 0, U, &ok, L, ids), I);         /* V = 0 */
  EXPECT_RC(who, S(1, 2, -5, 100, NULL, 0, 0, NULL, 0, U, &ok, L, ids), I);      /* V < 0 */
  EXPECT_RC(who, S(1, 2, 100, 99, NULL, 0, 0, NULL, 0, U, &ok, L, ids), I);      /* stride < V */
  EXPECT_RC(who, S(3, 2, 100, 100, NULL, 0, 0, NULL, 0, U, &ok, L, ids), I);     /* dtype */
  EXPECT_RC(who, S(-1, 2, 100, 100, NULL, 0, 0, NULL, 0, U, &ok, L, ids), I);    /* dtype */
  EXPECT_RC(who, S(1, 2, 100, 100, NULL, 0, 0, NULL, 0, U, &ok, NULL, ids), I);  /* no logits */
  EXPECT_RC(who, S(1, 2, 100, 100, NULL, 0, 0, NULL, 0, U, &ok, L, NULL), I);    /* no ids */
  p = ok; p.repetition_penalty = 0.0f;
  EXPECT_RC(who, S(1, 2, 100, 100, NULL, 0, 0, NULL, 0, U, &p, L, ids), I);
  p.repetition_penalty = -1.0f;
  EXPECT_RC(who, S(1, 2, 100, 100, NULL, 0, 0, NULL, 0, U, &p, L, ids), I);
  p.repetition_penalty = NAN;
  EXPECT_RC(who, S(1, 2, 100, 100, NULL, 0, 0, NULL, 0, U, &p, L, ids), I);
  EXPECT_RC(who, S(1, 2, 100, 100, NULL, 0, 0, M, 3, U, &ok, L, ids), I);        /* mask words */
  EXPECT_RC(who, S(1, 2, 100, 100, H, -1, 8, NULL, 0, U, &ok, L, ids), I);       /* hist_len < 0 */
  EXPECT_RC(who, S(1, 2, 100, 100, NULL, -1, 0, NULL, 0, U, &ok, L, ids), I);
  EXPECT_RC(who, S(1, 2, 100, 100, H, 5, 4, NULL, 0, U, &ok, L, ids), I);        /* hist stride */
  EXPECT_RC(who, S(1, 2, 100, 100, NULL, 0, 0, NULL, 0, NULL, &ok, L, ids), I);  /* no uniforms */
  EXPECT_RC(who, S(1, 2, GTP_SAMPLER_MAX_V + 1, GTP_SAMPLER_MAX_V + 1, NULL, 0, 0, NULL, 0, U,
                   &ok, L, ids), X);
  /* sizes at the edge of int64: rejected before any size arithmetic */
  EXPECT_RC(who, S(1, 2, INT64_MAX, INT64_MAX, NULL, 0, 0, M, 1, U, &ok, L, ids), X);
  EXPECT_RC(who, S(0, 2, INT64_MAX - 7, INT64_MAX, H, INT64_MAX, INT64_MAX, M, INT64_MAX, U, &ok,
                   L, ids), X);
  EXPECT_RC(who, S(1, (int64_t)1 << 31, 1000, 1000, NULL, 0, 0, NULL, 0, U, &ok, L, ids), X);
  EXPECT_RC(who, S(1, INT64_MAX, 151936, 151936, NULL, 0, 0, NULL, 0, U, &ok, L, ids), X);
  /* no rows: nothing to do, no pointers needed */
  EXPECT_RC(who, S(1, 0, 100, 100, NULL, 0, 0, NULL, 0, NULL, &ok, NULL, NULL), GTP_OK);
#undef S
}

static void logprob_arg_cases(logprob_fn f, const char* who) {
  const void* L = PH(const void*);
  const void* T = PH(const void*);
  float* o = PH(float*);
  const int I = GTP_ERR_INVALID_ARGUMENT, X = GTP_ERR_UNSUPPORTED;
  EXPECT_RC(who, f(L, 1, -1, 10, 10, T, 0, o, NULL, NULL), I);
  EXPECT_RC(who, f(L, 1, 4, 0, 0, T, 0, o, NULL, NULL), I);
  EXPECT_RC(who, f(L, 1, 4, 10, 9, T, 0, o, NULL, NULL), I);
  EXPECT_RC(who, f(NULL, 1, 4, 10, 10, T, 0, o, NULL, NULL), I);
  EXPECT_RC(who, f(L, 1, 4, 10, 10, NULL, 0, o, NULL, NULL), I);
  EXPECT_RC(who, f(L, 1, 4, 10, 10, T, 1, NULL, NULL, NULL), I);
  EXPECT_RC(who, f(L, 9, 4, 10, 10, T, 0, o, NULL, NULL), I);
  EXPECT_RC(who, f(L, 1, (int64_t)1 << 31, 10, 10, T, 0, o, NULL, NULL), X);
  EXPECT_RC(who, f(L, 1, INT64_MAX, INT64_MAX, INT64_MAX, T, 0, o, NULL, NULL), X);
  EXPECT_RC(who, f(NULL, 1, 0, 10, 10, NULL, 0, NULL, NULL, NULL), GTP_OK);
}

#endif
