/* The CPU oracle under AddressSanitizer and UndefinedBehaviorSanitizer: the
 * argument checks, then the sampler and logprob rows over small vocabularies
 * (1 to 1000 tokens, ragged mask words, padded and unpadded rows, every
 * dtype, NaN / +-inf / all--inf rows, histories with padding and bad ids,
 * finished rows, bad uniforms, greedy, top-k and top-p) with every input in
 * a buffer of exactly its documented size, so that any read past a row, a
 * mask word or a history ends the run.  Outputs are checked against the
 * contract's invariants. */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "argcases.h"

int gtp_oracle_sample_rows(const void*, int, int64_t, int64_t, int64_t, const int32_t*, int64_t,
                           int64_t, const uint32_t*, int64_t, const float*,
                           const gtp_sampler_params*, const uint8_t*, int64_t, int64_t*, float*,
                           float*, int32_t*, float*, int32_t*, int32_t*);
int gtp_oracle_logprob_entropy_rows(const void*, int, int64_t, int64_t, int64_t, const void*, int,
                                    float*, float*, int32_t*);
uint64_t gtp_oracle_detexp_fix(float);
uint64_t gtp_oracle_floor_mul(float, uint64_t);

static uint64_t g_rng = 0x9E3779B97F4A7C15ull;
static uint64_t rnd(void) {
  g_rng ^= g_rng << 13;
  g_rng ^= g_rng >> 7;
  g_rng ^= g_rng << 17;
  return g_rng;
}
static float frand(void) { return (float)(rnd() >> 40) * 0x1p-24f; } /* [0, 1) */

static uint32_t f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

/* fp32 -> fp16 bits, rounding toward zero (inputs stay in the normal range
 * or are +-inf / NaN). */
static uint16_t to_f16(float f) {
  const uint32_t u = f32_bits(f);
  const uint16_t s = (uint16_t)((u >> 16) & 0x8000u);
  if (f != f) return 0x7E00u;
  const float a = f < 0 ? -f : f;
  if (a >= 65520.0f) return s | 0x7C00u;
  if (a < 0x1p-14f) return s;
  const int e = (int)((u >> 23) & 0xFF) - 127 + 15;
  return s | (uint16_t)(e << 10) | (uint16_t)((u >> 13) & 0x3FFu);
}

/* A [B, V] row block with row_stride elements between rows, exactly
 * (B - 1) * row_stride + V elements long. */
static void* make_rows(int dtype, int64_t B, int64_t V, int64_t rs, int kind) {
  const int64_t n = (B - 1) * rs + V;
  const size_t es = dtype == GTP_DTYPE_F32 ? 4 : 2;
  unsigned char* p = (unsigned char*)malloc((size_t)n * es);
  for (int64_t b = 0; b < B; ++b)
    for (int64_t i = 0; i < rs && b * rs + i < n; ++i) {
      float x = (frand() - 0.5f) * 8.0f;
      if (kind == 1 && i == V / 2) x = NAN;
      if (kind == 2 && i == V - 1) x = INFINITY;
      if (kind == 3) x = -INFINITY;
      if (kind == 4 && (i & 1)) x = -INFINITY;
      if (kind == 5) x = (float)(int)(frand() * 3.0f); /* ties */
      if (i >= V) x = 1e30f;                          /* padding must be ignored */
      const int64_t k = b * rs + i;
      if (dtype == GTP_DTYPE_F32) ((float*)p)[k] = x;
      else if (dtype == GTP_DTYPE_BF16) ((uint16_t*)p)[k] = (uint16_t)(f32_bits(x) >> 16);
      else ((uint16_t*)p)[k] = to_f16(x);
    }
  return p;
}

static int allowed(const uint32_t* mask, int64_t ms, int64_t b, int64_t i) {
  return !mask || ((mask[b * ms + (i >> 5)] >> (i & 31)) & 1u);
}

#define CHECK(c)                                                              \
  do {                                                                        \
    ++g_checks;                                                               \
    if (!(c)) {                                                               \
      fprintf(stderr, "%s:%d: check failed: %s (V=%lld b=%lld)\n", __FILE__, \
              __LINE__, #c, (long long)V, (long long)b);                      \
      ++g_fails;                                                              \
    }                                                                         \
  } while (0)

static void run_sampler_case(int dtype, int64_t B, int64_t V, int64_t rs, int kind, int masked,
                             int64_t hl, const gtp_sampler_params* p, int with_finished) {
  void* x = make_rows(dtype, B, V, rs, kind);
  const int64_t mw = (V + 31) / 32, ms = mw + (B > 1 ? 1 : 0);
  uint32_t* mask = NULL;
  if (masked) {
    mask = (uint32_t*)malloc((size_t)((B - 1) * ms + mw) * 4);
    for (int64_t k = 0; k < (B - 1) * ms + mw; ++k)
      mask[k] = masked == 2 ? 0u : (uint32_t)rnd();
  }
  int32_t* hist = NULL;
  const int64_t hs = hl + 3;
  if (hl > 0) {
    hist = (int32_t*)malloc((size_t)((B - 1) * hs + hl) * 4);
    for (int64_t k = 0; k < (B - 1) * hs + hl; ++k)
      hist[k] = (int32_t)(rnd() % (uint64_t)(V + 1)) - 1; /* -1 .. V-1 */
    if (B > 2) hist[2 * hs] = (int32_t)V;               /* row 2: a bad id */
  }
  float* u = (float*)malloc((size_t)B * 4);
  for (int64_t b = 0; b < B; ++b) u[b] = frand();
  if (B > 1) u[1] = 0x1.fffffep-1f;
  if (B > 3) u[3] = 1.0f; /* bad uniform */
  uint8_t* fin = NULL;
  if (with_finished) {
    fin = (uint8_t*)malloc((size_t)B);
    for (int64_t b = 0; b < B; ++b) fin[b] = (uint8_t)(b % 2);
  }
  int64_t* ids = (int64_t*)malloc((size_t)B * 8);
  float *lp = (float*)malloc((size_t)B * 4), *slp = (float*)malloc((size_t)B * 4);
  float* tv = (float*)malloc((size_t)B * 4);
  int32_t *kept = (int32_t*)malloc((size_t)B * 4), *tid = (int32_t*)malloc((size_t)B * 4);
  int32_t* st = (int32_t*)malloc((size_t)B * 4);
  const int rc = gtp_oracle_sample_rows(x, dtype, B, V, rs, hist, hl, hs, mask, ms, u, p, fin, -7,
                                        ids, lp, slp, kept, tv, tid, st);
  int64_t b = -1;
  CHECK(rc == GTP_OK);
  const int greedy = !(p->temperature > 0.0f);
  for (b = 0; b < B; ++b) {
    CHECK(st[b] >= GTP_ROW_OK && st[b] <= GTP_ROW_BAD_UNIFORM);
    const int fb = fin && fin[b];
    if (st[b] != GTP_ROW_OK) {
      CHECK(ids[b] == (fb ? -7 : -1));
      CHECK(kept[b] == 0 && tid[b] == -1);
      continue;
    }
    const int64_t id = tid[b];
    CHECK(id >= 0 && id < V && allowed(mask, ms, b, id));
    CHECK(kept[b] >= 1 && kept[b] <= V);
    if (!fb) CHECK(ids[b] >= 0 && ids[b] < V && allowed(mask, ms, b, ids[b]));
    else CHECK(ids[b] == -7);
    if (greedy) CHECK(kept[b] == 1 && slp[b] == 0.0f);
    else CHECK(slp[b] <= 0.0f);
    if (p->top_k > 0 && !greedy) CHECK(kept[b] <= p->top_k);
    CHECK(!(lp[b] > 0.0f));
  }
  free(x);
  free(mask);
  free(hist);
  free(u);
  free(fin);
  free(ids);
  free(lp);
  free(slp);
  free(tv);
  free(kept);
  free(tid);
  free(st);
}

static void run_logprob_case(int dtype, int64_t N, int64_t V, int64_t rs, int kind, int t64) {
  void* x = make_rows(dtype, N, V, rs, kind);
  void* t = malloc((size_t)N * (t64 ? 8 : 4));
  for (int64_t r = 0; r < N; ++r) {
    int64_t v = (int64_t)(rnd() % (uint64_t)V);
    if (r == 1) v = -1;
    if (r == 2) v = V;
    if (t64) ((int64_t*)t)[r] = v;
    else ((int32_t*)t)[r] = (int32_t)v;
  }
  float *lp = (float*)malloc((size_t)N * 4), *ent = (float*)malloc((size_t)N * 4);
  int32_t* st = (int32_t*)malloc((size_t)N * 4);
  const int rc = gtp_oracle_logprob_entropy_rows(x, dtype, N, V, rs, t, t64, lp, ent, st);
  int64_t b = -1;
  CHECK(rc == GTP_OK);
  for (b = 0; b < N; ++b) {
    if (b == 1 || b == 2) {
      CHECK(st[b] == GTP_ROW_BAD_TARGET && lp[b] != lp[b]);
      continue;
    }
    CHECK(st[b] == GTP_ROW_OK);
    if (kind == 0) {
      CHECK(lp[b] <= 0.0f);
      CHECK(ent[b] >= -1e-6f && ent[b] <= logf((float)V) + 1e-4f);
    }
  }
  free(x);
  free(t);
  free(lp);
  free(ent);
  free(st);
}

static int sample_oracle(const void* a, int b, int64_t c, int64_t d, int64_t e, const int32_t* f,
                         int64_t g, int64_t h, const uint32_t* i, int64_t j, const float* k,
                         const gtp_sampler_params* l, const uint8_t* m, int64_t n, int64_t* o,
                         float* p, float* q, int32_t* r, float* s, int32_t* t, int32_t* u) {
  return gtp_oracle_sample_rows(a, b, c, d, e, f, g, h, i, j, k, l, m, n, o, p, q, r, s, t, u);
}

int main(void) {
  sample_arg_cases(sample_oracle, "oracle sampler");
  logprob_arg_cases(gtp_oracle_logprob_entropy_rows, "oracle logprob");

  /* DETEXP_FIX and floor_mul at their edges */
  {
    const int64_t V = 0, b = 0;
    const float ds[] = {0.0f, -0.0f, -1e-45f, -0x1p-126f, -1.0f, -29.999998f, -30.0f,
                        -30.000002f, -INFINITY, NAN, -1e30f};
    uint64_t prev = UINT64_MAX;
    for (size_t k = 0; k < sizeof ds / sizeof ds[0]; ++k) {
      const uint64_t w = gtp_oracle_detexp_fix(ds[k]);
      if (ds[k] == ds[k]) {
        CHECK(w <= prev);
        prev = w;
      }
      CHECK(w <= ((uint64_t)1 << 40));
    }
    CHECK(gtp_oracle_detexp_fix(0.0f) == ((uint64_t)1 << 40));
    CHECK(gtp_oracle_detexp_fix(NAN) == 0);
    CHECK(gtp_oracle_floor_mul(0.5f, UINT64_MAX) == UINT64_MAX / 2);
    CHECK(gtp_oracle_floor_mul(0x1.fffffep-1f, 0) == 0);
    CHECK(gtp_oracle_floor_mul(0x1.fffffep-1f, UINT64_MAX) < UINT64_MAX);
    CHECK(gtp_oracle_floor_mul(0.0f, 12345) == 0 && gtp_oracle_floor_mul(NAN, 7) == 0);
  }

  static const int64_t vs[] = {1, 2, 31, 32, 33, 100, 1000};
  const gtp_sampler_params ps[] = {
      {0.0f, 0, 1.0f, 1.0f},  {0.0f, 0, 1.0f, 1.3f}, {0.7f, 0, 0.9f, 1.0f},
      {1.0f, 5, 1.0f, 0.7f},  {1.5f, 1, 0.5f, 2.0f}, {0.3f, 2000, 0.99f, 1.1f},
      {1e-9f, 0, 0.5f, 1.0f}, {1e4f, 3, 0.0f, 1.0f},
  };
  for (size_t vi = 0; vi < sizeof vs / sizeof vs[0]; ++vi)
    for (int dtype = 0; dtype < 3; ++dtype)
      for (int kind = 0; kind < 6; ++kind) {
        const int64_t V = vs[vi];
        const gtp_sampler_params* p = &ps[(vi + (size_t)kind + (size_t)dtype) % 8];
        run_sampler_case(dtype, 5, V, V, kind, (kind + (int)vi) % 3, (kind & 1) ? 17 : 0, p,
                         kind == 2);
        run_sampler_case(dtype, 1, V, V, kind, kind % 2, 0, p, 0);
        run_sampler_case(dtype, 3, V, V + 5, kind, 1, 4, &ps[(size_t)kind % 8], 1);
        run_logprob_case(dtype, 4, V, V + (kind & 1) * 3, kind, kind & 1);
      }
  /* no rows */
  {
    const gtp_sampler_params p = {0.7f, 0, 0.9f, 1.0f};
    EXPECT_RC("oracle sampler", gtp_oracle_sample_rows(NULL, 1, 0, 10, 10, NULL, 0, 0, NULL, 0,
                                                       NULL, &p, NULL, 0, NULL, NULL, NULL, NULL,
                                                       NULL, NULL, NULL),
              GTP_OK);
  }

  printf("oracle sanitizer checks: %d run, %d failed\n", g_checks, g_fails);
  return g_fails ? 1 : 0;
}
