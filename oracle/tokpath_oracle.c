/*
 * tokpath_oracle.c -- CPU oracle for the vocabulary-wide token path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * of the HIP path.  The product (graspo_amd) never calls it and has no CPU
 * fallback.
 *
 * A sort-based restatement of the sampler contract written out in
 * include/graspo_tokpath.h, which extends the reference's
 *   _next_token_from_logits  src/graspo/backends/graspoflow/tensor_utils.py:649-658
 *   _sample_next_token       src/graspo/backends/graspoflow/tensor_utils.py:671-683
 * and of the logprob / entropy statement
 *   sequence_log_probs_from_logits  src/graspo/core/graspo_loss.py:19-21
 *   _selected_token_log_probs_from_hidden  tensor_utils.py:167-186 (logit - lse)
 * The GPU kernels select with thresholds, histograms and candidate lists; this
 * file sorts the whole row, so the two share the contract, not the algorithm.
 *
 * Pins (tests/test_oracle_*.py): DETEXP against libm exp; the penalty against
 * transformers' RepetitionPenaltyLogitsProcessor; top-k sets against
 * torch.topk; the top-p cut and draw against an fp64 literal restatement of
 * tensor_utils.py:671-683 and against exhaustive uniform grids on tiny rows;
 * closed forms (uniform rows, single allowed token, top_k = 1, greedy);
 * logprob / entropy against torch.log_softmax in fp64.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math), so every
 * fp32 step is exactly one IEEE operation, as on the GPU.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "../include/graspo_tokpath.h"

/* ---------------------------------------------------------------- helpers */

static float u32_as_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, sizeof f);
  return f;
}

static uint32_t f32_as_u32(float f) {
  uint32_t u;
  memcpy(&u, &f, sizeof u);
  return u;
}

/* IEEE binary16 -> binary32, exact (written out so the oracle does not depend
 * on compiler support for _Float16). */
static float f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t man = h & 0x3FFu;
  if (exp == 0x1Fu) return u32_as_f32(sign | 0x7F800000u | (man << 13));
  if (exp != 0) return u32_as_f32(sign | ((exp + 112u) << 23) | (man << 13));
  if (man == 0) return u32_as_f32(sign);
  /* subnormal half: value = man * 2^-24, exact in fp32 */
  float v = (float)man * 0x1p-24f;
  return sign ? -v : v;
}

static float load_x(const void* logits, int dtype, int64_t idx) {
  if (dtype == GTP_DTYPE_F32) return ((const float*)logits)[idx];
  uint16_t h = ((const uint16_t*)logits)[idx];
  if (dtype == GTP_DTYPE_BF16) return u32_as_f32((uint32_t)h << 16);
  return f16_to_f32(h);
}

/* ------------------------------------------------------------- DETEXP_FIX */

/* Fixed-point weight of a logit d = y - m <= 0:  round(e^d * 2^40).
 * Cody-Waite reduction d = n ln2 + r (ln2 split in a 15-bit head, so n * head
 * is exact for |n| < 2^9, and an fp32 tail), Taylor polynomial of degree 7 for
 * e^r on |r| <= ln2/2 (truncation error < 6e-9), then an exact integer
 * rounding of p * 2^(n+40), ties to even.  Every fp32 step is one IEEE op. */
#define DX_LOG2E 0x1.715476p+0f
#define DX_LN2_HI 0x1.62e4p-1f
#define DX_LN2_LO 0x1.7f7d1cp-20f
#define DX_C7 0x1.a01a02p-13f /* 1/5040 */
#define DX_C6 0x1.6c16c2p-10f /* 1/720 */
#define DX_C5 0x1.111112p-7f  /* 1/120 */
#define DX_C4 0x1.555556p-5f  /* 1/24 */
#define DX_C3 0x1.555556p-3f  /* 1/6 */
#define DX_C2 0x1p-1f         /* 1/2 */
#define DX_FRAC_BITS 40

uint64_t gtp_oracle_detexp_fix(float d) {
  if (!(d >= -30.0f)) return 0; /* also catches -inf */
  float n = rintf(d * DX_LOG2E);
  float r = fmaf(-n, DX_LN2_HI, d);
  r = fmaf(-n, DX_LN2_LO, r);
  float p = DX_C7;
  p = fmaf(p, r, DX_C6);
  p = fmaf(p, r, DX_C5);
  p = fmaf(p, r, DX_C4);
  p = fmaf(p, r, DX_C3);
  p = fmaf(p, r, DX_C2);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  uint32_t pb = f32_as_u32(p);
  uint64_t mant = (uint64_t)((pb & 0x7FFFFFu) | 0x800000u);
  int e = (int)((pb >> 23) & 0xFFu) - 150; /* p = mant * 2^e */
  int s = e + DX_FRAC_BITS + (int)n;
  if (s >= 0) return mant << s;
  int sh = -s;
  if (sh > 25) return 0;
  uint64_t q = mant >> sh;
  uint64_t rem = mant & ((1ull << sh) - 1ull);
  uint64_t half = 1ull << (sh - 1);
  if (rem > half || (rem == half && (q & 1ull))) q += 1;
  return q;
}

/* floor(f * W) for fp32 f in [0, 1) and W < 2^64, exact. */
uint64_t gtp_oracle_floor_mul(float f, uint64_t W) {
  if (!(f > 0.0f)) return 0;
  int e;
  float fr = frexpf(f, &e);                      /* f = fr * 2^e, fr in [0.5, 1) */
  uint64_t M = (uint64_t)ldexpf(fr, 24);         /* exact 24-bit integer */
  int sh = 24 - e;                               /* f = M * 2^-sh, sh >= 24 */
  if (sh >= 128) return 0;
  unsigned __int128 prod = (unsigned __int128)M * (unsigned __int128)W;
  return (uint64_t)(prod >> sh);
}

/* --------------------------------------------------------------- sampler */

typedef struct {
  float y;
  int32_t id;
} okey;

/* (y desc, id asc) */
static int okey_before(const okey* a, const okey* b) {
  if (a->y != b->y) return a->y > b->y;
  return a->id < b->id;
}

static int okey_cmp(const void* pa, const void* pb) {
  const okey* a = (const okey*)pa;
  const okey* b = (const okey*)pb;
  if (okey_before(a, b)) return -1;
  if (okey_before(b, a)) return 1;
  return 0;
}

/* Move the k first-in-order elements of v[0..n) to v[0..k) (any order). */
static void okey_select(okey* v, int64_t n, int64_t k) {
  int64_t lo = 0, hi = n - 1;
  while (lo < hi) {
    okey piv = v[lo + (hi - lo) / 2];
    int64_t i = lo, j = hi;
    while (i <= j) {
      while (okey_before(&v[i], &piv)) i++;
      while (okey_before(&piv, &v[j])) j--;
      if (i <= j) {
        okey t = v[i];
        v[i] = v[j];
        v[j] = t;
        i++;
        j--;
      }
    }
    if (k - 1 <= j)
      hi = j;
    else if (k - 1 >= i)
      lo = i;
    else
      break;
  }
}

static void write_bad_row(int64_t b, int32_t status, const uint8_t* finished,
                          int64_t pad_token_id, int64_t* out_ids,
                          float* out_logprob, float* out_sampled_logprob,
                          int32_t* out_kept, float* out_thresh_value,
                          int32_t* out_thresh_id, int32_t* out_status) {
  out_ids[b] = (finished && finished[b]) ? pad_token_id : -1;
  if (out_logprob) out_logprob[b] = NAN;
  if (out_sampled_logprob) out_sampled_logprob[b] = NAN;
  if (out_kept) out_kept[b] = 0;
  if (out_thresh_value) out_thresh_value[b] = 0.0f;
  if (out_thresh_id) out_thresh_id[b] = -1;
  if (out_status) out_status[b] = status;
}

int gtp_oracle_sample_rows(const void* logits, int dtype, int64_t B, int64_t V,
                           int64_t row_stride, const int32_t* history,
                           int64_t hist_len, int64_t hist_stride,
                           const uint32_t* allow_mask, int64_t mask_stride,
                           const float* uniforms,
                           const gtp_sampler_params* params,
                           const uint8_t* finished, int64_t pad_token_id,
                           int64_t* out_ids, float* out_logprob,
                           float* out_sampled_logprob, int32_t* out_kept,
                           float* out_thresh_value, int32_t* out_thresh_id,
                           int32_t* out_status) {
  if (!params || B < 0 || V <= 0 || row_stride < V || (B > 0 && (!logits || !out_ids)))
    return GTP_ERR_INVALID_ARGUMENT;
  if (dtype != GTP_DTYPE_F32 && dtype != GTP_DTYPE_BF16 && dtype != GTP_DTYPE_F16)
    return GTP_ERR_INVALID_ARGUMENT;
  if (!(params->repetition_penalty > 0.0f)) return GTP_ERR_INVALID_ARGUMENT;
  if (V > GTP_SAMPLER_MAX_V || B > 0x7FFFFFFFll) return GTP_ERR_UNSUPPORTED;
  if (allow_mask && mask_stride < (V + 31) / 32) return GTP_ERR_INVALID_ARGUMENT;
  if (hist_len < 0) return GTP_ERR_INVALID_ARGUMENT;
  if (history && hist_len > 0 && hist_stride < hist_len) return GTP_ERR_INVALID_ARGUMENT;
  const int greedy = !(params->temperature > 0.0f);
  if (!greedy && B > 0 && !uniforms) return GTP_ERR_INVALID_ARGUMENT;
  const float Tc = params->temperature > 1e-6f ? params->temperature : 1e-6f;
  const float rho = params->repetition_penalty;
  const int use_pen = history && hist_len > 0 && rho != 1.0f;

  okey* keys = (okey*)malloc((size_t)V * sizeof(okey));
  uint8_t* pen = (uint8_t*)malloc((size_t)V);
  uint64_t* w = (uint64_t*)malloc((size_t)V * sizeof(uint64_t));
  if (!keys || !pen || !w) {
    free(keys);
    free(pen);
    free(w);
    return GTP_ERR_UNSUPPORTED;
  }

  for (int64_t b = 0; b < B; ++b) {
    const int64_t base = b * row_stride;
    /* raw row: non-finite check and log-sum-exp (fp64) */
    int nonfinite = 0;
    double M = -INFINITY;
    for (int64_t i = 0; i < V; ++i) {
      float x = load_x(logits, dtype, base + i);
      if (isnan(x) || x == INFINITY) nonfinite = 1;
      if (x > M) M = x;
    }
    double S = 0.0;
    if (!nonfinite)
      for (int64_t i = 0; i < V; ++i) S += exp((double)load_x(logits, dtype, base + i) - M);

    int bad_hist = 0;
    memset(pen, 0, (size_t)V);
    if (history && hist_len > 0) {
      for (int64_t j = 0; j < hist_len; ++j) {
        int32_t h = history[b * hist_stride + j];
        if (h >= V) bad_hist = 1;
        else if (h >= 0) pen[h] = 1;
      }
    }
    const float u = greedy ? 0.0f : uniforms[b];
    int32_t status = GTP_ROW_OK;
    if (greedy) {
      /* T <= 0 is the reference's logits.argmax(dim=-1) (tensor_utils.py:658)
       * over the allowed tokens' penalised logits: a NaN beats every value
       * and +inf every finite one (torch's argmax propagates NaN), ties go
       * to the lowest id, and a row whose allowed tokens are all -inf
       * returns the first of them.  Only a row with no allowed token at all
       * (or a bad history id) has no answer. */
      if (bad_hist) {
        write_bad_row(b, GTP_ROW_BAD_HISTORY, finished, pad_token_id, out_ids, out_logprob,
                      out_sampled_logprob, out_kept, out_thresh_value, out_thresh_id,
                      out_status);
        continue;
      }
      int64_t best = -1;
      float by = 0.0f;
      for (int64_t i = 0; i < V; ++i) {
        if (allow_mask && !((allow_mask[b * mask_stride + (i >> 5)] >> (i & 31)) & 1u))
          continue;
        const float x = load_x(logits, dtype, base + i);
        float y = x;
        if (use_pen && pen[i]) y = (x < 0.0f) ? x * rho : x / rho;
        y = y + 0.0f;
        if (best < 0 || (!isnan(by) && (isnan(y) || y > by))) {
          best = i;
          by = y;
        }
      }
      if (best < 0) {
        write_bad_row(b, GTP_ROW_EMPTY, finished, pad_token_id, out_ids, out_logprob,
                      out_sampled_logprob, out_kept, out_thresh_value, out_thresh_id,
                      out_status);
        continue;
      }
      const double xb = load_x(logits, dtype, base + best);
      out_ids[b] = (finished && finished[b]) ? pad_token_id : best;
      if (out_logprob) out_logprob[b] = nonfinite ? NAN : (float)(xb - M - log(S));
      if (out_sampled_logprob) out_sampled_logprob[b] = 0.0f;
      if (out_kept) out_kept[b] = 1;
      if (out_thresh_value) out_thresh_value[b] = by;
      if (out_thresh_id) out_thresh_id[b] = (int32_t)best;
      if (out_status) out_status[b] = GTP_ROW_OK;
      continue;
    }
    if (nonfinite) status = GTP_ROW_NONFINITE;
    else if (bad_hist) status = GTP_ROW_BAD_HISTORY;
    else if (!greedy && !(u >= 0.0f && u < 1.0f)) status = GTP_ROW_BAD_UNIFORM;
    if (status != GTP_ROW_OK) {
      write_bad_row(b, status, finished, pad_token_id, out_ids, out_logprob,
                    out_sampled_logprob, out_kept, out_thresh_value, out_thresh_id,
                    out_status);
      continue;
    }

    /* penalty, mask, temperature */
    int64_t n = 0;
    for (int64_t i = 0; i < V; ++i) {
      if (allow_mask && !((allow_mask[b * mask_stride + (i >> 5)] >> (i & 31)) & 1u))
        continue;
      float x = load_x(logits, dtype, base + i);
      float xp = x;
      if (use_pen && pen[i]) xp = (x < 0.0f) ? x * rho : x / rho;
      float y = greedy ? xp : xp / Tc;
      y = y + 0.0f; /* -0 -> +0: the two zeros tie */
      if (y > -INFINITY) {
        keys[n].y = y;
        keys[n].id = (int32_t)i;
        n++;
      }
    }
    if (n == 0) {
      write_bad_row(b, GTP_ROW_EMPTY, finished, pad_token_id, out_ids, out_logprob,
                    out_sampled_logprob, out_kept, out_thresh_value, out_thresh_id,
                    out_status);
      continue;
    }
    /* order: (y desc, id asc) */
    int64_t nk = n;
    if (greedy)
      nk = 1;
    else if (params->top_k > 0 && (int64_t)params->top_k < n)
      nk = params->top_k;
    if (nk < n) okey_select(keys, n, nk);
    qsort(keys, (size_t)nk, sizeof(okey), okey_cmp);
    if (keys[0].y == INFINITY) {
      write_bad_row(b, GTP_ROW_NONFINITE, finished, pad_token_id, out_ids,
                    out_logprob, out_sampled_logprob, out_kept, out_thresh_value,
                    out_thresh_id, out_status);
      continue;
    }

    int64_t id;
    int64_t R;
    double sampled_lp;
    if (greedy) {
      id = keys[0].id;
      R = 1;
      sampled_lp = 0.0;
    } else {
      const float m = keys[0].y;
      uint64_t Wk = 0;
      for (int64_t r = 0; r < nk; ++r) {
        w[r] = gtp_oracle_detexp_fix(keys[r].y - m);
        Wk += w[r];
      }
      R = nk;
      if (params->top_p > 0.0f && params->top_p < 1.0f) {
        const uint64_t F = gtp_oracle_floor_mul(params->top_p, Wk);
        uint64_t Sr = 0;
        R = 0;
        while (R < nk && Sr <= F) {
          Sr += w[R];
          R++;
        }
      }
      uint64_t Wp = 0;
      for (int64_t r = 0; r < R; ++r) Wp += w[r];
      const uint64_t U = gtp_oracle_floor_mul(u, Wp);
      uint64_t Sr = 0;
      int64_t rs = 0;
      for (; rs < R; ++rs) {
        Sr += w[rs];
        if (Sr > U) break;
      }
      id = keys[rs].id;
      sampled_lp = log((double)w[rs] / (double)Wp);
    }
    const double xid = load_x(logits, dtype, base + id);
    out_ids[b] = (finished && finished[b]) ? pad_token_id : id;
    if (out_logprob) out_logprob[b] = (float)(xid - M - log(S));
    if (out_sampled_logprob) out_sampled_logprob[b] = (float)sampled_lp;
    if (out_kept) out_kept[b] = (int32_t)R;
    if (out_thresh_value) out_thresh_value[b] = keys[R - 1].y;
    if (out_thresh_id) out_thresh_id[b] = keys[R - 1].id;
    if (out_status) out_status[b] = GTP_ROW_OK;
  }
  free(keys);
  free(pen);
  free(w);
  return GTP_OK;
}

/* -------------------------------------------------------- logprob/entropy */

static int64_t load_target(const void* targets, int targets_int64, int64_t n) {
  return targets_int64 ? ((const int64_t*)targets)[n] : (int64_t)((const int32_t*)targets)[n];
}

int gtp_oracle_logprob_entropy_rows(const void* logits, int dtype, int64_t N,
                                    int64_t V, int64_t row_stride,
                                    const void* targets, int targets_int64,
                                    float* out_logprob, float* out_entropy,
                                    int32_t* out_status) {
  if (N < 0 || V <= 0 || row_stride < V || (N > 0 && (!logits || !targets || !out_logprob)))
    return GTP_ERR_INVALID_ARGUMENT;
  if (dtype != GTP_DTYPE_F32 && dtype != GTP_DTYPE_BF16 && dtype != GTP_DTYPE_F16)
    return GTP_ERR_INVALID_ARGUMENT;
  if (N > 0x7FFFFFFFll) return GTP_ERR_UNSUPPORTED;
  for (int64_t r = 0; r < N; ++r) {
    const int64_t base = r * row_stride;
    double M = -INFINITY;
    int has_nan = 0;
    for (int64_t i = 0; i < V; ++i) {
      float x = load_x(logits, dtype, base + i);
      if (isnan(x)) has_nan = 1;
      if (x > M) M = x;
    }
    double S = 0.0, T = 0.0;
    for (int64_t i = 0; i < V; ++i) {
      double d = (double)load_x(logits, dtype, base + i) - M;
      double e = exp(d);
      S += e;
      if (e > 0.0) T += e * d;
    }
    if (has_nan) S = NAN;
    const int64_t t = load_target(targets, targets_int64, r);
    const double lse = M + log(S);
    if (t < 0 || t >= V) {
      out_logprob[r] = NAN;
      if (out_status) out_status[r] = GTP_ROW_BAD_TARGET;
    } else {
      out_logprob[r] = (float)((double)load_x(logits, dtype, base + t) - lse);
      if (out_status) out_status[r] = GTP_ROW_OK;
    }
    if (out_entropy) out_entropy[r] = (float)(log(S) - T / S);
  }
  return GTP_OK;
}

const char* gtp_oracle_version(void) { return "graspo_tokpath oracle 0.1 (cpu)"; }
