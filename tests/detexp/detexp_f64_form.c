/* Checks the fp64 evaluation form of DETEXP_FIX that the fp32 top-p kernel
 * uses (graspo_amd/csrc/tokpath_sampler_topp32.h, detexp_fix_f64): the
 * contract's fp32 steps to p and n, then rint(p * 2^(n + 40)) in fp64, with
 * d clamped at -30.5 -- against the oracle's integer form
 * (oracle/tokpath_oracle.c, gtp_oracle_detexp_fix) on fp32 values of d in
 * [-31, 0]: every `stride`-th one, and every value within 2^-8 of the
 * cutoff -30 and of the points where n changes near it.
 * Usage: detexp_f64_form [stride]   (stride 1: every fp32 value, ~1 min)
 * Exit status 0 when every value agrees. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

uint64_t gtp_oracle_detexp_fix(float d);

static float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static double f64_form(float d) {
  d = d < -30.5f ? -30.5f : d;
  const float n = rintf(d * 0x1.715476p+0f);
  float r = fmaf(-n, 0x1.62e4p-1f, d);
  r = fmaf(-n, 0x1.7f7d1cp-20f, r);
  float p = 0x1.a01a02p-13f;
  p = fmaf(p, r, 0x1.6c16c2p-10f);
  p = fmaf(p, r, 0x1.111112p-7f);
  p = fmaf(p, r, 0x1.555556p-5f);
  p = fmaf(p, r, 0x1.555556p-3f);
  p = fmaf(p, r, 0x1p-1f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return rint(ldexp((double)p, (int)n + 40));
}

static uint64_t bad = 0, checked = 0;

static void check(float d) {
  const uint64_t a = gtp_oracle_detexp_fix(d);
  const double b = f64_form(d);
  ++checked;
  if ((double)a != b) {
    if (bad < 5) printf("mismatch d=%a oracle=%llu f64=%.1f\n", d, (unsigned long long)a, b);
    ++bad;
  }
}

int main(int argc, char** argv) {
  const uint32_t stride = argc > 1 ? (uint32_t)strtoul(argv[1], NULL, 10) : 509u;
  const uint32_t top = 0x41F80000u; /* 31.0 */
  for (uint32_t m = 0; m <= top; m += stride) check(u2f(0x80000000u | m));
  /* dense windows: the cutoff, and the n steps (d = k ln 2 / 2 near -30) */
  const float centers[] = {-30.0f, -30.5f, -29.8f, -29.46f, -28.76f, -27.73f, -0.3466f, -0.0078f};
  for (unsigned c = 0; c < sizeof centers / sizeof centers[0]; ++c) {
    const float lo = centers[c] - 0x1p-8f, hi = centers[c] + 0x1p-8f;
    for (float d = lo; d <= hi && d <= 0.0f; d = nextafterf(d, 1.0f)) check(d);
  }
  printf("checked %llu values, %llu mismatches\n", (unsigned long long)checked,
         (unsigned long long)bad);
  return bad != 0;
}
