// tokpath_common.h -- device helpers shared by the gfx950 token-path kernels.
//
// Wave64 reductions, logit loads (bf16 / fp16 / fp32, 16-byte vectors),
// order-preserving keys and the deterministic fixed-point exp (DETEXP_FIX)
// whose every fp32 step is one IEEE operation (the files are compiled with
// -ffp-contract=off), so host and device produce the same integers.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/graspo_tokpath.h"

namespace gtp {

constexpr int kWave = 64;
constexpr float kLog2e = 0x1.715476p+0f;
constexpr float kLn2 = 0x1.62e430p-1f;
constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kPosInf = __builtin_huge_valf();

// ------------------------------------------------------------ bit helpers

__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }

// bf16 pair packed in a uint32 -> two exact fp32 values
__device__ __forceinline__ float bf16_lo(uint32_t w) { return u2f(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return u2f(w & 0xFFFF0000u); }

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, h);
  return (float)v;
}

// Order-preserving 32-bit key of a (non-NaN) float: a < b  <=>  key(a) < key(b).
// -0 and +0 get different keys; callers canonicalise zeros first (y + 0.0f).
__device__ __forceinline__ uint32_t ord32(float f) {
  uint32_t u = f2u(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float unord32(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
  return u2f(u);
}

// 16-bit order-preserving key of a bf16 bit pattern.
__device__ __forceinline__ uint32_t ord16(uint32_t h) {
  return (h & 0x8000u) ? (~h & 0xFFFFu) : (h | 0x8000u);
}
__device__ __forceinline__ uint32_t unord16(uint32_t k) {
  return (k & 0x8000u) ? (k & 0x7FFFu) : (~k & 0xFFFFu);
}

// fp32 -> bf16 bit pattern rounded toward +inf (an upper bound), or toward
// -inf (a lower bound).  NaN never reaches these (callers pass maxima that
// skip NaN).
__device__ __forceinline__ uint32_t bf16_round_up(float f) {
  uint32_t u = f2u(f);
  uint32_t hi = u >> 16;
  if ((u & 0xFFFFu) == 0u) return hi;
  // positive: magnitude up; negative: magnitude down (truncate)
  return (u & 0x80000000u) ? hi : hi + 1u;
}
__device__ __forceinline__ uint32_t bf16_round_down(float f) {
  uint32_t u = f2u(f);
  uint32_t hi = u >> 16;
  if ((u & 0xFFFFu) == 0u) return hi;
  return (u & 0x80000000u) ? hi + 1u : hi;
}

// composite rank key: larger = earlier in the order (y desc, id asc)
__device__ __forceinline__ uint64_t rank_key(float y, int32_t id) {
  return ((uint64_t)ord32(y) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)id);
}
__device__ __forceinline__ int32_t rank_key_id(uint64_t k) {
  return (int32_t)(0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull));
}
__device__ __forceinline__ float rank_key_y(uint64_t k) { return unord32((uint32_t)(k >> 32)); }

// ------------------------------------------------- division by the temperature
// x / T rounded to nearest even, the IEEE quotient, for 2^-20 <= T <= 1024,
// with rT = RN(1 / T) and bh = RN(T 2^-25 (1 - 2^-20)) set once per call.
// q0 = RN(x rT) lies within 2 ulp of x / T; one correction with its fma
// residual, q = fma(x - q0 T, rT, q0) (Markstein's correction step), is
// almost always the rounded quotient.
// The check is exact whatever q is: with q = f 2^e (f in [0.5, 1)) and
// r = RN(x - q T) (one fma), |r| < bh 2^e gives |x - q T| < T ulp(q) / 2
// (r's own rounding is inside the 2^-20 margin, and with |q| >= 2^-60 it
// cannot underflow), so x / T lies strictly within half an ulp of q, and q
// is the rounded quotient whenever both neighbours of q lie ulp(q) away (q
// not a power of two).  Infinite or NaN x gives a NaN residual, q = 0 or a
// power of two fails the mantissa test, tiny q the exponent test: those
// tokens, and any other that fails (near-ties), take the division.
__device__ __forceinline__ float div_by_t(float x, float T, float rT, float bh) {
  const float q0 = x * rT;
  const float q = __builtin_fmaf(__builtin_fmaf(-q0, T, x), rT, q0);
  const float r = __builtin_fmaf(-q, T, x);
  const int e = __builtin_amdgcn_frexp_expf(q);
  // (bitwise: all three tests are evaluated, no branch between them)
  const bool ok = ((int)(__builtin_fabsf(r) < __builtin_ldexpf(bh, e)) & (int)(e >= -59) &
                   (int)((f2u(q) & 0x7FFFFFu) != 0u)) != 0;
  if (__builtin_expect(ok, 1)) return q;
  // (the empty asm keeps the division in its own block, off the common path)
  asm volatile("" ::: "memory");
  return x / T;
}
__host__ __device__ inline float div_by_t_bound(float T) { return T * 0x1p-25f * (1.0f - 0x1p-20f); }

// ------------------------------------------------------------ DETEXP_FIX
// round(e^d * 2^40) for d <= 0; the step list is the contract written out in
// include/graspo_tokpath.h and must not be reordered.  The final scaling by
// 2^s is branch-free: s >= 0 shifts left; s < 0 rounds half to even as
// (mant + 2^(sh-1) - 1 + lsb) >> sh with sh = -s clamped to [1, 26] (every
// sh >= 25 gives 0 for a 24-bit mant).  Equal to the plain two-branch form
// for every fp32 d <= 0 (checked over all of them).
__device__ __forceinline__ uint64_t detexp_fix(float d) {
  if (!(d >= -30.0f)) return 0ull;
  float n = __builtin_rintf(d * 0x1.715476p+0f);
  float r = __builtin_fmaf(-n, 0x1.62e4p-1f, d);
  r = __builtin_fmaf(-n, 0x1.7f7d1cp-20f, r);
  float p = 0x1.a01a02p-13f;
  p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
  p = __builtin_fmaf(p, r, 0x1.111112p-7f);
  p = __builtin_fmaf(p, r, 0x1.555556p-5f);
  p = __builtin_fmaf(p, r, 0x1.555556p-3f);
  p = __builtin_fmaf(p, r, 0x1p-1f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  const uint32_t pb = f2u(p);
  const uint32_t mant = (pb & 0x7FFFFFu) | 0x800000u;
  const int s = (int)((pb >> 23) & 0xFFu) - 150 + 40 + (int)n;
  int sh = -s;
  sh = sh < 1 ? 1 : (sh > 26 ? 26 : sh);
  const uint32_t q = (mant + ((1u << (sh - 1)) - 1u) + ((mant >> sh) & 1u)) >> sh;
  return s >= 0 ? (uint64_t)mant << s : (uint64_t)q;
}

// log_softmax(x)_i = x_i - m - ln s evaluated in fp64 and rounded once:
// |x - m| can be far above 2^24 (huge logits), where two fp32 roundings
// would differ from the correctly rounded value by an ulp.
__device__ __forceinline__ float raw_logprob(float x, float m, float ln_s) {
  return (float)(((double)x - (double)m) - (double)ln_s);
}

// floor(f * W) for fp32 f in [0, 1), exact (f = M * 2^-sh with M < 2^24).
__device__ __forceinline__ uint64_t floor_mul(float f, uint64_t W) {
  if (!(f > 0.0f)) return 0ull;
  uint32_t b = f2u(f);
  uint32_t E = (b >> 23) & 0xFFu;
  uint64_t M;
  int sh;
  if (E == 0) {
    M = b & 0x7FFFFFu;
    sh = 149;
  } else {
    M = (b & 0x7FFFFFu) | 0x800000u;
    sh = 150 - (int)E;
  }
  if (sh >= 128) return 0ull;
  unsigned __int128 prod = (unsigned __int128)M * (unsigned __int128)W;
  return (uint64_t)(prod >> sh);
}

// ------------------------------------------------------- wave reductions

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int o) {
  uint32_t lo = __shfl_xor((uint32_t)v, o, kWave);
  uint32_t hi = __shfl_xor((uint32_t)(v >> 32), o, kWave);
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t shfl_up_u64(uint64_t v, int o) {
  uint32_t lo = __shfl_up((uint32_t)v, o, kWave);
  uint32_t hi = __shfl_up((uint32_t)(v >> 32), o, kWave);
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    uint64_t w = shfl_xor_u64(v, o);
    v = w > v ? w : v;
  }
  return v;
}
// inclusive prefix sum over the 64 lanes
__device__ __forceinline__ uint64_t wave_incl_scan_u64(uint64_t v) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    uint64_t w = shfl_up_u64(v, o);
    if (lane >= o) v += w;
  }
  return v;
}

// Online log-sum-exp state in base-2 units: s = sum 2^{(x-m) log2e}.
struct LseState {
  float m;
  float s;
};
__device__ __forceinline__ LseState lse_merge(LseState a, LseState b) {
  float m = fmaxf(a.m, b.m);
  // NaN sums must survive the merge (they flag non-finite rows), also when
  // no finite value has been seen (a row of NaN and -inf only)
  if (a.s != a.s || b.s != b.s) return {m, __builtin_nanf("")};
  if (m == kNegInf) return {kNegInf, 0.0f};
  float sa = a.s == 0.0f ? 0.0f : a.s * __builtin_amdgcn_exp2f((a.m - m) * kLog2e);
  float sb = b.s == 0.0f ? 0.0f : b.s * __builtin_amdgcn_exp2f((b.m - m) * kLog2e);
  return {m, sa + sb};
}
__device__ __forceinline__ LseState wave_lse(LseState v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    LseState w{__shfl_xor(v.m, o, kWave), __shfl_xor(v.s, o, kWave)};
    v = lse_merge(v, w);
  }
  return v;
}

// --------------------------------------------------------------- loads
// A "group" is 8 consecutive logits: one 16-byte vector of bf16/fp16 or two
// of fp32.

template <typename T>
struct Elem;
template <>
struct Elem<uint16_t> {  // bf16 bit patterns
  static constexpr int kDtype = GTP_DTYPE_BF16;
  __device__ static __forceinline__ float get(const uint16_t* p, int64_t i) {
    return u2f((uint32_t)p[i] << 16);
  }
  __device__ static __forceinline__ void group(const uint16_t* p, float (&x)[8]) {
    uint4 v = *reinterpret_cast<const uint4*>(p);
    x[0] = bf16_lo(v.x); x[1] = bf16_hi(v.x);
    x[2] = bf16_lo(v.y); x[3] = bf16_hi(v.y);
    x[4] = bf16_lo(v.z); x[5] = bf16_hi(v.z);
    x[6] = bf16_lo(v.w); x[7] = bf16_hi(v.w);
  }
};
template <>
struct Elem<_Float16> {
  static constexpr int kDtype = GTP_DTYPE_F16;
  __device__ static __forceinline__ float get(const _Float16* p, int64_t i) {
    return (float)p[i];
  }
  __device__ static __forceinline__ void group(const _Float16* p, float (&x)[8]) {
    uint4 v = *reinterpret_cast<const uint4*>(p);
    uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      x[2 * k] = f16_to_f32((uint16_t)(w[k] & 0xFFFFu));
      x[2 * k + 1] = f16_to_f32((uint16_t)(w[k] >> 16));
    }
  }
};
template <>
struct Elem<float> {
  static constexpr int kDtype = GTP_DTYPE_F32;
  __device__ static __forceinline__ float get(const float* p, int64_t i) { return p[i]; }
  __device__ static __forceinline__ void group(const float* p, float (&x)[8]) {
    float4 a = *reinterpret_cast<const float4*>(p);
    float4 b = *reinterpret_cast<const float4*>(p + 4);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
  }
};

// Load group G (elements [8G, 8G+8)) of a row; elements >= V read as -inf.
// `vec_ok` says the row base is 16-byte aligned, so full groups use vector
// loads; otherwise every element is loaded on its own.
template <typename T>
__device__ __forceinline__ void load_group(const T* row, int64_t G, int64_t V, bool vec_ok,
                                           float (&x)[8]) {
  const int64_t e0 = G * 8;
  if (vec_ok && e0 + 8 <= V) {
    Elem<T>::group(row + e0, x);
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = (e0 + j < V) ? Elem<T>::get(row, e0 + j) : kNegInf;
  }
}

// Events that the next launch through launch_timed records at its start and
// end (hipExtLaunchKernelGGL takes them from the dispatch itself), set by
// gtp_time_next_launch; per host thread, cleared by the launch that uses them.
// Every call times as one launch: the top-p kernels run the row-wise path for
// the rows they cannot take inside the same launch.
struct LaunchEvents {
  hipEvent_t start, stop;
};
extern thread_local LaunchEvents g_next_launch_events;

template <typename Kernel, typename... Args>
inline void launch_timed(Kernel kernel, dim3 grid, dim3 block, hipStream_t s, Args... args) {
  LaunchEvents& e = g_next_launch_events;
  if (e.start && e.stop) {
    hipExtLaunchKernelGGL(kernel, grid, block, 0, s, e.start, e.stop, 0, args...);
    e = LaunchEvents{nullptr, nullptr};
  } else {
    hipLaunchKernelGGL(kernel, grid, block, 0, s, args...);
  }
}

__device__ __forceinline__ float max8(const float (&x)[8]) {
  float a = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
  float b = fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7]));
  return fmaxf(a, b);
}

}  // namespace gtp
