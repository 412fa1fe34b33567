// tokpath_stream.h -- the streaming core shared by the gfx950 token-path kernels.
//
// A row of logits is read once, as 16-byte vectors (8 bf16 / 8 fp16 / 4 fp32
// elements), NG vectors per thread per step.  Steps are double-buffered in
// registers: the loads of step i+1 are issued before step i is folded, so
// every wave keeps NG x 16 bytes per lane in flight while its VALU work runs.
// Everything here is force-inlined so the compiler sees global (not flat)
// pointers and can count outstanding loads exactly.
//
// The per-element VALU budget is what bounds these kernels on MI355X: 8 TB/s
// of bf16 is 4 T elements/s, against about 39 T VALU lane-slots/s (256 CUs x
// 64 lanes x 2.4 GHz), i.e. about 10 issue slots per element (v_exp_f32 alone
// takes 4).  The
// fold below spends: 1 convert, 0.5 max (v_max3 on raw values, no
// canonicalisation), 1 fma, 1 exp, 1 add (+2 for the entropy term).  NaN and
// +inf are not tested per element: a NaN logit makes exp2(d) NaN and a +inf
// logit makes d = inf - inf = NaN, so either poisons the running sum, which
// the caller reports as a non-finite row.
#pragma once

#include "tokpath_common.h"

namespace gtp {

// native 4 x u32 vector (what a 16-byte global load returns)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// max of three floats without the IEEE canonicalisation the compiler inserts
// around fmaxf of bit-cast values (v_max3_f32 ignores quiet NaN inputs; a NaN
// row is caught through the sum instead).
__device__ __forceinline__ float max3raw(float a, float b, float c) {
  float d;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
  return d;
}

// Value of lane (l ^ J) for lane l, without an LDS round trip where the
// pattern allows: DPP quad permutes for J = 1, 2, row shifts for J = 4, 8,
// a swizzle for J = 16, and a permute only for J = 32.
template <int J>
__device__ __forceinline__ uint32_t lane_xor(uint32_t v) {
  if constexpr (J == 1) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);  // quad_perm 1,0,3,2
  } else if constexpr (J == 2) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false);  // quad_perm 2,3,0,1
  } else if constexpr (J == 4 || J == 8) {
    const uint32_t up = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x100 + J, 0xF, 0xF, false);
    const uint32_t dn = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x110 + J, 0xF, 0xF, false);
    return (threadIdx.x & J) ? dn : up;  // row_shl:J reads lane + J, row_shr:J lane - J
  } else if constexpr (J == 16) {
    return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x401F);  // and 0x1F, xor 0x10
  } else {
    return (uint32_t)__shfl_xor((int)v, J, kWave);
  }
}

// maximum of one vector's E logits (same NaN rule as max3raw)
template <int E>
__device__ __forceinline__ float vec_max(const float (&x)[E]) {
  if constexpr (E == 8) {
    float m = max3raw(x[0], x[1], x[2]);
    m = max3raw(m, x[3], x[4]);
    m = max3raw(m, x[5], x[6]);
    return max3raw(m, x[7], x[7]);
  } else {
    const float m = max3raw(x[0], x[1], x[2]);
    return max3raw(m, x[3], x[3]);
  }
}

// One 16-byte vector of logits.
template <typename T>
struct Vec;

template <>
struct Vec<uint16_t> {  // bf16 bit patterns
  static constexpr int kE = 8;
  __device__ static __forceinline__ void cvt(const u32x4& v, float (&x)[8]) {
    x[0] = bf16_lo(v.x); x[1] = bf16_hi(v.x);
    x[2] = bf16_lo(v.y); x[3] = bf16_hi(v.y);
    x[4] = bf16_lo(v.z); x[5] = bf16_hi(v.z);
    x[6] = bf16_lo(v.w); x[7] = bf16_hi(v.w);
  }
};

template <>
struct Vec<_Float16> {
  static constexpr int kE = 8;
  __device__ static __forceinline__ void cvt(const u32x4& v, float (&x)[8]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      x[2 * k] = f16_to_f32((uint16_t)(w[k] & 0xFFFFu));
      x[2 * k + 1] = f16_to_f32((uint16_t)(w[k] >> 16));
    }
  }
};

template <>
struct Vec<float> {
  static constexpr int kE = 4;
  __device__ static __forceinline__ void cvt(const u32x4& v, float (&x)[4]) {
    x[0] = u2f(v.x); x[1] = u2f(v.y); x[2] = u2f(v.z); x[3] = u2f(v.w);
  }
};

// Maximum of an NG x E block of raw values (v_max3 chains).
template <int NG, int E>
__device__ __forceinline__ float block_max_raw(const float (&x)[NG][E]) {
  constexpr int N = NG * E;  // >= 4
  static_assert(N >= 4, "block too small");
  float m = max3raw(x[0][0], x[0][1], x[0][2]);
  // the flattened block, two values per v_max3
#pragma unroll
  for (int i = 3; i + 1 < N; i += 2) m = max3raw(m, x[i / E][i % E], x[(i + 1) / E][(i + 1) % E]);
  if ((N - 3) & 1) m = max3raw(m, x[(N - 1) / E][(N - 1) % E], x[(N - 1) / E][(N - 1) % E]);
  return m;
}

// Online log-sum-exp (+ entropy moment) of one thread, base-2 units:
//   s = sum 2^{d_i},  t = sum 2^{d_i} d_i,  d_i = (x_i - m) log2(e).
// ------------------------------------------------ DPP cross-lane helpers

// Orders one wave's LDS writes before its later LDS reads from other lanes.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Lane l receives lane l - s of its row of 16 (row_shr), lane 15 of the
// previous row (row_bcast:15, rows 1 and 3) or lane 31 (row_bcast:31, rows
// 2 and 3); lanes without a source read 0.
template <int kCtrl, int kRowMask>
__device__ __forceinline__ uint32_t dpp_take(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kCtrl, kRowMask, 0xF, false);
}
// Inclusive scans over the 64 lanes of a wave (DPP, no LDS round trip).
__device__ __forceinline__ uint32_t wave_scan_u32(uint32_t x) {
  x += dpp_take<0x111, 0xF>(x);
  x += dpp_take<0x112, 0xF>(x);
  x += dpp_take<0x114, 0xF>(x);
  x += dpp_take<0x118, 0xF>(x);
  x += dpp_take<0x142, 0xA>(x);
  x += dpp_take<0x143, 0xC>(x);
  return x;
}
__device__ __forceinline__ unsigned long long wave_scan_u64(unsigned long long x) {
#define GTP_SCAN64_STEP(ctrl, rm)                                                    \
  {                                                                                  \
    const uint32_t lo = dpp_take<ctrl, rm>((uint32_t)x);                             \
    const uint32_t hi = dpp_take<ctrl, rm>((uint32_t)(x >> 32));                     \
    x += ((unsigned long long)hi << 32) | lo;                                        \
  }
  GTP_SCAN64_STEP(0x111, 0xF)
  GTP_SCAN64_STEP(0x112, 0xF)
  GTP_SCAN64_STEP(0x114, 0xF)
  GTP_SCAN64_STEP(0x118, 0xF)
  GTP_SCAN64_STEP(0x142, 0xA)
  GTP_SCAN64_STEP(0x143, 0xC)
#undef GTP_SCAN64_STEP
  return x;
}
__device__ __forceinline__ uint32_t lane63_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, kWave - 1);
}
__device__ __forceinline__ unsigned long long lane63_u64(unsigned long long v) {
  return ((unsigned long long)lane63_u32((uint32_t)(v >> 32)) << 32) | lane63_u32((uint32_t)v);
}
// Reductions over the 64 lanes, the result in every lane: the scan's DPP
// steps (lanes without a source read the identity `id`) and a read of lane
// 63.  Unlike __shfl_xor they keep no per-lane addresses in registers, which
// the compiler may otherwise hoist, share with other code of the kernel and
// spill.
template <int kCtrl, int kRowMask>
__device__ __forceinline__ uint32_t dpp_take_id(uint32_t v, uint32_t id) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)id, (int)v, kCtrl, kRowMask, 0xF, false);
}
template <typename Op>
__device__ __forceinline__ uint32_t wave_reduce_u32(uint32_t x, uint32_t id, Op op) {
  x = op(x, dpp_take_id<0x111, 0xF>(x, id));
  x = op(x, dpp_take_id<0x112, 0xF>(x, id));
  x = op(x, dpp_take_id<0x114, 0xF>(x, id));
  x = op(x, dpp_take_id<0x118, 0xF>(x, id));
  x = op(x, dpp_take_id<0x142, 0xA>(x, id));
  x = op(x, dpp_take_id<0x143, 0xC>(x, id));
  return lane63_u32(x);
}
__device__ __forceinline__ uint32_t wave_total_u32(uint32_t x) { return lane63_u32(wave_scan_u32(x)); }
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t x) {
  return wave_reduce_u32(x, 0xFFFFFFFFu, [](uint32_t a, uint32_t b) { return a < b ? a : b; });
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
  return wave_reduce_u32(x, 0u, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
}
// Sums within each row of 16 lanes (inclusive; lane 15 of a row holds the
// row's total).
__device__ __forceinline__ uint32_t row_scan_u32(uint32_t x) {
  x += dpp_take<0x111, 0xF>(x);
  x += dpp_take<0x112, 0xF>(x);
  x += dpp_take<0x114, 0xF>(x);
  x += dpp_take<0x118, 0xF>(x);
  return x;
}
__device__ __forceinline__ unsigned long long row_scan_u64(unsigned long long x) {
#define GTP_ROW64_STEP(ctrl)                                                         \
  {                                                                                  \
    const uint32_t lo = dpp_take<ctrl, 0xF>((uint32_t)x);                            \
    const uint32_t hi = dpp_take<ctrl, 0xF>((uint32_t)(x >> 32));                    \
    x += ((unsigned long long)hi << 32) | lo;                                        \
  }
  GTP_ROW64_STEP(0x111)
  GTP_ROW64_STEP(0x112)
  GTP_ROW64_STEP(0x114)
  GTP_ROW64_STEP(0x118)
#undef GTP_ROW64_STEP
  return x;
}
// Wave maximum of a float (every lane gets it); NaN inputs are ignored.
template <int kCtrl, int kRowMask>
__device__ __forceinline__ float dpp_take_max(float v) {
  return u2f((uint32_t)__builtin_amdgcn_update_dpp((int)0xFF800000u, (int)f2u(v), kCtrl, kRowMask,
                                                   0xF, false));
}
__device__ __forceinline__ float wave_max_f(float x) {
  x = fmaxf(x, dpp_take_max<0x111, 0xF>(x));
  x = fmaxf(x, dpp_take_max<0x112, 0xF>(x));
  x = fmaxf(x, dpp_take_max<0x114, 0xF>(x));
  x = fmaxf(x, dpp_take_max<0x118, 0xF>(x));
  x = fmaxf(x, dpp_take_max<0x142, 0xA>(x));
  x = fmaxf(x, dpp_take_max<0x143, 0xC>(x));
  return u2f((uint32_t)__builtin_amdgcn_readlane((int)f2u(x), kWave - 1));
}
template <int kCtrl, int kRowMask>
__device__ __forceinline__ float dpp_take_f(float v) {
  return u2f((uint32_t)__builtin_amdgcn_update_dpp(0, (int)f2u(v), kCtrl, kRowMask, 0xF, false));
}
__device__ __forceinline__ float wave_sum_f(float x) {
  x += dpp_take_f<0x111, 0xF>(x);
  x += dpp_take_f<0x112, 0xF>(x);
  x += dpp_take_f<0x114, 0xF>(x);
  x += dpp_take_f<0x118, 0xF>(x);
  x += dpp_take_f<0x142, 0xA>(x);
  x += dpp_take_f<0x143, 0xC>(x);
  return u2f((uint32_t)__builtin_amdgcn_readlane((int)f2u(x), kWave - 1));
}

struct Lse3 {
  float m;  // running max, natural units (-inf while nothing finite is seen)
  float s;
  float t;
};

// Fold a block of raw logits whose maximum is cm (NaN values aside).
// kEntropy selects whether t is kept.
template <bool kEntropy, int NG, int E>
__device__ __forceinline__ void lse_fold_block_max(Lse3& st, const float (&x)[NG][E], float cm) {
  if (cm > st.m) {
    if (st.s > 0.0f) {
      const float dl = (st.m - cm) * kLog2e;
      const float f = __builtin_amdgcn_exp2f(dl);
      if (kEntropy) st.t = f * __builtin_fmaf(dl, st.s, st.t);
      st.s *= f;
    }
    st.m = cm;
  }
  // all -inf so far: any finite base keeps d = -inf (weight 0) and NaN = NaN.
  // Below |m| = 1024 the base-2 exponent is one fma, x log2e - m log2e (the
  // rounding of m log2e costs at most 2^-14 of a term, 3e-5 relative); above
  // it x - m is taken first, exact for x near m at any magnitude.
  const float mb = st.m == kNegInf ? 0.0f : st.m;
  float s0 = 0.0f, s1 = 0.0f, t0 = 0.0f, t1 = 0.0f;
  auto term = [&](float d, int i) __attribute__((always_inline)) {
    const float e = __builtin_amdgcn_exp2f(d);
    if (i & 1) {
      s1 += e;
      if (kEntropy) t1 = __builtin_fmaf(e, fmaxf(d, -256.0f), t1);
    } else {
      s0 += e;
      if (kEntropy) t0 = __builtin_fmaf(e, fmaxf(d, -256.0f), t0);
    }
  };
  if (__builtin_fabsf(mb) < 1024.0f) {
    const float mL = mb * kLog2e;
#pragma unroll
    for (int k = 0; k < NG; ++k)
#pragma unroll
      for (int j = 0; j < E; ++j) term(__builtin_fmaf(x[k][j], kLog2e, -mL), k * E + j);
  } else {
#pragma unroll
    for (int k = 0; k < NG; ++k)
#pragma unroll
      for (int j = 0; j < E; ++j) term((x[k][j] - mb) * kLog2e, k * E + j);
  }
  st.s += s0 + s1;
  if (kEntropy) st.t += t0 + t1;
}

template <bool kEntropy, int NG, int E>
__device__ __forceinline__ void lse_fold_block(Lse3& st, const float (&x)[NG][E]) {
  lse_fold_block_max<kEntropy, NG, E>(st, x, block_max_raw<NG, E>(x));
}

__device__ __forceinline__ Lse3 lse3_merge(Lse3 a, Lse3 b) {
  if (a.s != a.s || b.s != b.s) return {fmaxf(a.m, b.m), __builtin_nanf(""), __builtin_nanf("")};
  const float m = fmaxf(a.m, b.m);
  if (m == kNegInf) return {kNegInf, 0.0f, 0.0f};
  float s = 0.0f, t = 0.0f;
  if (a.s > 0.0f) {
    const float da = (a.m - m) * kLog2e;  // <= 0
    const float fa = __builtin_amdgcn_exp2f(da);
    s += a.s * fa;
    t += fa * __builtin_fmaf(da, a.s, a.t);
  }
  if (b.s > 0.0f) {
    const float db = (b.m - m) * kLog2e;
    const float fb = __builtin_amdgcn_exp2f(db);
    s += b.s * fb;
    t += fb * __builtin_fmaf(db, b.s, b.t);
  }
  return {m, s, t};
}

__device__ __forceinline__ Lse3 wave_lse3(Lse3 v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    Lse3 w{__shfl_xor(v.m, o, kWave), __shfl_xor(v.s, o, kWave), __shfl_xor(v.t, o, kWave)};
    v = lse3_merge(v, w);
  }
  return v;
}

// Block-wide merge; every thread gets the result.  `red` holds 3 floats per
// wave.  Callers sync before reusing `red`.
template <int NT>
__device__ __forceinline__ Lse3 block_lse3(Lse3 v, float (*red)[3]) {
  v = wave_lse3(v);
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  if (lane == 0) {
    red[wid][0] = v.m;
    red[wid][1] = v.s;
    red[wid][2] = v.t;
  }
  __syncthreads();
  Lse3 r{red[0][0], red[0][1], red[0][2]};
#pragma unroll
  for (int w = 1; w < NT / kWave; ++w) r = lse3_merge(r, Lse3{red[w][0], red[w][1], red[w][2]});
  return r;
}
// The same over the block, with the wave step on DPP and a swizzle within
// each half of the wave and a read of lanes 0 and 32 (no per-lane shuffle
// addresses; for kernels whose register budget is tight).
template <int NT>
__device__ __forceinline__ Lse3 block_lse3_dpp(Lse3 v, float (*red)[3]) {
  auto step = [&](auto xr) __attribute__((always_inline)) {
    v = lse3_merge(v, Lse3{u2f(xr(f2u(v.m))), u2f(xr(f2u(v.s))), u2f(xr(f2u(v.t)))});
  };
  step([](uint32_t x) { return lane_xor<1>(x); });
  step([](uint32_t x) { return lane_xor<2>(x); });
  step([](uint32_t x) { return lane_xor<4>(x); });
  step([](uint32_t x) { return lane_xor<8>(x); });
  step([](uint32_t x) { return lane_xor<16>(x); });
  auto at = [&](int l) {
    return Lse3{u2f((uint32_t)__builtin_amdgcn_readlane((int)f2u(v.m), l)),
                u2f((uint32_t)__builtin_amdgcn_readlane((int)f2u(v.s), l)),
                u2f((uint32_t)__builtin_amdgcn_readlane((int)f2u(v.t), l))};
  };
  v = lse3_merge(at(0), at(32));
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  if (lane == 0) {
    red[wid][0] = v.m;
    red[wid][1] = v.s;
    red[wid][2] = v.t;
  }
  __syncthreads();
  Lse3 r{red[0][0], red[0][1], red[0][2]};
#pragma unroll
  for (int w = 1; w < NT / kWave; ++w) r = lse3_merge(r, Lse3{red[w][0], red[w][1], red[w][2]});
  return r;
}

// (m, s) merge over a wave without per-step exponentials: the wave maximum
// first, then one rescale per lane and a plain sum.  NaN in s (a NaN or +inf
// logit) stays NaN.
__device__ __forceinline__ void wave_lse2(float& m, float& s) {
  const float mw = wave_max_f(m);
  const float sv = m == mw ? s : s * __builtin_amdgcn_exp2f((m - mw) * kLog2e);
  m = mw;
  s = wave_sum_f(sv);
}

// Block-wide (m, s) of NT threads; every thread gets the result.  `red`
// holds 2 floats per wave; callers sync before reusing it.
template <int NT>
__device__ __forceinline__ void block_lse2(float& m, float& s, float (*red)[3]) {
  wave_lse2(m, s);
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  if (lane == 0) {
    red[wid][0] = m;
    red[wid][1] = s;
  }
  __syncthreads();
  m = lane < NT / kWave ? red[lane][0] : kNegInf;
  s = lane < NT / kWave ? red[lane][1] : 0.0f;
  wave_lse2(m, s);
}

struct NoPrologue {
  __device__ __forceinline__ void operator()() const {}
};

// Stream vectors [v0, v1) of a 16-byte aligned row; thread tid folds vectors
// v0 + step*NT*NG + k*NT + tid.  `fold(x, sw, vec_index, last)` receives each
// step's converted block; on the last step (last == true) vectors past v1
// arrive as copies of vector v1-1 and must be ignored by the caller
// (vec_index + k*NT >= v1).  Loads of the next step are issued before the
// current step is folded.
//
// With kSide, vector v (absolute index) also loads side[v >> side_shift] in
// the same pipeline (e.g. the allow-mask word that holds its bits); sw[k] is
// that word (0xFFFFFFFF without kSide).
//
// `prologue()` runs once, after the first step's loads are issued: set-up
// work whose own loads then overlap the stream's first round trip.  It is
// called by every thread, also when the range is empty.
template <typename T, int NT, int NG, bool kNonTemporal, bool kSide, typename Fold,
          typename Prologue = NoPrologue>
__device__ __forceinline__ void stream_vectors_side(const T* __restrict__ row, int64_t v0,
                                                    int64_t v1,
                                                    const uint32_t* __restrict__ side,
                                                    int side_shift, Fold&& fold,
                                                    Prologue&& prologue = Prologue{}) {
  constexpr int E = Vec<T>::kE;
  const int64_t n = v1 - v0;
  if (n <= 0) {
    prologue();
    return;
  }
  // 32-bit byte offsets from a uniform base: rows are far below 4 GB, and the
  // saddr + voffset load form needs no 64-bit address arithmetic per vector
  const char* __restrict__ base = reinterpret_cast<const char*>(row) + v0 * 16;
  constexpr uint32_t kStep = (uint32_t)NT * NG;
  const uint32_t nsteps = (uint32_t)((n + kStep - 1) / kStep);
  const uint32_t tid = threadIdx.x;
  const uint32_t last = (uint32_t)(n - 1);
  u32x4 a[NG], b[NG];
  uint32_t sa[NG], sb[NG];
  auto issue = [&](u32x4(&buf)[NG], uint32_t(&sbuf)[NG], uint32_t step) {
    const uint32_t first = step * kStep + tid;
#pragma unroll
    for (int k = 0; k < NG; ++k) {
      uint32_t vi = first + (uint32_t)k * NT;
      vi = vi < last ? vi : last;
      const u32x4* p = reinterpret_cast<const u32x4*>(base + vi * 16u);
      if (kNonTemporal)
        buf[k] = __builtin_nontemporal_load(p);
      else
        buf[k] = *p;
      if (kSide) sbuf[k] = side[(uint64_t)(v0 + vi) >> side_shift];
    }
  };
  auto consume = [&](const u32x4(&buf)[NG], uint32_t(&sbuf)[NG], uint32_t step) {
    float x[NG][E];
#pragma unroll
    for (int k = 0; k < NG; ++k) {
      Vec<T>::cvt(buf[k], x[k]);
      if (!kSide) sbuf[k] = 0xFFFFFFFFu;
    }
    fold(x, sbuf, v0 + (int64_t)(step * kStep + tid), step == nsteps - 1);
  };
  // Two steps per trip with one back-edge; prefetches past the last step
  // re-load the last step's (cached) addresses instead of branching, so the
  // outstanding-load count is the same on every path.
  issue(a, sa, 0);
  prologue();
  for (uint32_t step = 0; step < nsteps; step += 2) {
    issue(b, sb, step + 1 < nsteps ? step + 1 : nsteps - 1);
    consume(a, sa, step);
    issue(a, sa, step + 2 < nsteps ? step + 2 : nsteps - 1);
    if (step + 1 < nsteps) consume(b, sb, step + 1);
  }
}

// The same without side words: fold(x, vec_index, last).
template <typename T, int NT, int NG, bool kNonTemporal, typename Fold,
          typename Prologue = NoPrologue>
__device__ __forceinline__ void stream_vectors(const T* __restrict__ row, int64_t v0, int64_t v1,
                                               Fold&& fold, Prologue&& prologue = Prologue{}) {
  constexpr int E = Vec<T>::kE;
  stream_vectors_side<T, NT, NG, kNonTemporal, false>(
      row, v0, v1, nullptr, 0,
      [&](float(&x)[NG][E], const uint32_t(&)[NG], int64_t vbase, bool last) {
        fold(x, vbase, last);
      },
      prologue);
}

// Per-wave dynamic variant.  The range is cut into chunks of 64 * NG vectors;
// each wave takes the next chunk from an LDS counter (`*counter` must be 0
// and visible to every wave before the call), so waves that the scheduler
// favours simply take more chunks and all waves of the workgroup finish
// together.  Lane l of a wave folds vectors chunk*64*NG + k*64 + l.
// `fold(x, sw, vec_index, last)`: vector k of the block is vec_index + k*64;
// when `last`, indices >= v1 are copies to be ignored.  After the range is
// exhausted a wave's prefetch loads one cached vector instead of branching.
template <typename T, int NG, bool kNonTemporal, bool kSide, typename Fold,
          typename Prologue = NoPrologue>
__device__ __forceinline__ void stream_vectors_dyn(const T* __restrict__ row, int64_t v0,
                                                   int64_t v1, const uint32_t* __restrict__ side,
                                                   int side_shift, uint32_t* counter, Fold&& fold,
                                                   Prologue&& prologue = Prologue{}) {
  constexpr int E = Vec<T>::kE;
  constexpr uint32_t kChunk = (uint32_t)kWave * NG;
  const int64_t n = v1 - v0;
  if (n <= 0) {
    prologue();
    return;
  }
  const char* __restrict__ base = reinterpret_cast<const char*>(row) + v0 * 16;
  const uint32_t nchunks = (uint32_t)((n + kChunk - 1) / kChunk);
  const uint32_t lane = threadIdx.x & (kWave - 1);
  const uint32_t last = (uint32_t)(n - 1);
  auto grab = [&]() -> uint32_t {
    uint32_t c = 0;
    if (lane == 0) c = atomicAdd(counter, 1u);
    return __builtin_amdgcn_readfirstlane(c);
  };
  u32x4 a[NG], b[NG];
  uint32_t sa[NG], sb[NG];
  auto issue = [&](u32x4(&buf)[NG], uint32_t(&sbuf)[NG], uint32_t chunk) {
    const bool live = chunk < nchunks;
    const uint32_t first = chunk * kChunk + lane;
#pragma unroll
    for (int k = 0; k < NG; ++k) {
      uint32_t vi = first + (uint32_t)k * kWave;
      vi = vi < last ? vi : last;
      vi = live ? vi : 0u;
      const u32x4* p = reinterpret_cast<const u32x4*>(base + vi * 16u);
      if (kNonTemporal)
        buf[k] = __builtin_nontemporal_load(p);
      else
        buf[k] = *p;
      if (kSide) sbuf[k] = side[(uint64_t)(v0 + vi) >> side_shift];
    }
  };
  auto consume = [&](const u32x4(&buf)[NG], uint32_t(&sbuf)[NG], uint32_t chunk) {
    float x[NG][E];
#pragma unroll
    for (int k = 0; k < NG; ++k) {
      Vec<T>::cvt(buf[k], x[k]);
      if (!kSide) sbuf[k] = 0xFFFFFFFFu;
    }
    fold(x, sbuf, v0 + (int64_t)(chunk * kChunk + lane), chunk == nchunks - 1);
  };
  uint32_t ca = grab();
  issue(a, sa, ca);
  prologue();
  while (ca < nchunks) {
    const uint32_t cb = grab();
    issue(b, sb, cb);
    consume(a, sa, ca);
    if (cb >= nchunks) break;
    ca = grab();
    issue(a, sa, ca);
    consume(b, sb, cb);
  }
}

// Stream vectors [v0, v1) (v1 > v0) of a 16-byte aligned row with a prefix
// pilot.  Thread t loads the pilot vectors v0 + q*NT + t (q < NP, inside the
// range; np = number of pilot vectors, entries at or past np re-read the
// first vector), then calls `prologue()` (block-wide set-up, which may hold a
// barrier: the pilot loads are already in flight) and `pre(p, sp, np)` on
// them before any other load is issued; then the wave's first two chunks of
// the rest are issued and
// `post(p, sp, np)` runs with them in flight.  `pre` must not hold block
// barriers: a wave that waits on another before issuing its own loads lets
// the memory pipeline drain.  The rest of the range is streamed as in
// stream_vectors_dyn: `fold(x, raw, sw, vec_index, last)`, vector k of the
// block (raw 16 bytes raw[k], converted x[k]) at vec_index + k*64.
// With kSide, `side` is a bit array with one bit per element (E bits per
// vector, bit i of word i >> 5): every vector, pilot or chunk, brings the
// word holding its bits (sp[q] for the pilot, sw[k] for vector k of a
// chunk).  Every load before the pilot is unconditional (out-of-range ones
// re-read the first vector), so the compiler can wait for the pilot data
// alone.
template <typename T, int NT, int NP, int NG, bool kNonTemporal, bool kSide, typename Prologue,
          typename Pre, typename Post, typename Fold>
__device__ __forceinline__ void stream_vectors_prefix(const T* __restrict__ row, int64_t v0,
                                                      int64_t v1, const uint32_t* __restrict__ side,
                                                      uint32_t* counter, Prologue&& prologue,
                                                      Pre&& pre, Post&& post, Fold&& fold) {
  constexpr int E = Vec<T>::kE;
  constexpr uint32_t kChunk = (uint32_t)kWave * NG;
  const int64_t n = v1 - v0 > 0 ? v1 - v0 : 0;
  const int64_t np = n < (int64_t)NP * NT ? n : (int64_t)NP * NT;
  const char* __restrict__ base = reinterpret_cast<const char*>(row) + v0 * 16;
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & (kWave - 1);
  u32x4 p[NP];
  uint32_t sp[NP];
#pragma unroll
  for (int q = 0; q < NP; ++q) {
    uint32_t vi = (uint32_t)q * NT + tid;
    vi = vi < (uint32_t)np ? vi : 0u;
    const u32x4* a = reinterpret_cast<const u32x4*>(base + vi * 16u);
    p[q] = kNonTemporal ? __builtin_nontemporal_load(a) : *a;
    sp[q] = kSide ? side[((uint64_t)(v0 + vi) * E) >> 5] : 0xFFFFFFFFu;
  }
  prologue();  // block-wide set-up (its barrier included) while the pilot loads fly
  pre(p, sp, np);
  // the rest: [v0 + np, v1) in per-wave chunks (an empty rest re-reads the
  // first vector of the range)
  const char* __restrict__ base2 = base + (np < n ? np : 0) * 16;
  const int64_t n2 = n - np;
  const uint32_t nchunks = (uint32_t)((n2 + kChunk - 1) / kChunk);
  const uint32_t last = n2 > 0 ? (uint32_t)(n2 - 1) : 0u;
  auto grab = [&]() -> uint32_t {
    uint32_t c = 0;
    if (lane == 0) c = atomicAdd(counter, 1u);
    return __builtin_amdgcn_readfirstlane(c);
  };
  const int64_t vfirst = v0 + (np < n ? np : 0);  // the vector at base2
  u32x4 a[NG], b[NG];
  uint32_t swa[NG], swb[NG];
  auto issue = [&](u32x4(&buf)[NG], uint32_t(&sw)[NG], uint32_t chunk) {
    const bool live = chunk < nchunks;
    const uint32_t first = chunk * kChunk + lane;
#pragma unroll
    for (int k = 0; k < NG; ++k) {
      uint32_t vi = first + (uint32_t)k * kWave;
      vi = vi < last ? vi : last;
      vi = live ? vi : 0u;
      const u32x4* q = reinterpret_cast<const u32x4*>(base2 + vi * 16u);
      if (kNonTemporal)
        buf[k] = __builtin_nontemporal_load(q);
      else
        buf[k] = *q;
      // the word holding this vector's bits, requested with its data (a
      // shuffle from the lane that loaded it would put an LDS round trip on
      // every vector's path)
      sw[k] = kSide ? side[((uint64_t)(vfirst + vi) * E) >> 5] : 0xFFFFFFFFu;
    }
  };
  auto consume = [&](const u32x4(&buf)[NG], const uint32_t(&sw)[NG], uint32_t chunk) {
    float x[NG][E];
#pragma unroll
    for (int k = 0; k < NG; ++k) Vec<T>::cvt(buf[k], x[k]);
    fold(x, buf, sw, v0 + np + (int64_t)(chunk * kChunk + lane), chunk == nchunks - 1);
  };
  uint32_t ca = grab();
  issue(a, swa, ca);
  uint32_t cb = grab();
  issue(b, swb, cb);
  post(p, sp, np);
  if (ca >= nchunks) return;
  consume(a, swa, ca);
  while (cb < nchunks) {
    ca = grab();
    issue(a, swa, ca);
    consume(b, swb, cb);
    if (ca >= nchunks) break;
    cb = grab();
    issue(b, swb, cb);
    consume(a, swa, ca);
  }
}

// Per-wave dynamic chunks of 64 x NG vectors over [v0, v1) (v1 > v0), as the
// main loop of stream_vectors_prefix: `fold(x, raw, sw, vec_index, last)`;
// with kSide lane l also brings word l of the chunk's bits in `side` (one bit
// per element; v0 * E must be a multiple of 32).
template <typename T, int NG, bool kNonTemporal, bool kSide, typename Fold>
__device__ __forceinline__ void stream_chunks(const T* __restrict__ row, int64_t v0, int64_t v1,
                                              const uint32_t* __restrict__ side,
                                              uint32_t* counter, Fold&& fold) {
  constexpr int E = Vec<T>::kE;
  constexpr uint32_t kChunk = (uint32_t)kWave * NG;
  const int64_t n = v1 - v0 > 0 ? v1 - v0 : 0;
  const char* __restrict__ base = reinterpret_cast<const char*>(row) + v0 * 16;
  const uint32_t lane = threadIdx.x & (kWave - 1);
  const uint32_t nchunks = (uint32_t)((n + kChunk - 1) / kChunk);
  const uint32_t last = n > 0 ? (uint32_t)(n - 1) : 0u;
  const uint64_t w_first = ((uint64_t)v0 * E) >> 5;
  const uint64_t w_last = n > 0 ? ((uint64_t)v1 * E - 1) >> 5 : w_first;
  auto grab = [&]() -> uint32_t {
    uint32_t c = 0;
    if (lane == 0) c = atomicAdd(counter, 1u);
    return __builtin_amdgcn_readfirstlane(c);
  };
  u32x4 a[NG], b[NG];
  uint32_t swa = 0xFFFFFFFFu, swb = 0xFFFFFFFFu;
  auto issue = [&](u32x4(&buf)[NG], uint32_t& sw, uint32_t chunk) {
    const bool live = chunk < nchunks;
    const uint32_t first = chunk * kChunk + lane;
#pragma unroll
    for (int k = 0; k < NG; ++k) {
      uint32_t vi = first + (uint32_t)k * kWave;
      vi = vi < last ? vi : last;
      vi = live ? vi : 0u;
      const u32x4* q = reinterpret_cast<const u32x4*>(base + vi * 16u);
      if (kNonTemporal)
        buf[k] = __builtin_nontemporal_load(q);
      else
        buf[k] = *q;
    }
    if (kSide) {
      const uint64_t w = w_first + (((uint64_t)(live ? chunk : 0u) * kChunk * E) >> 5) + lane;
      sw = side[w < w_last ? w : w_last];
    }
  };
  auto consume = [&](const u32x4(&buf)[NG], uint32_t sw, uint32_t chunk) {
    float x[NG][E];
#pragma unroll
    for (int k = 0; k < NG; ++k) Vec<T>::cvt(buf[k], x[k]);
    fold(x, buf, sw, v0 + (int64_t)(chunk * kChunk + lane), chunk == nchunks - 1);
  };
  if (n == 0) return;
  uint32_t ca = grab();
  issue(a, swa, ca);
  while (ca < nchunks) {
    const uint32_t cb = grab();
    issue(b, swb, cb);
    consume(a, swa, ca);
    if (cb >= nchunks) break;
    ca = grab();
    issue(a, swa, ca);
    consume(b, swb, cb);
  }
}

// Mark the vectors of a block that lie past the end (only on the last step).
template <int NG, int E, int NT>
__device__ __forceinline__ void mask_tail(float (&x)[NG][E], int64_t vbase, int64_t v1) {
#pragma unroll
  for (int k = 0; k < NG; ++k)
    if (vbase + (int64_t)k * NT >= v1) {
#pragma unroll
      for (int j = 0; j < E; ++j) x[k][j] = kNegInf;
    }
}

}  // namespace gtp
