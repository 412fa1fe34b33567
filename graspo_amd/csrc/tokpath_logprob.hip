// tokpath_logprob.hip -- selective log-softmax gather + softmax entropy (gfx950).
//
// One workgroup of 256 threads streams one row once (tokpath_stream.h:
// double-buffered 16-byte loads, 8 vectors per thread per step, non-temporal
// because nothing re-reads the row).  Each thread keeps an online (m, s, t)
// state in base-2 units:
//   d_i = (x_i - m) * log2(e),  s = sum 2^{d_i},  t = sum 2^{d_i} * d_i
// so logprob = x_target - m - ln s and entropy = ln s - ln2 * t / s.
// The row is never written back (no [N, V] log-softmax), so the kernel is
// bounded by one HBM read of the logits and by the VALU work per element.
//
// Replaces sequence_log_probs_from_logits (src/graspo/core/graspo_loss.py:19-21)
// and the logsumexp / logaddexp chunk loop of _selected_token_log_probs_from_hidden
// (src/graspo/backends/graspoflow/tensor_utils.py:180-186).
#include "tokpath_stream.h"

namespace gtp {

constexpr int kLpBlock = 256;
constexpr int kLpVecs = 8;  // 16-byte vectors per thread per step

// Scalar fold of one logit (remainders and unaligned rows only).
__device__ __forceinline__ void lse_fold_one(Lse3& st, float x) {
  if (x > st.m) {
    if (st.s > 0.0f) {
      const float dl = (st.m - x) * kLog2e;
      const float f = __builtin_amdgcn_exp2f(dl);
      st.t = f * __builtin_fmaf(dl, st.s, st.t);
      st.s *= f;
    }
    st.m = x;
  }
  if (x != x) st.s = __builtin_nanf("");
  const float d = (x - (st.m == kNegInf ? 0.0f : st.m)) * kLog2e;
  const float e = __builtin_amdgcn_exp2f(d);
  st.s += e;
  st.t = __builtin_fmaf(e, fmaxf(d, -256.0f), st.t);
}

// This thread's share of one row [0, V).
template <typename T>
__device__ __forceinline__ Lse3 lp_thread_state(const T* __restrict__ row, int64_t V) {
  constexpr int E = Vec<T>::kE;
  Lse3 st{kNegInf, 0.0f, 0.0f};
  const bool vec_ok = (reinterpret_cast<uintptr_t>(row) & 15u) == 0;
  const int64_t nvec = vec_ok ? V / E : 0;
  stream_vectors<T, kLpBlock, kLpVecs, true>(
      row, 0, nvec, [&](float(&x)[kLpVecs][E], int64_t vbase, bool last) {
        if (last) mask_tail<kLpVecs, E, kLpBlock>(x, vbase, nvec);
        lse_fold_block<true, kLpVecs, E>(st, x);
      });
  for (int64_t i = nvec * E + threadIdx.x; i < V; i += kLpBlock) lse_fold_one(st, Elem<T>::get(row, i));
  return st;
}

__device__ __forceinline__ int64_t load_target(const void* targets, int t64, int64_t n) {
  return t64 ? reinterpret_cast<const int64_t*>(targets)[n]
             : (int64_t)reinterpret_cast<const int32_t*>(targets)[n];
}

template <typename T>
__global__ __launch_bounds__(kLpBlock) void logprob_entropy_kernel(
    const T* __restrict__ logits, int64_t V, int64_t row_stride, const void* __restrict__ targets,
    int t64, float* __restrict__ out_lp, float* __restrict__ out_H, int32_t* __restrict__ out_status) {
  __shared__ float red[kLpBlock / kWave][3];
  const int64_t n = blockIdx.x;
  const T* row = logits + n * row_stride;
  const int64_t tgt = load_target(targets, t64, n);
  const bool tgt_ok = tgt >= 0 && tgt < V;
  float xt = 0.0f;
  if (threadIdx.x == 0 && tgt_ok) xt = Elem<T>::get(row, tgt);
  const Lse3 st = block_lse3<kLpBlock>(lp_thread_state<T>(row, V), red);
  if (threadIdx.x == 0) {
    const float ln_s = __builtin_amdgcn_logf(st.s) * kLn2;
    out_lp[n] = tgt_ok ? raw_logprob(xt, st.m, ln_s) : __builtin_nanf("");
    if (out_H) out_H[n] = ln_s - kLn2 * st.t / st.s;
    if (out_status) out_status[n] = tgt_ok ? GTP_ROW_OK : GTP_ROW_BAD_TARGET;
  }
}

// Chunk state layout: [N][4] = (m, s, t_nat, x_target), t_nat = ln2 * t.
template <typename T>
__global__ __launch_bounds__(kLpBlock) void lse_partial_kernel(
    const T* __restrict__ logits, int64_t Vc, int64_t row_stride, int64_t col_offset,
    const void* __restrict__ targets, int t64, float* __restrict__ state, int accumulate) {
  __shared__ float red[kLpBlock / kWave][3];
  const int64_t n = blockIdx.x;
  const T* row = logits + n * row_stride;
  const int64_t tgt = targets ? load_target(targets, t64, n) - col_offset : -1;
  Lse3 st = block_lse3<kLpBlock>(lp_thread_state<T>(row, Vc), red);
  if (threadIdx.x == 0) {
    float* sp = state + n * 4;
    float xt = __builtin_nanf("");
    if (accumulate) {
      const Lse3 old{sp[0], sp[1], sp[2] * kLog2e};
      st = lse3_merge(old, st);
      xt = sp[3];
    }
    if (tgt >= 0 && tgt < Vc) xt = Elem<T>::get(row, tgt);
    sp[0] = st.m;
    sp[1] = st.s;
    sp[2] = st.t * kLn2;
    sp[3] = xt;
  }
}

__global__ void lse_finalize_kernel(const float* __restrict__ state, int64_t N,
                                    float* __restrict__ out_lp, float* __restrict__ out_H) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const float m = state[n * 4 + 0], s = state[n * 4 + 1], t = state[n * 4 + 2], xt = state[n * 4 + 3];
  const float ln_s = __builtin_amdgcn_logf(s) * kLn2;
  if (out_lp) out_lp[n] = raw_logprob(xt, m, ln_s);
  if (out_H) out_H[n] = ln_s - t / s;
}

// ---------------------------------------------------------------- backward
//
// d logprob / d x_i = [i == target] - p_i with p_i = exp(x_i - lse), so the
// gradient of a loss with dL/dlogprob = g per row is g * ([i == t] - p_i):
// one read of the row and one write of the gradient in the logits' dtype.
// A row with g == 0 (an ignored SFT position) is written as zeros without
// reading it.

// fp32 -> bf16 bit pattern, round to nearest even (NaN stays NaN)
__device__ __forceinline__ uint32_t bf16_rne(float f) {
  const uint32_t u = f2u(f);
  const uint32_t r = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
  return (u & 0x7FFFFFFFu) > 0x7F800000u ? 0x7FC0u : r;
}

template <typename T>
struct GradOut;
template <>
struct GradOut<uint16_t> {
  // 8 gradients -> one 16-byte vector of bf16
  __device__ static __forceinline__ u32x4 pack(const float (&g)[8]) {
    u32x4 v;
    v.x = bf16_rne(g[0]) | (bf16_rne(g[1]) << 16);
    v.y = bf16_rne(g[2]) | (bf16_rne(g[3]) << 16);
    v.z = bf16_rne(g[4]) | (bf16_rne(g[5]) << 16);
    v.w = bf16_rne(g[6]) | (bf16_rne(g[7]) << 16);
    return v;
  }
  __device__ static __forceinline__ void put(uint16_t* p, int64_t i, float g) {
    p[i] = (uint16_t)bf16_rne(g);
  }
};
template <>
struct GradOut<_Float16> {
  __device__ static __forceinline__ u32x4 pack(const float (&g)[8]) {
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const _Float16 lo = (_Float16)g[2 * k], hi = (_Float16)g[2 * k + 1];
      w[k] = (uint32_t)__builtin_bit_cast(uint16_t, lo) |
             ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
    }
    u32x4 v;
    v.x = w[0];
    v.y = w[1];
    v.z = w[2];
    v.w = w[3];
    return v;
  }
  __device__ static __forceinline__ void put(_Float16* p, int64_t i, float g) {
    p[i] = (_Float16)g;
  }
};
template <>
struct GradOut<float> {
  __device__ static __forceinline__ u32x4 pack(const float (&g)[4]) {
    u32x4 v;
    v.x = f2u(g[0]);
    v.y = f2u(g[1]);
    v.z = f2u(g[2]);
    v.w = f2u(g[3]);
    return v;
  }
  __device__ static __forceinline__ void put(float* p, int64_t i, float g) { p[i] = g; }
};

// One row of g * ([i == t] - p_i), p_i = 2^((x_i - lse) log2 e): whole
// vectors go to emit_vec(vector index, gradients), the elements past the last
// whole vector (or every element when nvec == 0) to emit_one(i, gradient).
template <typename T, typename EmitVec, typename EmitOne>
__device__ __forceinline__ void logprob_backward_row(const T* __restrict__ row, int64_t V,
                                                     int64_t nvec, int64_t tgt, float g, float lse,
                                                     EmitVec&& emit_vec, EmitOne&& emit_one) {
  constexpr int E = Vec<T>::kE;
  const float ng = -g;
  stream_vectors<T, kLpBlock, kLpVecs, true>(
      row, 0, nvec, [&](float(&x)[kLpVecs][E], int64_t vbase, bool last) {
#pragma unroll
        for (int k = 0; k < kLpVecs; ++k) {
          const int64_t vi = vbase + (int64_t)k * kLpBlock;
          if (last && vi >= nvec) continue;
          float gr[E];
#pragma unroll
          for (int j = 0; j < E; ++j)
            gr[j] = ng * __builtin_amdgcn_exp2f((x[k][j] - lse) * kLog2e);
          const int64_t d = tgt - vi * E;
          if (d >= 0 && d < E) {
            // g (1 - p_t) as -g expm1(x_t - lse): no cancellation when p_t ~ 1
#pragma unroll
            for (int j = 0; j < E; ++j)
              if (j == (int)d) gr[j] = -g * expm1f(x[k][j] - lse);
          }
          emit_vec(vi, gr);
        }
      });
  for (int64_t i = nvec * E + threadIdx.x; i < V; i += kLpBlock) {
    const float xi = Elem<T>::get(row, i);
    emit_one(i, i == tgt ? -g * expm1f(xi - lse)
                         : ng * __builtin_amdgcn_exp2f((xi - lse) * kLog2e));
  }
}

template <typename T>
__global__ __launch_bounds__(kLpBlock) void logprob_backward_kernel(
    const T* __restrict__ logits, int64_t V, int64_t row_stride, int64_t col_offset,
    const void* __restrict__ targets, int t64, const float* __restrict__ grad_lp,
    const float* __restrict__ lse_in, T* __restrict__ grad, int64_t grad_stride) {
  constexpr int E = Vec<T>::kE;
  const int64_t n = blockIdx.x;
  const T* row = logits + n * row_stride;
  T* grow = grad + n * grad_stride;
  const float g = grad_lp[n];
  const int64_t tgt = load_target(targets, t64, n) - col_offset;  // outside [0, V): no one-hot term
  const bool vec_ok = ((reinterpret_cast<uintptr_t>(row) | reinterpret_cast<uintptr_t>(grow)) & 15u) == 0;
  const int64_t nvec = vec_ok ? V / E : 0;
  u32x4* gv = reinterpret_cast<u32x4*>(grow);
  if (g == 0.0f) {
    const u32x4 z = {0u, 0u, 0u, 0u};
    for (int64_t vi = threadIdx.x; vi < nvec; vi += kLpBlock) __builtin_nontemporal_store(z, gv + vi);
    for (int64_t i = nvec * E + threadIdx.x; i < V; i += kLpBlock) GradOut<T>::put(grow, i, 0.0f);
    return;
  }
  logprob_backward_row<T>(
      row, V, nvec, tgt, g, lse_in[n],
      [&](int64_t vi, const float(&gr)[E]) {
        __builtin_nontemporal_store(GradOut<T>::pack(gr), gv + vi);
      },
      [&](int64_t i, float gi) { GradOut<T>::put(grow, i, gi); });
}

// The same gradient of fp32 logits written as two bf16 arrays, hi = the
// gradient rounded to bf16 and lo = the remainder rounded to bf16, so that
// |grad - hi - lo| <= 2^-16 |grad| (each bf16 rounding is within 2^-8): bf16
// matrix-core GEMMs of both parts carry about 16 significant bits.
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void split_bf16(float v, uint32_t& hi, uint32_t& lo) {
  hi = bf16_rne(v);
  lo = (hi & 0x7F80u) == 0x7F80u ? 0u : bf16_rne(v - u2f(hi << 16));  // inf / NaN: no remainder
}
__global__ __launch_bounds__(kLpBlock) void logprob_backward_split_kernel(
    const float* __restrict__ logits, int64_t V, int64_t row_stride, int64_t col_offset,
    const void* __restrict__ targets, int t64, const float* __restrict__ grad_lp,
    const float* __restrict__ lse_in, uint16_t* __restrict__ ghi, uint16_t* __restrict__ glo,
    int64_t grad_stride) {
  const int64_t n = blockIdx.x;
  const float* row = logits + n * row_stride;
  uint16_t* hrow = ghi + n * grad_stride;
  uint16_t* lrow = glo + n * grad_stride;
  const float g = grad_lp[n];
  const int64_t tgt = load_target(targets, t64, n) - col_offset;
  const bool vec_ok = ((reinterpret_cast<uintptr_t>(row) & 15u) |
                       ((reinterpret_cast<uintptr_t>(hrow) | reinterpret_cast<uintptr_t>(lrow)) &
                        7u)) == 0;
  const int64_t nvec = vec_ok ? V / 4 : 0;
  u32x2* hv = reinterpret_cast<u32x2*>(hrow);
  u32x2* lv = reinterpret_cast<u32x2*>(lrow);
  if (g == 0.0f) {
    const u32x2 z = {0u, 0u};
    for (int64_t vi = threadIdx.x; vi < nvec; vi += kLpBlock) {
      __builtin_nontemporal_store(z, hv + vi);
      __builtin_nontemporal_store(z, lv + vi);
    }
    for (int64_t i = nvec * 4 + threadIdx.x; i < V; i += kLpBlock) hrow[i] = lrow[i] = 0;
    return;
  }
  logprob_backward_row<float>(
      row, V, nvec, tgt, g, lse_in[n],
      [&](int64_t vi, const float(&gr)[4]) {
        uint32_t h[4], l[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) split_bf16(gr[j], h[j], l[j]);
        const u32x2 ho = {h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
        const u32x2 lo = {l[0] | (l[1] << 16), l[2] | (l[3] << 16)};
        __builtin_nontemporal_store(ho, hv + vi);
        __builtin_nontemporal_store(lo, lv + vi);
      },
      [&](int64_t i, float gi) {
        uint32_t h, l;
        split_bf16(gi, h, l);
        hrow[i] = (uint16_t)h;
        lrow[i] = (uint16_t)l;
      });
}

}  // namespace gtp

using namespace gtp;

extern "C" int gtp_logprob_entropy_rows(const void* logits, int dtype, int64_t N, int64_t V,
                                        int64_t row_stride, const void* targets, int targets_int64,
                                        float* out_logprob, float* out_entropy, int32_t* out_status,
                                        void* stream) {
  if (N < 0 || V <= 0 || row_stride < V || (N > 0 && (!logits || !targets || !out_logprob)))
    return GTP_ERR_INVALID_ARGUMENT;
  if (N > 0x7FFFFFFFll) return GTP_ERR_UNSUPPORTED;
  if (N == 0) return GTP_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)N), block(kLpBlock);
  switch (dtype) {
    case GTP_DTYPE_BF16:
      launch_timed(logprob_entropy_kernel<uint16_t>, grid, block, s,
                         reinterpret_cast<const uint16_t*>(logits), V, row_stride, targets,
                         targets_int64, out_logprob, out_entropy, out_status);
      break;
    case GTP_DTYPE_F16:
      launch_timed(logprob_entropy_kernel<_Float16>, grid, block, s,
                         reinterpret_cast<const _Float16*>(logits), V, row_stride, targets,
                         targets_int64, out_logprob, out_entropy, out_status);
      break;
    case GTP_DTYPE_F32:
      launch_timed(logprob_entropy_kernel<float>, grid, block, s,
                         reinterpret_cast<const float*>(logits), V, row_stride, targets,
                         targets_int64, out_logprob, out_entropy, out_status);
      break;
    default:
      return GTP_ERR_INVALID_ARGUMENT;
  }
  return hipGetLastError() == hipSuccess ? GTP_OK : GTP_ERR_LAUNCH;
}

namespace gtp {
thread_local LaunchEvents g_next_launch_events{nullptr, nullptr};
}

extern "C" int gtp_time_next_launch(void* start_event, void* stop_event) {
  if (!start_event || !stop_event) return GTP_ERR_INVALID_ARGUMENT;
  g_next_launch_events = LaunchEvents{reinterpret_cast<hipEvent_t>(start_event),
                                      reinterpret_cast<hipEvent_t>(stop_event)};
  return GTP_OK;
}

namespace gtp {
// Read-only streaming floor: one workgroup of 1024 threads per row reads the
// row's 16-byte vectors once (non-temporal, 8 per lane in flight, the
// samplers' access pattern) and XORs them; a row whose XOR equals a fixed
// pattern writes it, so the loads cannot be dropped.
__global__ __launch_bounds__(1024) void stream_read_kernel(const unsigned char* __restrict__ data,
                                                           int64_t row_bytes, int64_t stride,
                                                           uint32_t* __restrict__ out) {
  typedef uint32_t v4 __attribute__((ext_vector_type(4)));
  const v4* row = reinterpret_cast<const v4*>(data + (int64_t)blockIdx.x * stride);
  const int64_t nvec = row_bytes / 16;
  constexpr int G = 8;
  v4 acc = {0u, 0u, 0u, 0u};
  for (int64_t v0 = threadIdx.x; v0 < nvec; v0 += (int64_t)1024 * G) {
    v4 q[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int64_t v = v0 + (int64_t)g * 1024;
      q[g] = v < nvec ? __builtin_nontemporal_load(row + v) : v4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int g = 0; g < G; ++g) acc ^= q[g];
  }
  const uint32_t x = acc.x ^ acc.y ^ acc.z ^ acc.w;
  if (x == 0x9E3779B9u) out[blockIdx.x] = x;
}
}  // namespace gtp

extern "C" int gtp_stream_read_rows(const void* data, int64_t rows, int64_t row_bytes,
                                    int64_t row_stride_bytes, uint32_t* out, void* stream) {
  if (rows < 0 || row_bytes < 0 || row_stride_bytes < row_bytes || (rows > 0 && (!data || !out)))
    return GTP_ERR_INVALID_ARGUMENT;
  if ((reinterpret_cast<uintptr_t>(data) & 15u) || (row_bytes & 15) || (row_stride_bytes & 15))
    return GTP_ERR_UNSUPPORTED;
  if (rows > 0x7FFFFFFFll) return GTP_ERR_UNSUPPORTED;
  if (rows == 0 || row_bytes == 0) return GTP_OK;
  launch_timed(stream_read_kernel, dim3((unsigned)rows), dim3(1024),
               reinterpret_cast<hipStream_t>(stream), reinterpret_cast<const unsigned char*>(data),
               row_bytes, row_stride_bytes, out);
  return hipGetLastError() == hipSuccess ? GTP_OK : GTP_ERR_LAUNCH;
}

extern "C" int gtp_lse_partial_rows(const void* logits, int dtype, int64_t N, int64_t Vc,
                                    int64_t row_stride, int64_t col_offset, const void* targets,
                                    int targets_int64, float* state, int accumulate, void* stream) {
  if (N < 0 || Vc <= 0 || row_stride < Vc || col_offset < 0 || (N > 0 && (!logits || !state)))
    return GTP_ERR_INVALID_ARGUMENT;
  if (N > 0x7FFFFFFFll) return GTP_ERR_UNSUPPORTED;
  if (N == 0) return GTP_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)N), block(kLpBlock);
  switch (dtype) {
    case GTP_DTYPE_BF16:
      hipLaunchKernelGGL(lse_partial_kernel<uint16_t>, grid, block, 0, s,
                         reinterpret_cast<const uint16_t*>(logits), Vc, row_stride, col_offset,
                         targets, targets_int64, state, accumulate);
      break;
    case GTP_DTYPE_F16:
      hipLaunchKernelGGL(lse_partial_kernel<_Float16>, grid, block, 0, s,
                         reinterpret_cast<const _Float16*>(logits), Vc, row_stride, col_offset,
                         targets, targets_int64, state, accumulate);
      break;
    case GTP_DTYPE_F32:
      hipLaunchKernelGGL(lse_partial_kernel<float>, grid, block, 0, s,
                         reinterpret_cast<const float*>(logits), Vc, row_stride, col_offset,
                         targets, targets_int64, state, accumulate);
      break;
    default:
      return GTP_ERR_INVALID_ARGUMENT;
  }
  return hipGetLastError() == hipSuccess ? GTP_OK : GTP_ERR_LAUNCH;
}

extern "C" int gtp_lse_finalize_rows(const float* state, int64_t N, float* out_logprob,
                                     float* out_entropy, void* stream) {
  if (N < 0 || (N > 0 && !state)) return GTP_ERR_INVALID_ARGUMENT;
  if (N > 0x7FFFFFFFll) return GTP_ERR_UNSUPPORTED;
  if (N == 0) return GTP_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const unsigned blocks = (unsigned)((N + 255) / 256);
  hipLaunchKernelGGL(lse_finalize_kernel, dim3(blocks), dim3(256), 0, s, state, N, out_logprob,
                     out_entropy);
  return hipGetLastError() == hipSuccess ? GTP_OK : GTP_ERR_LAUNCH;
}

extern "C" const char* gtp_version(void) { return "graspo_tokpath 0.2 gfx950"; }

extern "C" int gtp_logprob_backward_split_rows(const float* logits, int64_t N, int64_t V,
                                               int64_t row_stride, int64_t col_offset,
                                               const void* targets, int targets_int64,
                                               const float* grad_logprob, const float* lse,
                                               uint16_t* grad_hi, uint16_t* grad_lo,
                                               int64_t grad_stride, void* stream) {
  if (N < 0 || V <= 0 || row_stride < V || grad_stride < V ||
      (N > 0 && (!logits || !targets || !grad_logprob || !lse || !grad_hi || !grad_lo)))
    return GTP_ERR_INVALID_ARGUMENT;
  if (N > 0x7FFFFFFFll) return GTP_ERR_UNSUPPORTED;
  if (N == 0) return GTP_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(logprob_backward_split_kernel, dim3((unsigned)N), dim3(kLpBlock), 0, s,
                     logits, V, row_stride, col_offset, targets, targets_int64, grad_logprob,
                     lse, grad_hi, grad_lo, grad_stride);
  return hipGetLastError() == hipSuccess ? GTP_OK : GTP_ERR_LAUNCH;
}

// bf16(-g_n p) of vocabulary-major fp32 logits, p = exp(x_t[v, n] - lse_n):
// the softmax part of g_n ([v == t_n] - p) without the one-hot term, which
// the caller adds in fp32 (it is the one term of a token's gradient near g
// in size; here every element is g p, rounded once to bf16, within 2^-8 of
// it).  A workgroup takes 1024 consecutive tokens (4 per thread, their g and
// lse held in registers) of kSgRows vocabulary rows; a token with g == 0
// gets zeros.
constexpr int kSgRows = 16;
typedef float f32x4v __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void softmax_grad_bf16_cols_kernel(
    const float* __restrict__ logits_t, int64_t V, int64_t N, int64_t ld,
    const float* __restrict__ grad_lp, const float* __restrict__ lse_in,
    uint16_t* __restrict__ grad_t, int64_t gld, int vec) {
  const int64_t n0 = (int64_t)blockIdx.x * 1024 + threadIdx.x * 4;
  if (n0 >= N) return;
  const int64_t v0 = (int64_t)blockIdx.y * kSgRows;
  const int cnt = (int)min((int64_t)4, N - n0);
  float ng[4], c[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float g = j < cnt ? grad_lp[n0 + j] : 0.0f;
    ng[j] = -g;
    // a token with g == 0 gets exactly zero
    c[j] = g == 0.0f ? kNegInf : (j < cnt ? lse_in[n0 + j] : 0.0f);
  }
  // x - lse first: exact for x near lse at any magnitude
  auto grad_of = [&](float x, int j) {
    return c[j] == kNegInf ? 0.0f : ng[j] * __builtin_amdgcn_exp2f((x - c[j]) * kLog2e);
  };
  if (vec && cnt == 4) {
#pragma unroll 4
    for (int r = 0; r < kSgRows; ++r) {
      const int64_t v = v0 + r;
      if (v >= V) break;
      const f32x4v x = __builtin_nontemporal_load(reinterpret_cast<const f32x4v*>(logits_t + v * ld + n0));
      const u32x2 o = {bf16_rne(grad_of(x.x, 0)) | (bf16_rne(grad_of(x.y, 1)) << 16),
                       bf16_rne(grad_of(x.z, 2)) | (bf16_rne(grad_of(x.w, 3)) << 16)};
      __builtin_nontemporal_store(o, reinterpret_cast<u32x2*>(grad_t + v * gld + n0));
    }
    return;
  }
  for (int r = 0; r < kSgRows; ++r) {
    const int64_t v = v0 + r;
    if (v >= V) break;
    for (int j = 0; j < cnt; ++j)
      grad_t[v * gld + n0 + j] = (uint16_t)bf16_rne(grad_of(logits_t[v * ld + n0 + j], j));
  }
}

// The same values written token-major as well, grad_n[n, v] (and, unless
// grad_t is null, vocabulary-major as above), from one read of the logits: a
// workgroup takes 256 tokens x 64 vocabulary rows.  Each thread computes 4
// consecutive tokens of 16 rows (16-byte loads along the tokens, 8-byte
// vocabulary-major stores) and puts them in an LDS tile [64][256 + 2]; then
// each group of 8 lanes writes one token's 64 values, a whole 128-byte line,
// 16 bytes a lane.  The tile's row pitch of 129 words puts the 8 rows a group
// reads at once on distinct banks.
constexpr int kDgTok = 256, kDgRows = 64, kDgPitch = kDgTok + 2;
__global__ __launch_bounds__(256) void softmax_grad_bf16_dual_kernel(
    const float* __restrict__ logits_t, int64_t V, int64_t N, int64_t ld,
    const float* __restrict__ grad_lp, const float* __restrict__ lse_in,
    uint16_t* __restrict__ grad_t, int64_t gld, uint16_t* __restrict__ grad_n, int64_t nld,
    int vec) {
  __shared__ __attribute__((aligned(16))) uint16_t tile[kDgRows * kDgPitch];
  const int t = threadIdx.x;
  const int64_t nb = (int64_t)blockIdx.x * kDgTok, vb = (int64_t)blockIdx.y * kDgRows;
  const int nl = (t & 63) * 4;  // the thread's first token in the tile
  const int64_t n0 = nb + nl;
  const int cnt = (int)max((int64_t)0, min((int64_t)4, N - n0));
  float ng[4], c[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float g = j < cnt ? grad_lp[n0 + j] : 0.0f;
    ng[j] = -g;
    c[j] = g == 0.0f ? kNegInf : (j < cnt ? lse_in[n0 + j] : 0.0f);
  }
  auto grad_of = [&](float x, int j) {
    return c[j] == kNegInf ? 0.0f : ng[j] * __builtin_amdgcn_exp2f((x - c[j]) * kLog2e);
  };
#pragma unroll 4
  for (int i = 0; i < kDgRows / 4; ++i) {
    const int r = (t >> 6) + 4 * i;
    const int64_t v = vb + r;
    uint32_t o[4] = {0u, 0u, 0u, 0u};
    if (v < V) {
      if (vec && cnt == 4) {
        const f32x4v x = __builtin_nontemporal_load(reinterpret_cast<const f32x4v*>(logits_t + v * ld + n0));
        o[0] = bf16_rne(grad_of(x.x, 0));
        o[1] = bf16_rne(grad_of(x.y, 1));
        o[2] = bf16_rne(grad_of(x.z, 2));
        o[3] = bf16_rne(grad_of(x.w, 3));
        if (grad_t) {
          const u32x2 w = {o[0] | (o[1] << 16), o[2] | (o[3] << 16)};
          __builtin_nontemporal_store(w, reinterpret_cast<u32x2*>(grad_t + v * gld + n0));
        }
      } else {
        for (int j = 0; j < cnt; ++j) {
          o[j] = bf16_rne(grad_of(logits_t[v * ld + n0 + j], j));
          if (grad_t) grad_t[v * gld + n0 + j] = (uint16_t)o[j];
        }
      }
    }
    uint32_t* dst = reinterpret_cast<uint32_t*>(tile + r * kDgPitch + nl);
    dst[0] = o[0] | (o[1] << 16);
    dst[1] = o[2] | (o[3] << 16);
  }
  __syncthreads();
  // token-major: 8 lanes per token, lane c8 of the group the values of rows
  // 8 c8 .. 8 c8 + 7, 32 tokens per pass
  const int c8 = t & 7;
  const int64_t nv = min((int64_t)kDgRows, V - vb);
#pragma unroll 2
  for (int p = 0; p < kDgTok / 32; ++p) {
    const int tl = p * 32 + (t >> 3);
    const int64_t n = nb + tl;
    if (n >= N) break;
    uint16_t* row = grad_n + n * nld + vb;
    if (vec && nv == kDgRows) {
      uint32_t h[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) h[k] = tile[(8 * c8 + k) * kDgPitch + tl];
      const u32x4 w = {h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16),
                       h[6] | (h[7] << 16)};
      *reinterpret_cast<u32x4*>(row + 8 * c8) = w;
    } else {
      for (int k = 0; k < 8; ++k)
        if (8 * c8 + k < nv) row[8 * c8 + k] = tile[(8 * c8 + k) * kDgPitch + tl];
    }
  }
}

extern "C" int gtp_softmax_grad_bf16_cols(const float* logits_t, int64_t V, int64_t N,
                                          int64_t logits_stride, const float* grad_logprob,
                                          const float* lse, uint16_t* grad_t, int64_t grad_stride,
                                          uint16_t* grad_n, int64_t grad_n_stride,
                                          void* stream) {
  if (N < 0 || V <= 0 || logits_stride < N || (grad_t && grad_stride < N) ||
      (grad_n && grad_n_stride < V) ||
      (N > 0 && (!logits_t || !grad_logprob || !lse || (!grad_t && !grad_n))))
    return GTP_ERR_INVALID_ARGUMENT;
  if (N > 0x7FFFFFFFll || V > ((int64_t)65535 * kSgRows) ||
      logits_stride > ((int64_t)1 << 40) / V || (grad_t && grad_stride > ((int64_t)1 << 40) / V) ||
      (grad_n && (N > 0 && grad_n_stride > ((int64_t)1 << 40) / N)))
    return GTP_ERR_UNSUPPORTED;
  if (N == 0) return GTP_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool in_vec = (reinterpret_cast<uintptr_t>(logits_t) & 15u) == 0 && (logits_stride & 3) == 0;
  const bool t_vec = !grad_t || ((reinterpret_cast<uintptr_t>(grad_t) & 7u) == 0 && (grad_stride & 3) == 0);
  if (grad_n) {
    const int vec = in_vec && t_vec && (reinterpret_cast<uintptr_t>(grad_n) & 15u) == 0 &&
                            (grad_n_stride & 7) == 0
                        ? 1
                        : 0;
    const dim3 grid((unsigned)((N + kDgTok - 1) / kDgTok), (unsigned)((V + kDgRows - 1) / kDgRows));
    launch_timed(softmax_grad_bf16_dual_kernel, grid, dim3(256), s, logits_t, V, N, logits_stride,
                 grad_logprob, lse, grad_t, grad_stride, grad_n, grad_n_stride, vec);
  } else {
    const int vec = in_vec && t_vec ? 1 : 0;
    const dim3 grid((unsigned)((N + 1023) / 1024), (unsigned)((V + kSgRows - 1) / kSgRows));
    launch_timed(softmax_grad_bf16_cols_kernel, grid, dim3(256), s, logits_t, V, N, logits_stride,
                 grad_logprob, lse, grad_t, grad_stride, vec);
  }
  return hipGetLastError() == hipSuccess ? GTP_OK : GTP_ERR_LAUNCH;
}

extern "C" int gtp_logprob_backward_rows(const void* logits, int dtype, int64_t N, int64_t V,
                                         int64_t row_stride, int64_t col_offset,
                                         const void* targets, int targets_int64,
                                         const float* grad_logprob, const float* lse, void* grad,
                                         int64_t grad_stride, void* stream) {
  if (N < 0 || V <= 0 || row_stride < V || grad_stride < V ||
      (N > 0 && (!logits || !targets || !grad_logprob || !lse || !grad)))
    return GTP_ERR_INVALID_ARGUMENT;
  if (N > 0x7FFFFFFFll) return GTP_ERR_UNSUPPORTED;
  if (N == 0) return GTP_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)N), block(kLpBlock);
  switch (dtype) {
    case GTP_DTYPE_BF16:
      launch_timed(logprob_backward_kernel<uint16_t>, grid, block, s,
                         reinterpret_cast<const uint16_t*>(logits), V, row_stride, col_offset,
                         targets, targets_int64, grad_logprob, lse,
                         reinterpret_cast<uint16_t*>(grad), grad_stride);
      break;
    case GTP_DTYPE_F16:
      launch_timed(logprob_backward_kernel<_Float16>, grid, block, s,
                         reinterpret_cast<const _Float16*>(logits), V, row_stride, col_offset,
                         targets, targets_int64, grad_logprob, lse,
                         reinterpret_cast<_Float16*>(grad), grad_stride);
      break;
    case GTP_DTYPE_F32:
      launch_timed(logprob_backward_kernel<float>, grid, block, s,
                         reinterpret_cast<const float*>(logits), V, row_stride, col_offset,
                         targets, targets_int64, grad_logprob, lse,
                         reinterpret_cast<float*>(grad), grad_stride);
      break;
    default:
      return GTP_ERR_INVALID_ARGUMENT;
  }
  return hipGetLastError() == hipSuccess ? GTP_OK : GTP_ERR_LAUNCH;
}
