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
  const float mL = st.m == kNegInf ? 0.0f : st.m * kLog2e;
  const float d = __builtin_fmaf(x, kLog2e, -mL);
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
    out_lp[n] = tgt_ok ? xt - st.m - ln_s : __builtin_nanf("");
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
  if (out_lp) out_lp[n] = xt - m - ln_s;
  if (out_H) out_H[n] = ln_s - t / s;
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
      hipLaunchKernelGGL(logprob_entropy_kernel<uint16_t>, grid, block, 0, s,
                         reinterpret_cast<const uint16_t*>(logits), V, row_stride, targets,
                         targets_int64, out_logprob, out_entropy, out_status);
      break;
    case GTP_DTYPE_F16:
      hipLaunchKernelGGL(logprob_entropy_kernel<_Float16>, grid, block, 0, s,
                         reinterpret_cast<const _Float16*>(logits), V, row_stride, targets,
                         targets_int64, out_logprob, out_entropy, out_status);
      break;
    case GTP_DTYPE_F32:
      hipLaunchKernelGGL(logprob_entropy_kernel<float>, grid, block, 0, s,
                         reinterpret_cast<const float*>(logits), V, row_stride, targets,
                         targets_int64, out_logprob, out_entropy, out_status);
      break;
    default:
      return GTP_ERR_INVALID_ARGUMENT;
  }
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
  if (N == 0) return GTP_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const unsigned blocks = (unsigned)((N + 255) / 256);
  hipLaunchKernelGGL(lse_finalize_kernel, dim3(blocks), dim3(256), 0, s, state, N, out_logprob,
                     out_entropy);
  return hipGetLastError() == hipSuccess ? GTP_OK : GTP_ERR_LAUNCH;
}

extern "C" const char* gtp_version(void) { return "graspo_tokpath 0.2 gfx950"; }
