// tokpath_logprob.hip -- selective log-softmax gather + softmax entropy (gfx950).
//
// One workgroup of 256 threads streams one row once.  Each thread keeps an
// online (m, s, t) state in base-2 units:
//   d_i = (x_i - m) * log2(e),  s = sum 2^{d_i},  t = sum 2^{d_i} * d_i
// so logprob = x_target - m - ln s and entropy = ln s - ln2 * t / s.
// Loads are 16-byte vectors (8 bf16/fp16 or 4 fp32), eight groups per thread
// in flight; the row is never written back (no [N, V] log-softmax), so the
// kernel is bounded by one HBM read of the logits.
//
// Replaces sequence_log_probs_from_logits (src/graspo/core/graspo_loss.py:19-21)
// and the logsumexp / logaddexp chunk loop of _selected_token_log_probs_from_hidden
// (src/graspo/backends/graspoflow/tensor_utils.py:180-186).
#include "tokpath_common.h"

namespace gtp {

constexpr int kLpBlock = 256;
constexpr int kLpGroups = 8;  // groups of 8 logits per thread per iteration

struct LpState {
  float m;  // running max (natural units)
  float s;  // sum 2^d
  float t;  // sum 2^d * d
};

__device__ __forceinline__ LpState lp_merge(LpState a, LpState b) {
  if (a.s != a.s || b.s != b.s) return {fmaxf(a.m, b.m), __builtin_nanf(""), __builtin_nanf("")};
  const float m = fmaxf(a.m, b.m);
  if (m == kNegInf) return {kNegInf, 0.0f, 0.0f};
  float s = 0.0f, t = 0.0f;
  if (a.s > 0.0f) {
    const float da = (a.m - m) * kLog2e;  // <= 0
    const float fa = __builtin_amdgcn_exp2f(da);
    s += a.s * fa;
    t += fa * (a.t + da * a.s);
  }
  if (b.s > 0.0f) {
    const float db = (b.m - m) * kLog2e;
    const float fb = __builtin_amdgcn_exp2f(db);
    s += b.s * fb;
    t += fb * (b.t + db * b.s);
  }
  return {m, s, t};
}

// Fold 8*NG logits of one thread into its state.
template <int NG>
__device__ __forceinline__ void lp_fold(LpState& st, const float (&x)[NG][8]) {
  float cm = kNegInf;
#pragma unroll
  for (int k = 0; k < NG; ++k) cm = fmaxf(cm, max8(x[k]));
  const float mn = fmaxf(st.m, cm);
  if (mn == kNegInf) return;  // only -inf (or NaN, caught below) so far
  if (mn != st.m && st.s > 0.0f) {
    const float dl = (st.m - mn) * kLog2e;
    const float f = __builtin_amdgcn_exp2f(dl);
    st.t = f * (st.t + dl * st.s);
    st.s = st.s * f;
  }
  st.m = mn;
  const float mL = mn * kLog2e;
  float s = 0.0f, t = 0.0f;
#pragma unroll
  for (int k = 0; k < NG; ++k) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float d = __builtin_fmaf(x[k][j], kLog2e, -mL);
      const float e = __builtin_amdgcn_exp2f(d);  // NaN stays NaN
      s += e;
      t = __builtin_fmaf(e, fmaxf(d, -256.0f), t);  // -inf logits add 0
    }
  }
  st.s += s;
  st.t += t;
}

// NaN logits never move the max (fmaxf skips NaN) but poison s: detect it.
template <int NG>
__device__ __forceinline__ void lp_fold_nan_guard(LpState& st, const float (&x)[NG][8]) {
  if (st.m == kNegInf) {
    // all -inf so far: lp_fold returns early, so NaNs must be caught here
    bool nan = false;
#pragma unroll
    for (int k = 0; k < NG; ++k)
#pragma unroll
      for (int j = 0; j < 8; ++j) nan |= (x[k][j] != x[k][j]);
    if (nan) st.s = __builtin_nanf("");
  }
  lp_fold<NG>(st, x);
}

template <typename T>
__device__ LpState lp_row_state(const T* __restrict__ row, int64_t V) {
  const int tid = threadIdx.x;
  const bool vec_ok = (reinterpret_cast<uintptr_t>(row) & 15u) == 0;
  const int64_t ngroups = (V + 7) / 8;
  const int64_t nfull = vec_ok ? V / 8 : 0;  // groups loadable as vectors
  constexpr int64_t kStep = (int64_t)kLpBlock * kLpGroups;
  LpState st{kNegInf, 0.0f, 0.0f};
  int64_t base = 0;
  for (; base + kStep <= nfull; base += kStep) {
    float x[kLpGroups][8];
#pragma unroll
    for (int k = 0; k < kLpGroups; ++k) Elem<T>::group(row + (base + k * kLpBlock + tid) * 8, x[k]);
    lp_fold_nan_guard<kLpGroups>(st, x);
  }
  for (; base < ngroups; base += kStep) {
    float x[kLpGroups][8];
#pragma unroll
    for (int k = 0; k < kLpGroups; ++k) {
      const int64_t G = base + k * kLpBlock + tid;
      if (G < ngroups) {
        load_group<T>(row, G, V, vec_ok, x[k]);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) x[k][j] = kNegInf;
      }
    }
    lp_fold_nan_guard<kLpGroups>(st, x);
  }
  return st;
}

__device__ __forceinline__ LpState lp_block_reduce(LpState st) {
  __shared__ float sm[kLpBlock / kWave][3];
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    LpState w{__shfl_xor(st.m, o, kWave), __shfl_xor(st.s, o, kWave), __shfl_xor(st.t, o, kWave)};
    st = lp_merge(st, w);
  }
  if (lane == 0) {
    sm[wid][0] = st.m;
    sm[wid][1] = st.s;
    sm[wid][2] = st.t;
  }
  __syncthreads();
  LpState r{sm[0][0], sm[0][1], sm[0][2]};
#pragma unroll
  for (int w = 1; w < kLpBlock / kWave; ++w) r = lp_merge(r, LpState{sm[w][0], sm[w][1], sm[w][2]});
  return r;
}

__device__ __forceinline__ int64_t load_target(const void* targets, int t64, int64_t n) {
  return t64 ? reinterpret_cast<const int64_t*>(targets)[n]
             : (int64_t)reinterpret_cast<const int32_t*>(targets)[n];
}

template <typename T>
__global__ __launch_bounds__(kLpBlock) void logprob_entropy_kernel(
    const T* __restrict__ logits, int64_t V, int64_t row_stride, const void* __restrict__ targets,
    int t64, float* __restrict__ out_lp, float* __restrict__ out_H, int32_t* __restrict__ out_status) {
  const int64_t n = blockIdx.x;
  const T* row = logits + n * row_stride;
  const int64_t tgt = load_target(targets, t64, n);
  const bool tgt_ok = tgt >= 0 && tgt < V;
  float xt = 0.0f;
  if (threadIdx.x == 0 && tgt_ok) xt = Elem<T>::get(row, tgt);
  LpState st = lp_block_reduce(lp_row_state<T>(row, V));
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
  const int64_t n = blockIdx.x;
  const T* row = logits + n * row_stride;
  const int64_t tgt = targets ? load_target(targets, t64, n) - col_offset : -1;
  LpState st = lp_block_reduce(lp_row_state<T>(row, Vc));
  if (threadIdx.x == 0) {
    float* sp = state + n * 4;
    float xt = __builtin_nanf("");
    if (accumulate) {
      LpState old{sp[0], sp[1], sp[2] * kLog2e};
      st = lp_merge(old, st);
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

extern "C" const char* gtp_version(void) { return "graspo_tokpath 0.1 gfx950"; }
