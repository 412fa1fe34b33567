// tokpath_loss.hip -- the GRASPO PPO-clip loss over token logprobs, fused
// (gfx950).
//
// loss = mean_b ( sum_t m_bt l_bt / max(1, sum_t m_bt) ),
// l_bt = -min(r A, clip(r, lo, hi) A), r = exp(logp - logp_old),
// lo = 1 - eps, hi = 1 + eps (rounded to fp32 by the caller, as torch does),
// as the reference's chain of elementwise torch ops computes it
// (src/graspo/core/graspo_loss.py:10-16 masked_mean, :45-63 GRASPOLoss).
//
// Forward: one workgroup per sequence writes its masked mean; one wave
// then averages the sequences in a fixed order (deterministic, no atomics).
// Backward: dloss/dlogp_bt = g / B * m_bt / max(1, sum_t m_bt) * dl_bt/dlogp,
// with dl/dlogp = -A r where the minimum takes r A or r lies inside the
// clip range (torch's min splits a tie in halves of equal value, and
// clamp passes the gradient on its closed range), else 0.
//
// Non-finite values follow torch: min and clamp pass NaN through (fminf
// and fmaxf would drop it), a masked position still multiplies its loss by
// the mask (NaN * 0 = NaN poisons the sum, as (tensor * mask).sum() does),
// and the gradient is formed in autograd's order -- the minimum's gradient
// goes to both operands when they are unordered, clamp's to neither -- so
// a NaN or an inf reaches the same gradient positions.
#include "tokpath_common.h"

namespace gtp {

constexpr int kLsBlock = 256;

__device__ __forceinline__ float block_sum_256(float v, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float s = 0.0f;
#pragma unroll
  for (int w = 0; w < kLsBlock / kWave; ++w) s += red[w];
  __syncthreads();
  return s;
}

// torch.minimum: NaN if either operand is NaN
__device__ __forceinline__ float min_nan(float a, float b) {
  return (a != a || b != b) ? a + b : (a < b ? a : b);
}
// torch.clamp(r, lo, hi) with finite bounds: NaN stays NaN
__device__ __forceinline__ float clamp_nan(float r, float lo, float hi) {
  return r != r ? r : fminf(fmaxf(r, lo), hi);
}

// action mask: fp32 weights, bytes (bool, 0 or 1), or none (all ones)
struct MaskIn {
  const void* p;
  int kind;  // 0: fp32, 1: uint8
  __device__ __forceinline__ float at(int64_t i) const {
    if (!p) return 1.0f;
    return kind ? (reinterpret_cast<const uint8_t*>(p)[i] ? 1.0f : 0.0f)
                : reinterpret_cast<const float*>(p)[i];
  }
};

__global__ __launch_bounds__(kLsBlock) void graspo_loss_rows_kernel(
    const float* __restrict__ logp, const float* __restrict__ old_logp,
    const float* __restrict__ adv, MaskIn mask, int64_t T, float lo, float hi,
    float* __restrict__ per_seq, float* __restrict__ inv_denom) {
  __shared__ float red[kLsBlock / kWave];
  const int64_t b = blockIdx.x;
  float s = 0.0f, d = 0.0f;
  for (int64_t t = threadIdx.x; t < T; t += kLsBlock) {
    const int64_t i = b * T + t;
    const float m = mask.at(i);
    const float r = expf(logp[i] - old_logp[i]);
    const float A = adv[i];
    const float s1 = r * A;
    const float s2 = clamp_nan(r, lo, hi) * A;
    s += -min_nan(s1, s2) * m;
    d += m;
  }
  s = block_sum_256(s, red);
  d = block_sum_256(d, red);
  if (threadIdx.x == 0) {
    const float den = fmaxf(d, 1.0f);
    per_seq[b] = s / den;
    inv_denom[b] = 1.0f / den;
  }
}

// mean over the B sequences (one wave, fixed order)
__global__ __launch_bounds__(kWave) void graspo_loss_mean_kernel(const float* __restrict__ per_seq,
                                                                 int64_t B, float* __restrict__ out) {
  float s = 0.0f;
  for (int64_t b = threadIdx.x; b < B; b += kWave) s += per_seq[b];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, kWave);
  if (threadIdx.x == 0) out[0] = s / (float)B;
}

__global__ __launch_bounds__(kLsBlock) void graspo_loss_backward_kernel(
    const float* __restrict__ logp, const float* __restrict__ old_logp,
    const float* __restrict__ adv, MaskIn mask,
    const float* __restrict__ inv_denom, const float* __restrict__ grad_loss, int64_t B,
    int64_t T, float lo, float hi, float* __restrict__ grad_logp) {
  const int64_t n = (int64_t)blockIdx.x * kLsBlock + threadIdx.x;
  if (n >= B * T) return;
  const int64_t b = n / T;
  const float m = mask.at(n);
  const float r = expf(logp[n] - old_logp[n]);
  const float A = adv[n];
  const float s1 = r * A;
  const float s2 = clamp_nan(r, lo, hi) * A;
  // d loss_bt: the mean over sequences, the masked mean and the negation
  const float gl = -(grad_loss[0] / (float)B * inv_denom[b] * m);
  // torch.minimum's backward: all to the smaller operand, halves on a tie,
  // the whole to both when the comparison is unordered (a NaN)
  float w1 = 1.0f, w2 = 1.0f;
  if (s1 < s2) w2 = 0.0f;
  else if (s1 > s2) w1 = 0.0f;
  else if (s1 == s2) w1 = w2 = 0.5f;
  const float g2 = (r >= lo && r <= hi) ? (w2 * gl) * A : 0.0f;  // clamp passes [lo, hi]
  grad_logp[n] = ((w1 * gl) * A + g2) * r;                        // exp's backward: * r
}

}  // namespace gtp

using namespace gtp;

extern "C" int gtp_graspo_loss_forward(const float* logp, const float* old_logp, const float* adv,
                                       const void* mask, int mask_u8, int64_t B, int64_t T, float clip_lo,
                                       float clip_hi, float* out_loss, float* per_seq, float* inv_denom,
                                       void* stream) {
  if (B <= 0 || T <= 0 || !logp || !old_logp || !adv || !out_loss || !per_seq || !inv_denom)
    return GTP_ERR_INVALID_ARGUMENT;
  if (B > 0x7FFFFFFFll) return GTP_ERR_UNSUPPORTED;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(graspo_loss_rows_kernel, dim3((unsigned)B), dim3(kLsBlock), 0, s, logp,
                     old_logp, adv, MaskIn{mask, mask_u8 ? 1 : 0}, T, clip_lo, clip_hi, per_seq,
                     inv_denom);
  hipLaunchKernelGGL(graspo_loss_mean_kernel, dim3(1), dim3(kWave), 0, s, per_seq, B, out_loss);
  return hipGetLastError() == hipSuccess ? GTP_OK : GTP_ERR_LAUNCH;
}

extern "C" int gtp_graspo_loss_backward(const float* logp, const float* old_logp,
                                        const float* adv, const void* mask, int mask_u8,
                                        const float* inv_denom, const float* grad_loss,
                                        int64_t B, int64_t T, float clip_lo, float clip_hi,
                                        float* grad_logp, void* stream) {
  if (B <= 0 || T <= 0 || !logp || !old_logp || !adv || !inv_denom || !grad_loss || !grad_logp)
    return GTP_ERR_INVALID_ARGUMENT;
  if (T > (int64_t)0x7FFFFFFF * kLsBlock / B) return GTP_ERR_UNSUPPORTED;  // grid <= 2^31 - 1
  const int64_t n = B * T;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(graspo_loss_backward_kernel, dim3((unsigned)((n + kLsBlock - 1) / kLsBlock)),
                     dim3(kLsBlock), 0, s, logp, old_logp, adv, MaskIn{mask, mask_u8 ? 1 : 0},
                     inv_denom, grad_loss, B, T,
                     clip_lo, clip_hi, grad_logp);
  return hipGetLastError() == hipSuccess ? GTP_OK : GTP_ERR_LAUNCH;
}
