// tokpath_narrow.hip -- exact fp32 -> bf16 narrowing with an exactness flag
// (gfx950).
//
// The reference's hidden-state logprob path receives fp32 copies of bf16
// tensors (hidden[:, :-1].float(), lm_head.weight.float(); qwen3/model.py:
// 361-365, qwen35_36/training.py:619-623) and runs its vocabulary-chunk GEMMs
// in fp32 (tensor_utils.py:180-184).  When every value is a bf16 value, the
// same products are exact in a bf16 x bf16 -> fp32 matrix-core GEMM; this
// kernel recovers the bf16 operands in one HBM pass (read 4 B, write 2 B per
// element) and reports whether any value was not a bf16 value (its low 16
// bits not zero), in which case the caller keeps the fp32 path.
#include "tokpath_stream.h"

namespace gtp {

constexpr int kNbBlock = 256;
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__global__ __launch_bounds__(kNbBlock) void narrow_bf16_vec_kernel(const u32x4* __restrict__ src,
                                                                   int64_t n4,
                                                                   u32x2* __restrict__ dst,
                                                                   uint32_t* __restrict__ inexact) {
  // kU 16-byte loads in flight per thread: one at a time left the pass
  // latency-bound at about 3.3 TB/s
  constexpr int kU = 4;
  uint32_t low = 0;
  const int64_t step = (int64_t)gridDim.x * kNbBlock;
  for (int64_t i0 = (int64_t)blockIdx.x * kNbBlock + threadIdx.x; i0 < n4; i0 += step * kU) {
    u32x4 v[kU];
#pragma unroll
    for (int q = 0; q < kU; ++q) {
      const int64_t i = i0 + q * step;
      v[q] = i < n4 ? __builtin_nontemporal_load(src + i) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int q = 0; q < kU; ++q) {
      const int64_t i = i0 + q * step;
      low |= (v[q].x | v[q].y | v[q].z | v[q].w) & 0xFFFFu;
      u32x2 o;
      o.x = (v[q].x >> 16) | (v[q].y & 0xFFFF0000u);
      o.y = (v[q].z >> 16) | (v[q].w & 0xFFFF0000u);
      if (i < n4) __builtin_nontemporal_store(o, dst + i);
    }
  }
  if (__ballot(low != 0u) && (threadIdx.x & (kWave - 1)) == 0) atomicOr(inexact, 1u);
}

// any alignment and the elements past the last whole group of four
__global__ __launch_bounds__(kNbBlock) void narrow_bf16_scalar_kernel(
    const uint32_t* __restrict__ src, int64_t i0, int64_t n, uint16_t* __restrict__ dst,
    uint32_t* __restrict__ inexact) {
  uint32_t low = 0;
  const int64_t step = (int64_t)gridDim.x * kNbBlock;
  for (int64_t i = i0 + (int64_t)blockIdx.x * kNbBlock + threadIdx.x; i < n; i += step) {
    const uint32_t v = src[i];
    low |= v & 0xFFFFu;
    dst[i] = (uint16_t)(v >> 16);
  }
  if (__ballot(low != 0u) && (threadIdx.x & (kWave - 1)) == 0) atomicOr(inexact, 1u);
}

}  // namespace gtp

using namespace gtp;

extern "C" int gtp_f32_to_bf16_exact(const float* src, int64_t n, uint16_t* dst,
                                     uint32_t* inexact, void* stream) {
  if (n < 0 || !inexact || (n > 0 && (!src || !dst))) return GTP_ERR_INVALID_ARGUMENT;
  if (n > ((int64_t)1 << 56)) return GTP_ERR_UNSUPPORTED;  // beyond any address space
  if (n == 0) return GTP_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool aligned = (reinterpret_cast<uintptr_t>(src) & 15u) == 0 &&
                       (reinterpret_cast<uintptr_t>(dst) & 7u) == 0;
  int64_t done = 0;
  if (aligned) {
    const int64_t n4 = n / 4;
    if (n4 > 0) {
      const int64_t want = (n4 + kNbBlock - 1) / kNbBlock;
      const unsigned grid = (unsigned)(want < 8192 ? want : 8192);  // 32 workgroups per CU
      hipLaunchKernelGGL(narrow_bf16_vec_kernel, dim3(grid), dim3(kNbBlock), 0, s,
                         reinterpret_cast<const u32x4*>(src), n4, reinterpret_cast<u32x2*>(dst),
                         inexact);
    }
    done = n4 * 4;
  }
  if (done < n) {
    const int64_t rest = n - done;
    const int64_t want = (rest + kNbBlock - 1) / kNbBlock;
    const unsigned grid = (unsigned)(want < 8192 ? want : 8192);
    hipLaunchKernelGGL(narrow_bf16_scalar_kernel, dim3(grid), dim3(kNbBlock), 0, s,
                       reinterpret_cast<const uint32_t*>(src), done, n, dst, inexact);
  }
  return hipGetLastError() == hipSuccess ? GTP_OK : GTP_ERR_LAUNCH;
}
