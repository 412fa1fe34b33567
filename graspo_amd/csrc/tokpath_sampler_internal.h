// tokpath_sampler_internal.h -- pieces shared by the sampler's two paths
// (tokpath_sampler.hip: one workgroup per row, any shape; tokpath_sampler_fast.hip:
// vocabulary split over workgroups with a last-arriving-workgroup merge).
#pragma once

#include "tokpath_common.h"

namespace gtp {

struct SamplerArgs {
  const void* logits;
  int64_t V;
  int64_t row_stride;
  const int32_t* hist;
  int64_t hist_len;
  int64_t hist_stride;
  const uint32_t* mask;
  int64_t mask_stride;
  const float* uniforms;
  float T;
  int32_t K;
  float P;
  float rho;
  const uint8_t* finished;
  int64_t pad_id;
  int64_t* out_ids;
  float* out_lp;
  float* out_slp;
  int32_t* out_kept;
  float* out_tv;
  int32_t* out_tid;
  int32_t* out_status;
};

// One workgroup of 1024 threads per row (any layout, V <= GTP_SAMPLER_MAX_V).
int launch_sampler_general(const SamplerArgs& a, int dtype, int64_t B, hipStream_t s);

}  // namespace gtp
