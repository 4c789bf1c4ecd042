// Internal launchers of the gfx950 kernels (host side). Each validates nothing: the C-ABI layer
// (jc_abi.cpp) checks shapes, pointers and alignment before calling them.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "time_mask.hpp"

namespace jc {

// Chronos-2 (ts = false) or Timestral (ts = true) time attention (time_mask.hpp); a.qgroups is set
// by the launcher. fp32: dh a multiple of 8, at most 128; bf16/fp16: a multiple of 16, at most 128.
hipError_t time_attention_f32_launch(const TimeArgs& a, int dh, bool ts, hipStream_t stream);
hipError_t time_attention_lp_launch(const TimeArgs& a, int dh, bool ts, bool fp16, hipStream_t stream);
int time_attention_max_tokens();
// att[i] *= sigmoid(g[i]) for i < count (dtype: 0 fp32, 1 bf16, 2 fp16)
hipError_t gate_launch(void* att, const void* g, uint64_t count, int dtype, hipStream_t stream);
hipError_t c2_group_attention_f32_launch(const float* qkv, float* out, const int32_t* live, const int32_t* gs,
                                         const int32_t* ge, int rows, int n, int heads, int dh, int inner,
                                         hipStream_t stream);

hipError_t fill_normal_launch(float* out, uint64_t count, uint64_t stream_seed, double mean, double stdv,
                              hipStream_t stream);
hipError_t fill_uniform_launch(float* out, uint64_t count, uint64_t stream_seed, double lo, double hi,
                               hipStream_t stream);

}  // namespace jc
