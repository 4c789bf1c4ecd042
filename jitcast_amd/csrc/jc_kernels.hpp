// Internal launchers of the gfx950 kernels (host side). Each validates nothing: the C-ABI layer
// (jc_abi.cpp) checks shapes, pointers and alignment before calling them.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace jc {

hipError_t c2_time_attention_f32_launch(const float* qkv, float* out, const int32_t* live, const float* table,
                                        int rows, int n, int heads, int dh, int inner, hipStream_t stream);
int c2_time_attention_max_tokens();
// bf16 (fp16 = false) or fp16 qkv/out, fp32 accumulation; dh a multiple of 16, at most 64
hipError_t c2_time_attention_lp_launch(const void* qkv, void* out, const int32_t* live, const float* table, int rows,
                                       int n, int heads, int dh, int inner, bool fp16, hipStream_t stream);
hipError_t c2_group_attention_f32_launch(const float* qkv, float* out, const int32_t* live, const int32_t* gs,
                                         const int32_t* ge, int rows, int n, int heads, int dh, int inner,
                                         hipStream_t stream);

hipError_t fill_normal_launch(float* out, uint64_t count, uint64_t stream_seed, double mean, double stdv,
                              hipStream_t stream);
hipError_t fill_uniform_launch(float* out, uint64_t count, uint64_t stream_seed, double lo, double hi,
                               hipStream_t stream);

}  // namespace jc
