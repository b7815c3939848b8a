// kernels.hpp -- host-side launchers of the fused-group kernels (internal).
// The C-ABI layer (abi.hip) validates descriptors, then calls these with
// plain device pointers and int32 sizes (every tensor is checked to hold
// fewer than 2^31 elements before a launch).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace npu {

struct MatmulArgs {
  const float *A, *B, *bias;  // bias may be null
  float *out;
  int M, N, K, act;
};
hipError_t launch_matmul_bias_act_f32(const MatmulArgs &a, hipStream_t s);

struct ConvArgs {
  const void *x, *w;   // f32 or bf16 (uint16 bits)
  const float *bias;   // may be null
  void *out;
  int N, H, W, C, F, KH, KW, pad, Ho, Wo, act;
};
hipError_t launch_conv2d_nhwc_f32(const ConvArgs &a, hipStream_t s);
hipError_t launch_conv2d_nhwc_bf16(const ConvArgs &a, hipStream_t s);

}  // namespace npu
