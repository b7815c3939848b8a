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
  const void *res = nullptr;  // residual [N,Ho,Wo,F], the output's type (may be null)
  int stride = 1;             // both spatial dimensions (the NCHW kernels; NHWC takes 1)
};
hipError_t launch_conv2d_nhwc_f32(const ConvArgs &a, hipStream_t s);
hipError_t launch_conv2d_nhwc_bf16(const ConvArgs &a, hipStream_t s);
// NCHW activations, FCHW filters (conv_2d_nchw_fchw), f32, any filter size
// and stride: ConvArgs with H/W/C/F as named, x [N,C,H,W], w [F,C,KH,KW],
// out and res [N,F,Ho,Wo].
hipError_t launch_conv2d_nchw_f32(const ConvArgs &a, hipStream_t s);
// 3x3 / stride 1 / pad 1 with rows of at most 64 pixels: LDS halo kernel.
bool conv3x3_rows_supported(const ConvArgs &a, int elem_bytes);
hipError_t launch_conv3x3_f32(const ConvArgs &a, hipStream_t s);
hipError_t launch_conv3x3_bf16(const ConvArgs &a, hipStream_t s);

struct QBottleneckArgs {
  const int8_t *x, *w1, *w2, *w3;
  const int32_t *m1, *s1, *m2, *s2, *m3, *s3;
  int8_t *out;
  int N, H, W, C, M1;
};
bool qbottleneck_supported(int C, int M1);
hipError_t launch_qbottleneck_i8(const QBottleneckArgs &a, hipStream_t s);

struct IrbArgs {
  const float *x, *we, *wdw, *wp;
  float *out;
  int N, H, W, C, E;
};
bool irb_supported(int C, int E);
hipError_t launch_irb_f32(const IrbArgs &a, hipStream_t s);

// fill -> matmul -> generic(bias, act) as the reference's bufferized tile
// loop, every SRAM buffer at its planned LDS byte offset (k_planned.hip).
struct PlannedMatmulArgs {
  const float *A, *B, *bias;  // bias may be null
  float *out;
  int M, N, K, act;
  int tm, tn, tk, lds_bytes;
  int off_a[2], off_b[2], off_bias, off_c, off_y;  // off_bias -1: no bias
  void *lds_dump;             // may be null: else tile (0,0)'s LDS, lds_bytes
};
bool planned_matmul_tiles_ok(int tm, int tn, int tk);
hipError_t launch_planned_matmul(const PlannedMatmulArgs &a, hipStream_t s);

struct PlannedConvArgs {
  const float *x, *w, *bias;  // bias may be null
  float *out;
  int N, C, Hp, Wp, F, KH, KW, Ho, Wo, act;
  int tco, lds_bytes;
  // -1: spilled (in, w: read from HBM), no prefetch region, no bias
  int off_in[2], off_w[2], off_bias[2], off_in_pre, off_w_pre, off_bias_pre, off_c, off_y;
  void *lds_dump;             // may be null: else workgroup 0's LDS, lds_bytes
};
hipError_t launch_planned_conv(const PlannedConvArgs &a, hipStream_t s);

// Llama layer GEMM variants: A prologue and epilogue kinds.
enum { kProPlain = 0, kProRmsnorm = 1 };
enum { kEpiQkvRope = 0, kEpiResidual = 1, kEpiSwiglu = 2 };
struct LlamaGemmArgs {
  const uint16_t *A;      // [M][K] bf16
  const float *gamma;     // [K] (RMSNorm prologue)
  float eps;
  const uint16_t *B[3];   // each [K][Npart] bf16; QKV: 3 parts, SwiGLU: gate, up
  int nparts;
  int M, K, Npart, Dh;
  const float *cos_t, *sin_t;  // [M][Dh/2] (RoPE epilogue)
  const uint16_t *res;    // [M][Npart] (residual epilogue)
  uint16_t *out[3];       // each [M][Npart]
};
hipError_t launch_llama_gemm(const LlamaGemmArgs &a, int pro, int epi, hipStream_t s);
hipError_t launch_llama_attention(const uint16_t *Q, const uint16_t *K, const uint16_t *V,
                                  uint16_t *O, int S, int H, int dh, float scale, hipStream_t s);

}  // namespace npu
