// k_conv.hip -- group `pad -> fill -> conv_2d_nhwc_fhwc -> generic(bias, act)`.
//
// Implicit GEMM on MFMA: rows = output pixels (n, oh, ow), columns = filters
// f, reduction = (kh, kw, c).  NHWC activations and FHWC filters both keep
// the channel dimension contiguous, so every lane's MFMA operand is one
// 16-byte run of channels of one pixel (A) or one filter (B) -- no transpose
// and no im2col buffer.  tensor.pad (test/conv2d_relu.mlir:13-16) is not
// materialised: out-of-image taps load zeros (predicated halo loads).  The
// spatial split the reference picks over Co (test/lit/spatial_tiling_conv2d.mlir:28-34)
// becomes the grid's y dimension; the pixel dimension is the grid's x.
//
// Workgroup tile: 64 pixels x 64 filters, 4 waves as 2 x 2, each wave
// 32 x 32 = four 16x16 MFMA tiles.  The epilogue (bias add, residual add,
// act, and the bf16 rounding of the bf16 variant) runs on the accumulators.
// C need not be a multiple of an MFMA fragment's 16 (f32) or 32 (bf16)
// channels: a lane's 16-byte run past C loads zeros.  F need not be a
// multiple of 16 either: filters past F are zero and not stored.
#include "kernels.hpp"
#include "npu_device.hpp"
#include "plans.hpp"

namespace npu {

namespace {

template <class MM, typename T>
__global__ __launch_bounds__(256) void conv2d_nhwc_kernel(
    const T *__restrict__ x, const T *__restrict__ w, const float *__restrict__ bias,
    const T *__restrict__ res, T *__restrict__ out, int Nb, int H, int W, int C, int F, int KH,
    int KW, int pad, int Ho, int Wo, int act) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int P = Nb * Ho * Wo;
  const int p0 = blockIdx.x * 64 + (wave & 1) * 32;
  const int f0 = blockIdx.y * 64 + (wave >> 1) * 32;

  int pbase[2], poh[2], pow_[2];
  bool pok[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int p = p0 + 16 * i + r;
    pok[i] = p < P;
    const int pp = pok[i] ? p : 0;
    const int n = pp / (Ho * Wo);
    const int rem = pp - n * Ho * Wo;
    poh[i] = rem / Wo;
    pow_[i] = rem - poh[i] * Wo;
    pbase[i] = n * H * W;  // pixel index of (n, 0, 0) in the input
  }
  bool fok[2];
  int fbase[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int f = f0 + 16 * j + r;
    fok[j] = f < F;
    fbase[j] = (fok[j] ? f : 0) * KH * KW * C;
  }

  typename MM::acc_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = typename MM::acc_t{0, 0, 0, 0};

  const int cl = q * MM::kPerLane;
  for (int kh = 0; kh < KH; ++kh) {
    for (int kw = 0; kw < KW; ++kw) {
      int aoff[2];
      bool aok[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int ih = poh[i] + kh - pad, iw = pow_[i] + kw - pad;
        aok[i] = pok[i] && ih >= 0 && ih < H && iw >= 0 && iw < W;
        aoff[i] = (pbase[i] + ih * W + iw) * C + cl;
      }
      const int woff = (kh * KW + kw) * C + cl;
      for (int c0 = 0; c0 < C; c0 += MM::kPerFrag) {
        const bool cin = c0 + cl < C;  // this lane's run lies within the C channels
        Frag16 a[2], b[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) a[i] = aok[i] && cin ? load16(x + aoff[i] + c0) : frag_zero();
#pragma unroll
        for (int j = 0; j < 2; ++j) b[j] = fok[j] && cin ? load16(w + fbase[j] + woff + c0) : frag_zero();
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) MM::mma(acc[i][j], a[i], b[j]);
      }
    }
  }

  // Epilogue: rows 4q + e of each 16-pixel block, column r of each 16-filter block.
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int f = f0 + 16 * j + r;
    if (f >= F) continue;
    const float bv = bias ? bias[f] : 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int p = p0 + 16 * i + 4 * q + e;
        if (p >= P) continue;
        float v = acc[i][j][e] + bv;
        if constexpr (sizeof(T) == 4) {
          if (res) v += res[(size_t)p * F + f];
          out[(size_t)p * F + f] = act_apply(v, act);
        } else {
          if (res) v += bf16_to_f32(res[(size_t)p * F + f]);
          out[(size_t)p * F + f] = f32_to_bf16(act_apply(v, act));
        }
      }
    }
  }
}

template <class MM, typename T>
hipError_t launch_conv(const ConvArgs &a, hipStream_t s) {
  const int P = a.N * a.Ho * a.Wo;
  dim3 grid((P + 63) / 64, (a.F + 63) / 64);
  const int iters = a.KH * a.KW * ((a.C + MM::kPerFrag - 1) / MM::kPerFrag);
  npu_launch_plan p = make_plan("conv2d_nhwc", grid.x * grid.y, wg_per_cu(conv2d_nhwc_kernel<MM, T>),
                                grid.x * grid.y, 8 * sizeof(T));
  p.load_phases = iters;  // each (tap, channel chunk) step loads, then multiplies
  p.tile_macs = 64.0 * 64 * iters * MM::kPerFrag;
  p.tile_valu = 4.0 * (40.0 * iters + 150);  // per wave: addressing per step, epilogue
  p.tile_load_bytes = iters * 4.0 * 4 * 1024;  // per wave 2 A and 2 B fragments of 1 KB
  p.tile_store_bytes = 64.0 * 64 * sizeof(T);
  p.hbm_bytes = (double)sizeof(T) * ((double)a.N * a.H * a.W * a.C + (double)a.F * a.KH * a.KW * a.C +
                                     (double)P * a.F * (a.res ? 2 : 1)) + (a.bias ? 4.0 * a.F : 0.0);
  plans_add(p);
  hipLaunchKernelGGL((conv2d_nhwc_kernel<MM, T>), grid, dim3(256), 0, s,
                     static_cast<const T *>(a.x), static_cast<const T *>(a.w), a.bias,
                     static_cast<const T *>(a.res), static_cast<T *>(a.out), a.N, a.H, a.W, a.C,
                     a.F, a.KH, a.KW, a.pad, a.Ho, a.Wo, a.act);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_conv2d_nhwc_f32(const ConvArgs &a, hipStream_t s) {
  return launch_conv<MfmaF32, float>(a, s);
}
hipError_t launch_conv2d_nhwc_bf16(const ConvArgs &a, hipStream_t s) {
  return launch_conv<MfmaBF16, uint16_t>(a, s);
}

}  // namespace npu
