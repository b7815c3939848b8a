// k_matmul.hip -- group `fill -> matmul -> generic(bias, act)` in f32.
//
// Replaces the tile loops the reference wraps around the outlined call
// (FusionPass.cpp:306-359 tile-and-fuse of the consumer generic, then
// OutlineFusedGroupsPass.cpp:306-316): one launch covers the whole output.
//
// Decomposition.  The matmul+bias+ReLU shape (256x512 . 512x256) has only
// 256 output tiles of 16x16, one per CU, so each workgroup owns one 16x16
// tile and splits K across its 4 waves (split-K inside the workgroup; the
// reference's analogue is a K split with a reduce penalty,
// CostModel.cpp:798-812).  Each wave runs v_mfma_f32_16x16x4_f32 over its K
// share, the partial tiles meet in LDS, and the epilogue (bias add, act) is
// applied once while the tile is in registers: the matmul result never
// reaches HBM.
#include "kernels.hpp"
#include "npu_device.hpp"
#include "plans.hpp"

namespace npu {

namespace {

constexpr int kWaves = 4;
constexpr int kBatch = 8;  // K chunks whose loads are all issued before their MFMAs

__global__ __launch_bounds__(kWaves * 64) void matmul_bias_act_f32_kernel(
    const float *__restrict__ A, const float *__restrict__ B,
    const float *__restrict__ bias, float *__restrict__ out, int M, int N, int K,
    int act) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int m0 = blockIdx.y * 16, n0 = blockIdx.x * 16;
  // Rows past M and columns past N read row M-1 / column N-1: they only feed
  // outputs that are never stored.  Every load is issued unconditionally
  // from a valid address and masked afterwards (a load under a divergent
  // branch would make the compiler wait for all outstanding loads).
  const float *arow = A + (size_t)min(m0 + r, M - 1) * K;
  const int bcol = min(n0 + r, N - 1);

  // K is walked in chunks of 16 (four MFMA k-steps); waves take contiguous
  // chunk ranges.  K % 4 == 0, so a lane's 4-element run is all in or all out.
  const int nchunks = (K + 15) >> 4;
  const int c_begin = (wave * nchunks) / kWaves;
  const int c_end = ((wave + 1) * nchunks) / kWaves;

  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int c = c_begin; c < c_end; c += kBatch) {
    Frag16 a[kBatch], b[kBatch];
#pragma unroll
    for (int t = 0; t < kBatch; ++t) {
      const int k = (c + t) * 16 + 4 * q;
      const bool ok = c + t < c_end && k < K;
      const int kk = ok ? k : 0;
      a[t] = load16(arow + kk);
#pragma unroll
      for (int s = 0; s < 4; ++s) b[t].f[s] = B[(size_t)(kk + s) * N + bcol];
      a[t].u = masked(a[t].u, ok);
      b[t].u = masked(b[t].u, ok);
    }
#pragma unroll
    for (int t = 0; t < kBatch; ++t) MfmaF32::mma(acc, a[t], b[t]);
  }

  // Split-K reduction through LDS, then the fused epilogue.
  __shared__ float red[kWaves][256];
#pragma unroll
  for (int i = 0; i < 4; ++i) red[wave][(4 * q + i) * 16 + r] = acc[i];
  __syncthreads();
  const ActBounds ab = act_bounds(act);
  for (int e = threadIdx.x; e < 256; e += blockDim.x) {
    float s = red[0][e];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) s += red[w][e];
    const int row = m0 + (e >> 4), col = n0 + (e & 15);
    if (row < M && col < N) {
      if (bias) s += bias[col];
      out[(size_t)row * N + col] = act_clamp(s, ab);
    }
  }
}

}  // namespace

hipError_t launch_matmul_bias_act_f32(const MatmulArgs &a, hipStream_t s) {
  dim3 grid((a.N + 15) / 16, (a.M + 15) / 16);
  const int nchunks = (a.K + 15) / 16;
  npu_launch_plan p = make_plan("matmul_bias_act_f32", grid.x * grid.y,
                                wg_per_cu(matmul_bias_act_f32_kernel), grid.x * grid.y, 32);
  p.load_phases = ((nchunks + kWaves - 1) / kWaves + kBatch - 1) / kBatch;
  p.tile_macs = 16.0 * 16 * nchunks * 16;
  // Vector instructions per wave, from the compiled loops: 40 to set up and
  // write the split-K partials; 209 per batch of kBatch K chunks (a chunk's
  // five loads: 64-bit addresses, eight mask selects, the bounds tests; a
  // short last batch runs the whole unrolled body); 19 per epilogue pass.
  const int batches = ((nchunks + kWaves - 1) / kWaves + kBatch - 1) / kBatch;
  p.tile_valu = kWaves * (40.0 + 209.0 * batches + 19.0 * ((256 + kWaves * 64 - 1) / (kWaves * 64)));
  p.tile_lds_bytes = 2.0 * kWaves * 256 * 4;                   // partials written, read
  p.tile_load_bytes = 2.0 * 16 * nchunks * 16 * 4;             // 16 rows of A, 16 columns of B
  p.tile_store_bytes = 16.0 * 16 * 4;
  p.hbm_bytes = 4.0 * ((double)a.M * a.K + (double)a.K * a.N + (double)a.M * a.N + (a.bias ? a.N : 0));
  plans_add(p);
  hipLaunchKernelGGL(matmul_bias_act_f32_kernel, grid, dim3(kWaves * 64), 0, s, a.A,
                     a.B, a.bias, a.out, a.M, a.N, a.K, a.act);
  return hipGetLastError();
}

}  // namespace npu
