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
#include <type_traits>

#include "kernels.hpp"
#include "npu_device.hpp"
#include "persistent.hpp"
#include "plans.hpp"

namespace npu {

namespace {

constexpr int kWaves = 4;
constexpr int kBatch = 8;   // K chunks whose loads are all issued before their MFMAs
constexpr int kBRow = 20;   // LDS row stride of a staged B chunk, in floats (80 bytes)

// B operand staging.  The MFMA wants, per lane (column j, group q), the
// values B[k][j] of four consecutive k: a column walk, one 4-byte load per
// value.  Instead each wave loads its B rows whole -- lane l takes 16 bytes
// of row l/4 of a chunk (columns 4(l%4)..+3 of the tile), so one
// instruction moves a chunk's 16 rows x 64 bytes -- parks them in its own
// LDS slice and reads the column runs back (four 4-byte LDS reads per
// chunk).  The 80-byte row stride puts rows 4q + s of the four lane groups
// 16 banks apart: the reads are free of bank conflicts.  Each wave only
// reads what it wrote, so no barrier is needed (a wave's LDS operations
// complete in order).
//
// VEC: N % 4 == 0, so a 16-byte run is all inside a row or all past it; else
// four 4-byte loads with the column clamped.
template <bool VEC>
__global__ __launch_bounds__(kWaves * 64) void matmul_bias_act_f32_kernel(
    const float *__restrict__ A, const float *__restrict__ B,
    const float *__restrict__ bias, float *__restrict__ out, int M, int N, int K,
    int act, int tiles_n) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  // Tiles in XCD-contiguous ranges (consecutive workgroups go to the eight
  // XCDs in turn, each with its own L2): an XCD's tiles share rows of A.
  const int nb = gridDim.x, b = blockIdx.x;
  const int t = nb % kXcds == 0 ? (b % kXcds) * (nb / kXcds) + b / kXcds : b;
  const int m0 = (t / tiles_n) * 16, n0 = (t % tiles_n) * 16;
  // Rows past M and columns past N read row M-1 / the last columns: they
  // only feed outputs that are never stored.  Every load is issued
  // unconditionally from a valid address and masked afterwards (a load
  // under a divergent branch would make the compiler wait for all
  // outstanding loads).
  const float *arow = A + (size_t)min(m0 + r, M - 1) * K;
  const int br = lane >> 2, bq = lane & 3;
  const int bcol = n0 + 4 * bq;
  const int bcol_v = min(bcol, N - 4);  // VEC: N >= 4
  __shared__ __attribute__((aligned(16))) float bs[kWaves][kBatch * 16 * kBRow];
  float *const myb = bs[wave];

  // K is walked in chunks of 16 (four MFMA k-steps); waves take contiguous
  // chunk ranges.  K % 4 == 0, so a lane's 4-element run of A is all in or
  // all out; a B row is in when its k is.
  const int nchunks = (K + 15) >> 4;
  const int c_begin = (wave * nchunks) / kWaves;
  const int c_end = ((wave + 1) * nchunks) / kWaves;

  // this thread's epilogue element is (row e / 16, column e % 16) of the
  // tile, e = threadIdx.x: its bias is fetched now, not after the K loop
  const int ecol = n0 + (threadIdx.x & 15);
  const float bias_e = bias ? bias[min(ecol, N - 1)] : 0.0f;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  // One batch of kBatch chunks from chunk c: loads, B staged, MFMAs.  MASK:
  // the batch runs past the wave's range or past K (its last, partial
  // batch), so indices are clamped and values masked; full batches (a
  // uniform test) skip both.
  auto batch = [&](int c, auto mask) __attribute__((always_inline)) {
    constexpr bool MASK = decltype(mask)::value;
    Frag16 a[kBatch], bv[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int k = (c + u) * 16 + 4 * q, kb = (c + u) * 16 + br;
      const bool ok = !MASK || (c + u < c_end && k < K), okb = !MASK || (c + u < c_end && kb < K);
      a[u] = load16(arow + (ok ? k : 0));
      const float *brow = B + (size_t)(okb ? kb : 0) * N;
      if constexpr (VEC) {
        bv[u] = load16(brow + bcol_v);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) bv[u].f[e] = brow[min(bcol + e, N - 1)];
      }
      if constexpr (MASK) {
        a[u].u = masked(a[u].u, ok);
        bv[u].u = masked(bv[u].u, okb);
      }
    }
    // chunk by chunk, so each chunk's MFMAs wait only for its own loads
    // (issued in order) and run while the later chunks arrive
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      *reinterpret_cast<u32x4 *>(myb + (u * 16 + br) * kBRow + 4 * bq) = bv[u].u;
      // the reads below take values other lanes of this wave just wrote:
      // order them after the writes explicitly
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
      for (int s = 0; s < 4; ++s)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u].f[s], myb[(u * 16 + 4 * q + s) * kBRow + r], acc, 0, 0, 0);
    }
  };
  for (int c = c_begin; c < c_end; c += kBatch) {
    if (c + kBatch <= c_end && (c + kBatch) * 16 <= K)
      batch(c, std::false_type{});
    else
      batch(c, std::true_type{});
  }

  // Split-K reduction through LDS, then the fused epilogue.
  __shared__ float red[kWaves][256];
#pragma unroll
  for (int i = 0; i < 4; ++i) red[wave][(4 * q + i) * 16 + r] = acc[i];
  __syncthreads();
  const ActBounds ab = act_bounds(act);
  static_assert(kWaves * 64 == 256, "one epilogue element per thread");
  const int e = threadIdx.x;
  float sum = red[0][e];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) sum += red[w][e];
  const int row = m0 + (e >> 4);
  if (row < M && ecol < N) out[(size_t)row * N + ecol] = act_clamp(bias ? sum + bias_e : sum, ab);
}

}  // namespace

hipError_t launch_matmul_bias_act_f32(const MatmulArgs &a, hipStream_t s) {
  const int tiles_n = (a.N + 15) / 16, tiles = tiles_n * ((a.M + 15) / 16);
  const int nchunks = (a.K + 15) / 16;
  const bool vec = a.N % 4 == 0;
  auto kern = vec ? matmul_bias_act_f32_kernel<true> : matmul_bias_act_f32_kernel<false>;
  npu_launch_plan p = make_plan("matmul_bias_act_f32", tiles, wg_per_cu(kern), tiles, 32);
  const int batches = ((nchunks + kWaves - 1) / kWaves + kBatch - 1) / kBatch;
  p.load_phases = batches;
  p.tile_macs = 16.0 * 16 * nchunks * 16;
  // Vector instructions per wave, from the compiled loops: 60 to set up and
  // write the split-K partials; 62 per full batch of kBatch K chunks (the
  // B rows' 64-bit addresses, LDS offsets), 146 for a partial one (indices
  // clamped, values masked); 19 per epilogue pass.
  const int cpw = (nchunks + kWaves - 1) / kWaves;
  const bool partial = cpw % kBatch != 0 || nchunks % kWaves != 0 || a.K % 16 != 0;
  p.tile_valu = kWaves * (60.0 + 62.0 * batches + (partial ? 84.0 : 0.0) +
                          19.0 * ((256 + kWaves * 64 - 1) / (kWaves * 64)));
  p.tile_lds_bytes = 2.0 * 16 * nchunks * 16 * 4 +           // B chunks staged, read back
                     2.0 * kWaves * 256 * 4;                  // partials written, read
  p.tile_load_bytes = 2.0 * 16 * nchunks * 16 * 4;           // 16 rows of A, 16 columns of B
  p.tile_store_bytes = 16.0 * 16 * 4;
  p.hbm_bytes = 4.0 * ((double)a.M * a.K + (double)a.K * a.N + (double)a.M * a.N + (a.bias ? a.N : 0));
  plans_add(p);
  hipLaunchKernelGGL(kern, dim3(tiles), dim3(kWaves * 64), 0, s, a.A, a.B, a.bias, a.out, a.M, a.N,
                     a.K, a.act, tiles_n);
  return hipGetLastError();
}

}  // namespace npu
