// k_planned.hip -- the group `fill -> matmul -> generic(bias add, act)`
// run as the tile loop the reference's passes produce, with the LDS layout
// taken from the reference's SRAM plan instead of chosen by the kernel.
//
// After npu-temporal-tiling and npu-bufferize, one core of the reference
// runs, per output tile (tm x tn) and per K step (tk):
//   dma_copy A[m0:+tm, k0:+tk] -> SRAM, dma_copy B[k0:+tk, n0:+tn] -> SRAM,
//   matmul into the SRAM accumulator tile,
// then the generic over the accumulator and the bias tile into the output
// tile and one dma_copy of it back (BufferizePass.cpp:97-222); the SRAM
// buffers are placed by NPUSRAMAllocationPass's dual-end plan, the inputs
// of the tile loop in ping/pong pairs (SRAMAllocationPass.cpp:172-342),
// and npu-barrier-alloc cuts the loop into DMA-in -> compute -> DMA-out
// subgraphs (DMASchedulingPass.cpp:92-147).
//
// Here a workgroup is that core for one output tile.  Every buffer lives at
// the plan's byte offset in the workgroup's LDS, in the slice's own layout
// (row-major [tm][tk], [tk][tn], [tm][tn], [tn] f32, unpadded):
//   A, B        ping at `off`, pong at `off_pong`; K step i uses ping when
//               i is even, pong when odd (generation parity);
//   bias        its ping slot (its slice is the same for every K step),
//               when the group has one;
//   C           the accumulator tile (the fill's / matmul's output buffer);
//   Y           the generic's output tile, copied back to HBM.
// A DMA into SRAM is a global load per element and an LDS store at the
// plan's offset; the copy back reads Y from LDS.  Tiles of any size run
// (16x16 MFMA blocks, rows, columns and k past the tile multiply zeros).
// Each K step is one subgraph and has one s_barrier: the step's slices are
// in SRAM before any wave multiplies them, and the buffers the next step's
// DMA overwrites were last read by the step before, behind that barrier.
//
// This is the plan-parity path (the layout and schedule are the reference's,
// not tuned for the MI355X); fused_matmul_bias_act is the fast kernel for
// the same group.
#include "kernels.hpp"
#include "npu_device.hpp"
#include "plans.hpp"

namespace npu {

namespace {

constexpr int kPT = 256;        // threads: four waves
constexpr int kMaxBlocks = 16;  // 16x16 output blocks per wave

__global__ __launch_bounds__(kPT) void planned_matmul_kernel(const PlannedMatmulArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char sram[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int tm = a.tm, tn = a.tn, tk = a.tk, M = a.M, N = a.N, K = a.K;
  const int m0 = blockIdx.y * tm, n0 = blockIdx.x * tn;
  const int nk = (K + tk - 1) / tk;
  float *const sA[2] = {reinterpret_cast<float *>(sram + a.off_a[0]), reinterpret_cast<float *>(sram + a.off_a[1])};
  float *const sB[2] = {reinterpret_cast<float *>(sram + a.off_b[0]), reinterpret_cast<float *>(sram + a.off_b[1])};
  float *const sBias = reinterpret_cast<float *>(sram + (a.off_bias >= 0 ? a.off_bias : 0));
  float *const sC = reinterpret_cast<float *>(sram + a.off_c);
  float *const sY = reinterpret_cast<float *>(sram + a.off_y);

  // DMA of K step `kt` into SRAM buffer `buf`: element by element, slices
  // in their row-major layouts; k past K is zero, rows and columns past the
  // operand are clamped (they only reach outputs that are never stored)
  auto dma_in = [&](int kt, int buf) {
    const int k0 = kt * tk;
    for (int e = tid; e < tm * tk; e += kPT) {
      const int r = e / tk, c = e - r * tk;
      const float v = a.A[(size_t)min(m0 + r, M - 1) * K + min(k0 + c, K - 1)];
      sA[buf][e] = k0 + c < K ? v : 0.0f;
    }
    for (int e = tid; e < tk * tn; e += kPT) {
      const int r = e / tn, c = e - r * tn;
      const float v = a.B[(size_t)min(k0 + r, K - 1) * N + min(n0 + c, N - 1)];
      sB[buf][e] = k0 + r < K ? v : 0.0f;
    }
  };

  // the bias slice, once (the same for every K step of this tile); a group
  // without a bias has no such buffer
  const bool has_bias = a.off_bias >= 0;
  if (has_bias)
    for (int c = tid; c < tn; c += kPT) sBias[c] = a.bias[min(n0 + c, N - 1)];

  // wave w owns 16x16 output blocks w, w + 4, ... of the tile (row-major
  // over ceil(tm/16) x ceil(tn/16) blocks; rows and columns past the tile
  // multiply zeros)
  const int nbn = (tn + 15) / 16, nblocks = (tm + 15) / 16 * nbn;
  f32x4 acc[kMaxBlocks];
#pragma unroll
  for (int b = 0; b < kMaxBlocks; ++b) acc[b] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int r = lane & 15, kq = lane >> 4;

  dma_in(0, 0);
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    // subgraph kt: its DMA-in is in SRAM, and every wave is done with step
    // kt - 1, whose buffers step kt + 1's DMA overwrites
    __syncthreads();
    if (kt + 1 < nk) dma_in(kt + 1, buf ^ 1);
    const float *A_ = sA[buf], *B_ = sB[buf];
    for (int k = 0; k < tk; k += 4) {
      const bool kin = k + kq < tk;
#pragma unroll
      for (int b = 0; b < kMaxBlocks; ++b) {
        const int blk = wave + 4 * b;
        if (blk >= nblocks) break;
        const int bm = (blk / nbn) * 16 + r, bn = (blk % nbn) * 16 + r;
        const float av = kin && bm < tm ? A_[bm * tk + k + kq] : 0.0f;
        const float bv = kin && bn < tn ? B_[(k + kq) * tn + bn] : 0.0f;
        acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc[b], 0, 0, 0);
      }
    }
  }
  // the accumulator tile into its SRAM buffer (lane: rows 4 kq + e, column r)
#pragma unroll
  for (int b = 0; b < kMaxBlocks; ++b) {
    const int blk = wave + 4 * b;
    if (blk >= nblocks) break;
    const int bm = (blk / nbn) * 16, bn = (blk % nbn) * 16 + r;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (bm + 4 * kq + e < tm && bn < tn) sC[(bm + 4 * kq + e) * tn + bn] = acc[b][e];
  }
  __syncthreads();
  // the generic: Y = act(C + bias) in SRAM
  const ActBounds ab = act_bounds(a.act);
  for (int i = tid; i < tm * tn; i += kPT)
    sY[i] = act_clamp(has_bias ? sC[i] + sBias[i % tn] : sC[i], ab);
  __syncthreads();
  // DMA out: Y's rows and columns inside the output
  for (int i = tid; i < tm * tn; i += kPT) {
    const int row = i / tn, col = i - row * tn;
    if (m0 + row < M && n0 + col < N) a.out[(size_t)(m0 + row) * N + n0 + col] = sY[i];
  }
  // the layout itself, for a caller that asks: tile (0, 0)'s whole SRAM
  if (a.lds_dump && blockIdx.x == 0 && blockIdx.y == 0) {
    __syncthreads();
    for (int i = tid; i < a.lds_bytes / 4; i += kPT)
      reinterpret_cast<uint32_t *>(a.lds_dump)[i] = reinterpret_cast<const uint32_t *>(sram)[i];
  }
}

// The conv group's tile loop (see npu_planned_conv2d_nchw_bias_act): one
// workgroup per output row (n, ho), the loop over output-channel tiles of
// tco, every buffer at the plan's offset in its slice's own row-major f32
// layout.  Step i: [barrier] the tile's MACs from its input-rows and filter
// slots into C, [barrier] the generic C + bias -> Y, [barrier] Y back to
// HBM and the DMA-in of tile i+1 into the other slots (from the prefetch
// region, SRAM to SRAM, for a buffer that has one), [barrier] tile i+2's
// copies from HBM into the prefetch regions.
__global__ __launch_bounds__(kPT) void planned_conv_kernel(const PlannedConvArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char sram[];
  const int tid = threadIdx.x;
  const int C = a.C, KH = a.KH, KW = a.KW, Wp = a.Wp, Hp = a.Hp, Wo = a.Wo, F = a.F;
  const int tco = a.tco, CKK = C * KH * KW;
  const int n = blockIdx.x / a.Ho, ho = blockIdx.x - n * a.Ho;
  const int nt = (F + tco - 1) / tco;
  auto at = [&](int off) { return reinterpret_cast<float *>(sram + (off >= 0 ? off : 0)); };
  const bool in_lds = a.off_in[0] >= 0, w_lds = a.off_w[0] >= 0;
  const bool in_pre = a.off_in_pre >= 0, w_pre = a.off_w_pre >= 0, has_bias = a.off_bias[0] >= 0;
  const bool b_pre = has_bias && a.off_bias_pre >= 0;
  float *const sIn[2] = {at(a.off_in[0]), at(a.off_in[1] >= 0 ? a.off_in[1] : a.off_in[0])};
  float *const sW[2] = {at(a.off_w[0]), at(a.off_w[1] >= 0 ? a.off_w[1] : a.off_w[0])};
  float *const sB[2] = {at(a.off_bias[0]), at(a.off_bias[1] >= 0 ? a.off_bias[1] : a.off_bias[0])};
  float *const sInPre = at(a.off_in_pre), *const sWPre = at(a.off_w_pre);
  float *const sBPre = at(a.off_bias_pre), *const sC = at(a.off_c), *const sY = at(a.off_y);
  // the input rows ho .. ho+KH-1 of image n where they lie in HBM
  const float *const xrow = a.x + (size_t)n * C * Hp * Wp + (size_t)ho * Wp;

  // DMA of the input rows (all channels) into `dst`, as [C][KH][Wp]
  auto dma_in = [&](float *dst) {
    for (int e = tid; e < C * KH * Wp; e += kPT) {
      const int c = e / (KH * Wp), rc = e - c * KH * Wp;
      dst[e] = xrow[(size_t)c * Hp * Wp + rc];
    }
  };
  // DMA of tile i's filter slice; filters past F are zero
  auto dma_w = [&](int i, float *dst) {
    for (int e = tid; e < tco * CKK; e += kPT) {
      const int f = i * tco + e / CKK;
      dst[e] = f < F ? a.w[(size_t)f * CKK + e % CKK] : 0.0f;
    }
  };
  auto copy = [&](const float *src, float *dst, int count) {
    for (int e = tid; e < count; e += kPT) dst[e] = src[e];
  };
  // DMA of tile i's bias slice; channels past F are zero
  auto dma_bias = [&](int i, float *dst) {
    for (int co = tid; co < tco; co += kPT) dst[co] = i * tco + co < F ? a.bias[i * tco + co] : 0.0f;
  };

  if (in_lds) dma_in(sIn[0]);
  if (w_lds) dma_w(0, sW[0]);
  if (has_bias) dma_bias(0, sB[0]);
  if (in_pre && nt > 1) dma_in(sInPre);
  if (w_pre && nt > 1) dma_w(1, sWPre);
  if (b_pre && nt > 1) dma_bias(1, sBPre);
  const ActBounds ab = act_bounds(a.act);
  for (int i = 0; i < nt; ++i) {
    // operands of tile i: its LDS slots, or HBM for a spilled buffer
    const float *in = in_lds ? sIn[i & 1] : xrow;
    const int cstride = in_lds ? KH * Wp : Hp * Wp;
    const float *wt = w_lds ? sW[i & 1] : a.w + (size_t)i * tco * CKK;
    const float *bs = sB[i & 1];
    __syncthreads();
    for (int o = tid; o < tco * Wo; o += kPT) {
      const int co = o / Wo, wo = o - co * Wo;
      float acc = 0.0f;
      if (i * tco + co < F)
        for (int c = 0; c < C; ++c)
          for (int kh = 0; kh < KH; ++kh)
            for (int kw = 0; kw < KW; ++kw)
              acc += in[c * cstride + kh * Wp + wo + kw] * wt[co * CKK + (c * KH + kh) * KW + kw];
      sC[o] = acc;
    }
    __syncthreads();
    for (int o = tid; o < tco * Wo; o += kPT)
      sY[o] = act_clamp(has_bias ? sC[o] + bs[o / Wo] : sC[o], ab);
    __syncthreads();
    for (int o = tid; o < tco * Wo; o += kPT) {
      const int co = o / Wo, wo = o - co * Wo, f = i * tco + co;
      if (f < F) a.out[((size_t)(n * F + f) * a.Ho + ho) * Wo + wo] = sY[o];
    }
    if (i + 1 < nt) {
      const int nb = (i + 1) & 1;
      if (in_lds) {
        if (in_pre)
          copy(sInPre, sIn[nb], C * KH * Wp);
        else
          dma_in(sIn[nb]);
      }
      if (w_lds) {
        if (w_pre)
          copy(sWPre, sW[nb], tco * CKK);
        else
          dma_w(i + 1, sW[nb]);
      }
      if (has_bias) {
        if (b_pre)
          copy(sBPre, sB[nb], tco);
        else
          dma_bias(i + 1, sB[nb]);
      }
    }
    __syncthreads();
    if (i + 2 < nt) {
      if (in_pre) dma_in(sInPre);
      if (w_pre) dma_w(i + 2, sWPre);
      if (b_pre) dma_bias(i + 2, sBPre);
    }
  }
  if (a.lds_dump && blockIdx.x == 0) {
    __syncthreads();
    for (int e = tid; e < a.lds_bytes / 4; e += kPT)
      reinterpret_cast<uint32_t *>(a.lds_dump)[e] = reinterpret_cast<const uint32_t *>(sram)[e];
  }
}

}  // namespace

bool planned_matmul_tiles_ok(int tm, int tn, int tk) {
  return tm >= 1 && tn >= 1 && tk >= 1 && (tm + 15) / 16 * ((tn + 15) / 16) <= 4 * kMaxBlocks;
}

hipError_t launch_planned_matmul(const PlannedMatmulArgs &a, hipStream_t s) {
  if (!planned_matmul_tiles_ok(a.tm, a.tn, a.tk) || a.lds_bytes <= 0 || a.lds_bytes > 160 * 1024 || a.lds_bytes % 4 != 0)
    return hipErrorInvalidValue;
  const void *kern = reinterpret_cast<const void *>(planned_matmul_kernel);
  const int ok = cached_per_kernel(kern, [&](int) {
    return hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) ==
                   hipSuccess
               ? 1 : 0;
  });
  if (!ok) return hipErrorInvalidValue;
  const dim3 grid((a.N + a.tn - 1) / a.tn, (a.M + a.tm - 1) / a.tm);
  {
    // per tile: the K loop's DMA and MFMAs, then the generic and the copy back
    const double nk = (a.K + a.tk - 1) / a.tk, tiles = (double)grid.x * grid.y;
    npu_launch_plan p = make_plan("planned_matmul_bias_act", (int)tiles, wg_per_cu(planned_matmul_kernel),
                                  (int)tiles, 32);
    p.load_phases = 1 + 1;  // the first DMA-in, and the copy back's wait
    p.tile_macs = (double)a.tm * a.tn * nk * a.tk;
    const double pieces = (a.tm * a.tk + a.tk * a.tn) / 4.0;
    // per K step and wave: 3 per piece staged and stored, 4 per MFMA (two LDS
    // addresses, two reads); the generic 4 per element; the copy back 6 per piece
    p.tile_valu = nk * (3.0 * pieces / 64.0 * 4 + 4.0 * (a.tm / 16) * (a.tn / 16) * a.tk / 4) +
                  (4.0 * a.tm * a.tn + 6.0 * a.tm * a.tn / 4) / 64.0;
    p.tile_lds_bytes = nk * (2.0 * pieces * 16 + (double)(a.tm / 16) * (a.tn / 16) * (a.tk / 4) * 512) +
                       4.0 * a.tm * a.tn * 4;
    p.tile_load_bytes = nk * pieces * 16;
    p.tile_store_bytes = (double)a.tm * a.tn * 4;
    p.hbm_bytes = 4.0 * ((double)a.M * a.K + (double)a.K * a.N + (double)a.M * a.N + a.N);
    plans_add(p);
  }
  hipLaunchKernelGGL(planned_matmul_kernel, grid, dim3(kPT), a.lds_bytes, s, a);
  return hipGetLastError();
}

hipError_t launch_planned_conv(const PlannedConvArgs &a, hipStream_t s) {
  if (a.tco < 1 || a.lds_bytes <= 0 || a.lds_bytes > 160 * 1024 || a.lds_bytes % 4 != 0)
    return hipErrorInvalidValue;
  const void *kern = reinterpret_cast<const void *>(planned_conv_kernel);
  const int ok = cached_per_kernel(kern, [&](int) {
    return hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) ==
                   hipSuccess
               ? 1 : 0;
  });
  if (!ok) return hipErrorInvalidValue;
  const int grid = a.N * a.Ho;
  {
    // per workgroup (one output row): every tile's scalar MACs, the generic
    // and the copy back; the DMA of the input rows and filter slices
    const double nt = (a.F + a.tco - 1) / a.tco, macs = (double)a.tco * a.Wo * a.C * a.KH * a.KW;
    npu_launch_plan p = make_plan("planned_conv2d_nchw_bias_act", grid, wg_per_cu(planned_conv_kernel),
                                  grid, 32);
    p.load_phases = 1 + 1;
    p.tile_macs = 0.0;  // scalar FMAs, priced as vector work below
    p.tile_valu = nt * (2.0 * macs / 64.0 + 8.0 * a.tco * a.Wo / 64.0 +
                        3.0 * ((double)a.C * a.KH * a.Wp + a.tco * a.C * a.KH * a.KW) / 64.0);
    p.tile_lds_bytes = nt * (8.0 * macs + 16.0 * a.tco * a.Wo +
                             4.0 * ((double)a.C * a.KH * a.Wp + 2.0 * a.tco * a.C * a.KH * a.KW));
    p.tile_load_bytes = nt * 4.0 * ((double)a.C * a.KH * a.Wp + a.tco * a.C * a.KH * a.KW);
    p.tile_store_bytes = 4.0 * a.F * a.Wo;
    p.hbm_bytes = 4.0 * ((double)a.N * a.C * a.Hp * a.Wp + (double)a.F * a.C * a.KH * a.KW +
                         (double)a.N * a.F * a.Ho * a.Wo + a.F);
    plans_add(p);
  }
  hipLaunchKernelGGL(planned_conv_kernel, dim3(grid), dim3(kPT), a.lds_bytes, s, a);
  return hipGetLastError();
}

}  // namespace npu
