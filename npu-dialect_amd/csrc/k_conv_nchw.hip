// k_conv_nchw.hip -- the reference's own conv group kind:
// `fill -> conv_2d_nchw_fchw -> generic...`, outlined as
// @fused_fill_conv2d_generic[_generic]_<idx> (test/conv2d_relu.mlir:7-42,
// test/resnet_block.mlir, test/resnet50_block.mlir, test/mobilenet_block.mlir;
// lib/Transforms/OutlineFusedGroupsPass.cpp:69-82).  NCHW activations, FCHW
// filters, any stride, the feeding tensor.pad folded into the halo loads and the
// layout kept on both sides: no transposed copy of either tensor in HBM.
//
// Implicit GEMM on the f32 MFMA: rows = output pixels of one row segment,
// columns = filters, reduction = (channel, tap).  Per chunk of 16 channels a
// workgroup stages, each in the order it is stored in HBM:
//   * the input halo: 16 channels x KH rows x (PX + KW - 1) columns (a
//     channel's row segment is contiguous in NCHW, so lanes load consecutive
//     words), zero outside the image (the pad) and past C;
//   * its 64 filters' chunk: 16 channels x KH*KW taps per filter, one
//     contiguous run in FCHW, each filter's record padded to an odd number of
//     words.
// MFMA step s of lane (r, q) takes channel 4q + s of the chunk at one tap:
// A = halo word (channel, tap row, pixel r + tap column), B = filter r's word
// (channel, tap).  Sixteen lanes read consecutive halo words or records of odd
// stride, so neither read has bank conflicts.  A chunk's loads are issued
// before the barrier that ends the previous chunk's multiply; several
// workgroups per CU overlap one's staging with another's MFMAs.
//
// Accumulator: lane (r, q) of pixel block i holds pixels 16 i + 4q .. +3 of
// the segment for filter r -- four consecutive NCHW outputs -- finished with
// the bias, the residual (same layout) and the activation.
#include "kernels.hpp"
#include "npu_device.hpp"
#include "persistent.hpp"
#include "plans.hpp"

namespace npu {

namespace {

constexpr int kNchwChunk = 16;  // channels per staged chunk

template <int KH, int KW, int ST, int NB>
__global__ __launch_bounds__(256) void conv2d_nchw_kernel(
    const float *__restrict__ x, const float *__restrict__ w, const float *__restrict__ bias,
    const float *__restrict__ res, float *__restrict__ out, int C, int H, int W, int F, int pad,
    int Ho, int Wo, int nseg, int act) {
  constexpr int CK = kNchwChunk;
  constexpr int PX = 16 * NB;                  // pixels of the row segment
  constexpr int HC = (PX - 1) * ST + KW;       // halo columns (stride ST)
  constexpr int HROWS = CK * KH;               // halo rows (channel, tap row)
  constexpr int HALO = HROWS * HC;             // halo words
  constexpr int TAPS = KH * KW;
  constexpr int WRUN = CK * TAPS;              // a filter's chunk (words)
  constexpr int WREC = WRUN + 1;               // its LDS record: an odd stride
  constexpr int NT = 256;
  constexpr int HPT = (HALO + NT - 1) / NT;    // halo words per thread
  constexpr int WPT = (64 * WRUN + NT - 1) / NT;  // filter words per thread
  __shared__ float halo[HALO];
  __shared__ float wl[64 * WREC];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int seg = blockIdx.x % nseg, orow = blockIdx.x / nseg;  // orow = n * Ho + oh
  const int n = orow / Ho, oh = orow - n * Ho;
  const int ow0 = seg * PX;
  const int f0 = blockIdx.y * 64;

  // Staging slots: halo word e = tid + NT j is (channel e / (KH HC), tap row,
  // column); filter word e is (filter e / WRUN, word e % WRUN of its chunk).
  // Addresses are recomputed per chunk (constant divisors; opaque() keeps
  // the compiler from hoisting them into registers held across the loop).  Loads come from clamped addresses and are masked when
  // written, so none waits under a condition.
  static_assert(HPT <= 64 && WPT <= 64, "slot masks fit 64 bits");
  float hv[HPT], wv[WPT];
  auto halo_slot = [&](int j, int c0, int &src) __attribute__((always_inline)) {
    const int t = opaque(tid) + NT * j;
    const int e = min(t, HALO - 1);
    const int hr = e / HC, col = e - hr * HC;
    const int c = hr / KH, kh = hr - c * KH;
    const int ih = oh * ST + kh - pad, iw = ow0 * ST + col - pad;
    src = ((n * C + min(c0 + c, C - 1)) * H + min(max(ih, 0), H - 1)) * W + min(max(iw, 0), W - 1);
    return t < HALO && c0 + c < C && ih >= 0 && ih < H && iw >= 0 && iw < W;
  };
  auto filter_slot = [&](int j, int c0, int &src) __attribute__((always_inline)) {
    const int t = opaque(tid) + NT * j;
    const int e = min(t, 64 * WRUN - 1);
    const int fl = e / WRUN, k = e - fl * WRUN, c = k / TAPS;
    src = (min(f0 + fl, F - 1) * C + min(c0 + c, C - 1)) * TAPS + (k - c * TAPS);
    return t < 64 * WRUN && f0 + fl < F && c0 + c < C;
  };
  auto fetch = [&](int c0) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < HPT; ++j) {
      int src;
      halo_slot(j, c0, src);
      hv[j] = x[src];
    }
#pragma unroll
    for (int j = 0; j < WPT; ++j) {
      int src;
      filter_slot(j, c0, src);
      wv[j] = w[src];
    }
  };
  auto commit = [&](int c0) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < HPT; ++j) {
      int src;
      const bool in = halo_slot(j, c0, src);
      const int e = tid + NT * j;
      if (e < HALO) halo[e] = in ? hv[j] : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < WPT; ++j) {
      int src;
      const bool in = filter_slot(j, c0, src);
      const int e = tid + NT * j;
      if (e < 64 * WRUN) {
        const int fl = e / WRUN;
        wl[fl * WREC + (e - fl * WRUN)] = in ? wv[j] : 0.0f;
      }
    }
  };

  f32x4 acc[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) acc[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const float *const wrow = wl + (wave * 16 + r) * WREC;

  for (int c0 = 0; c0 < C; c0 += CK) {
    fetch(c0);
    __syncthreads();  // the previous chunk's reads are done
    commit(c0);
    __syncthreads();
#pragma unroll 1
    for (int kh = 0; kh < KH; ++kh)
#pragma unroll
      for (int kw = 0; kw < KW; ++kw) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int c = 4 * q + s;
          const float b = wrow[c * TAPS + kh * KW + kw];
          const float *hrow = halo + (c * KH + kh) * HC + r * ST + kw;
#pragma unroll
          for (int i = 0; i < NB; ++i)
            acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(hrow[16 * ST * i], b, acc[i], 0, 0, 0);
        }
      }
  }

  const int f = f0 + wave * 16 + r;
  if (f >= F) return;
  const float bv = bias ? bias[f] : 0.0f;
  const ActBounds ab = act_bounds(act);
  const size_t obase = ((size_t)(n * F + f) * Ho + oh) * Wo;
#pragma unroll
  for (int i = 0; i < NB; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int ow = ow0 + 16 * i + 4 * q + e;
      if (ow < Wo) {
        float v = acc[i][e] + bv;
        if (res) v += res[obase + ow];
        out[obase + ow] = act_clamp(v, ab);
      }
    }
}

template <int KH, int KW, int ST, int NB>
hipError_t launch_nchw(const ConvArgs &a, hipStream_t s) {
  constexpr int PX = 16 * NB;
  const int nseg = (a.Wo + PX - 1) / PX;
  dim3 grid(a.N * a.Ho * nseg, (a.F + 63) / 64);
  const int chunks = (a.C + kNchwChunk - 1) / kNchwChunk;
  npu_launch_plan p = make_plan("conv2d_nchw", grid.x * grid.y,
                                wg_per_cu(conv2d_nchw_kernel<KH, KW, ST, NB>), grid.x * grid.y, 32);
  p.load_phases = chunks;  // each chunk's staging waits for its loads
  p.tile_macs = 64.0 * PX * a.C * KH * KW;
  // per wave: staging address selects and LDS writes per chunk, the tap loop's
  // LDS reads, the epilogue
  p.tile_valu = 4.0 * (chunks * (3.0 * ((KH * ((PX - 1) * ST + KW) * kNchwChunk + 255) / 256 +
                                         (64 * kNchwChunk * KH * KW + 255) / 256)) + 60.0);
  p.tile_lds_bytes = chunks * 4.0 * (KH * ((PX - 1) * ST + KW) * kNchwChunk + 64.0 * kNchwChunk * KH * KW) +
                     chunks * 4.0 * 64 * KH * KW * 4 * (NB + 1) * 4;
  p.tile_load_bytes = chunks * 4.0 * (KH * ((PX - 1) * ST + KW) * kNchwChunk + 64.0 * kNchwChunk * KH * KW);
  p.tile_store_bytes = 4.0 * PX * 64 * (a.res ? 2 : 1);
  p.hbm_bytes = 4.0 * ((double)a.N * a.C * a.H * a.W + (double)a.F * a.C * KH * KW +
                       (double)a.N * a.F * a.Ho * a.Wo * (a.res ? 2 : 1)) + (a.bias ? 4.0 * a.F : 0.0);
  plans_add(p);
  hipLaunchKernelGGL((conv2d_nchw_kernel<KH, KW, ST, NB>), grid, dim3(256), 0, s,
                     static_cast<const float *>(a.x), static_cast<const float *>(a.w), a.bias,
                     static_cast<const float *>(a.res), static_cast<float *>(a.out), a.C, a.H, a.W,
                     a.F, a.pad, a.Ho, a.Wo, nseg, a.act);
  return hipGetLastError();
}

// Row segments of 64 pixels, or of 32 when 64-pixel segments would leave
// fewer than two workgroups per CU.
template <int KH, int KW, int ST>
hipError_t launch_nchw_k(const ConvArgs &a, hipStream_t s) {
  const long long big = (long long)a.N * a.Ho * ((a.Wo + 63) / 64) * ((a.F + 63) / 64);
  return big >= 512 ? launch_nchw<KH, KW, ST, 4>(a, s) : launch_nchw<KH, KW, ST, 2>(a, s);
}

// Any filter size and stride (the model zoo's 7x7 stems, 5x5 and 9x9
// filters, its classifier written as a conv over the last feature map):
// implicit GEMM with the reduction index k = (c, kh, kw) in FCHW order, so a
// filter's operand is its own contiguous run of k, and each MFMA step's A
// word is the input pixel that k and the output pixel address (zero in the
// pad).  Operands come straight from L2: no staging, no halo reuse.
// Workgroup tile: 64 output pixels (flattened n, oh, ow) x 64 filters, waves
// as 2 x 2, each 32 x 32 = four 16x16 MFMA tiles; accumulator rows are
// pixels, so a lane's four values are consecutive pixels of one filter.
__global__ __launch_bounds__(256) void conv2d_nchw_direct_kernel(
    const float *__restrict__ x, const float *__restrict__ w, const float *__restrict__ bias,
    const float *__restrict__ res, float *__restrict__ out, int N, int C, int H, int W, int F,
    int KH, int KW, int st, int pad, int Ho, int Wo, int act) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int P = N * Ho * Wo, K = C * KH * KW, T = KH * KW;
  const int p0 = blockIdx.x * 64 + (wave & 1) * 32;
  const int f0 = blockIdx.y * 64 + (wave >> 1) * 32;
  int pn[2], ph[2], pw[2];
  bool pok[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int p = p0 + 16 * i + r;
    pok[i] = p < P;
    const int pp = pok[i] ? p : 0;
    pn[i] = pp / (Ho * Wo);
    const int rem = pp - pn[i] * Ho * Wo;
    ph[i] = (rem / Wo) * st - pad;
    pw[i] = (rem - (rem / Wo) * Wo) * st - pad;
  }
  const float *wr[2];
  bool fok[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int f = f0 + 16 * j + r;
    fok[j] = f < F;
    wr[j] = w + (size_t)(fok[j] ? f : 0) * K;
  }
  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  // lane group q takes k = k0 + 4q + s; (c, kh, kw) of each k is kept and
  // advanced by 16 per step instead of divided out
  int kc[4], kh_[4], kw_[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int k = 4 * q + s;
    kc[s] = k / T;
    kh_[s] = (k - kc[s] * T) / KW;
    kw_[s] = k - kc[s] * T - kh_[s] * KW;
  }
  for (int k0 = 0; k0 < K; k0 += 16) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int k = k0 + 4 * q + s;
      const bool kin = k < K;
      float a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int ih = ph[i] + kh_[s], iw = pw[i] + kw_[s];
        const bool in = kin && pok[i] && ih >= 0 && ih < H && iw >= 0 && iw < W;
        a[i] = in ? x[((size_t)(pn[i] * C + kc[s]) * H + ih) * W + iw] : 0.0f;
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = kin && fok[j] ? wr[j][k] : 0.0f;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
      // advance this slot's k by 16
      kw_[s] += 16;
      while (kw_[s] >= KW) {
        kw_[s] -= KW;
        if (++kh_[s] == KH) {
          kh_[s] = 0;
          ++kc[s];
        }
      }
    }
  }
  const ActBounds ab = act_bounds(act);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int f = f0 + 16 * j + r;
    if (f >= F) continue;
    const float bv = bias ? bias[f] : 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int p = p0 + 16 * i + 4 * q + e;
        if (p >= P) continue;
        const int n = p / (Ho * Wo), hw = p - n * Ho * Wo;
        const size_t o = (size_t)(n * F + f) * Ho * Wo + hw;
        float v = acc[i][j][e] + bv;
        if (res) v += res[o];
        out[o] = act_clamp(v, ab);
      }
  }
}

hipError_t launch_nchw_direct(const ConvArgs &a, hipStream_t s) {
  const int P = a.N * a.Ho * a.Wo;
  dim3 grid((P + 63) / 64, (a.F + 63) / 64);
  const double K = (double)a.C * a.KH * a.KW, steps = (K + 15) / 16;
  npu_launch_plan p = make_plan("conv2d_nchw_direct", grid.x * grid.y,
                                wg_per_cu(conv2d_nchw_direct_kernel), grid.x * grid.y, 32);
  p.load_phases = (int)steps;  // each k step loads, then multiplies
  p.tile_macs = 64.0 * 64 * K;
  p.tile_valu = 4.0 * (steps * 4 * 24.0 + 80.0);  // per wave: per k slot addresses, bounds, k advance
  p.tile_load_bytes = steps * 4 * 4.0 * 256 * 4;  // four words per lane and k slot, four waves
  p.tile_store_bytes = 4.0 * 64 * 64 * (a.res ? 2 : 1);
  p.hbm_bytes = 4.0 * ((double)a.N * a.C * a.H * a.W + (double)a.F * K +
                       (double)P * a.F * (a.res ? 2 : 1)) + (a.bias ? 4.0 * a.F : 0.0);
  plans_add(p);
  hipLaunchKernelGGL(conv2d_nchw_direct_kernel, grid, dim3(256), 0, s,
                     static_cast<const float *>(a.x), static_cast<const float *>(a.w), a.bias,
                     static_cast<const float *>(a.res), static_cast<float *>(a.out), a.N, a.C, a.H,
                     a.W, a.F, a.KH, a.KW, a.stride, a.pad, a.Ho, a.Wo, a.act);
  return hipGetLastError();
}

}  // namespace

// 1x1 and 3x3 filters at stride 1 or 2 take the staged kernel, every other
// shape the direct one.
hipError_t launch_conv2d_nchw_f32(const ConvArgs &a, hipStream_t s) {
  if (a.stride == 1) {
    if (a.KH == 1 && a.KW == 1) return launch_nchw_k<1, 1, 1>(a, s);
    if (a.KH == 3 && a.KW == 3) return launch_nchw_k<3, 3, 1>(a, s);
  } else if (a.stride == 2) {
    if (a.KH == 1 && a.KW == 1) return launch_nchw_k<1, 1, 2>(a, s);
    if (a.KH == 3 && a.KW == 3) return launch_nchw_k<3, 3, 2>(a, s);
  }
  return launch_nchw_direct(a, s);
}

}  // namespace npu
