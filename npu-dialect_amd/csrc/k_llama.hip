// k_llama.hip -- the fused groups of one Llama decoder layer, bf16 storage,
// f32 accumulation (the Llama block the reference approximates in
// test/llama_attention.mlir:5-67, with the softmax, RMSNorm, RoPE and SwiGLU
// that it replaces by ReLU or omits, :39-52):
//
//   qkv   : xn = bf16(rmsnorm(x)*g1); Q,K = bf16(rope(xn@Wq|Wk)); V = bf16(xn@Wv)
//   attn  : A = bf16(softmax_causal(Q K^T / sqrt(Dh)) V) per head
//   oproj : h = bf16(x + A@Wo)
//   swiglu: hn = bf16(rmsnorm(h)*g2); act = bf16(silu(hn@Wg) * (hn@Wu))
//   down  : out = bf16(h + act@Wd)
//
// The four matmul groups share one bf16 MFMA GEMM (v_mfma_f32_16x16x32_bf16)
// with a 64x64 workgroup tile and K chunks of 32 staged through LDS.  The
// weights are row-major [K][N] as linalg.matmul takes them, so each B chunk
// is transposed on its way into LDS to give every lane a 16-byte k run.  The
// RMSNorm is fused as a prologue (row inverse-RMS first, then the normalised
// bf16 A chunk is produced while staging), RoPE / residual / SiLU-gating as
// epilogues on the accumulators; nothing between the ops touches HBM.
//
// Attention is a causal flash kernel: one wave per 16 query rows of one head,
// online softmax in f32, P rounded to bf16 for its MFMA with V.
#include "kernels.hpp"
#include "npu_device.hpp"

namespace npu {

namespace {

constexpr int TM = 64, TN = 64, TK = 32;
constexpr int LDK = TK + 8;  // LDS row stride (elements) of the [row][k] staging tiles

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

template <int PRO, int EPI>
__global__ __launch_bounds__(256) void llama_gemm_kernel(const LlamaGemmArgs a) {
  constexpr int NB = (EPI == kEpiSwiglu) ? 2 : 1;
  __shared__ __attribute__((aligned(16))) uint16_t As[TM * LDK];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[NB][TN * LDK];
  __shared__ float inv_rms[TM];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int m0 = blockIdx.y * TM;
  const int tiles_per_part = a.Npart / TN;
  const int part = (EPI == kEpiQkvRope) ? blockIdx.x / tiles_per_part : 0;
  const int n0 = (blockIdx.x % tiles_per_part) * TN;
  const uint16_t *B0 = a.B[part];
  const uint16_t *B1 = a.B[NB - 1];

  if (PRO == kProRmsnorm) {
    // inverse RMS of the tile's rows: wave w reduces rows 16w .. 16w+15
    for (int rr = 0; rr < 16; ++rr) {
      const int row = m0 + wave * 16 + rr;
      float s = 0.0f;
      if (row < a.M) {
        for (int k = lane * 8; k < a.K; k += 512) {
          const Frag16 v = load16(a.A + (size_t)row * a.K + k);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float lo = __uint_as_float(v.u[j] << 16), hi = __uint_as_float(v.u[j] & 0xffff0000u);
            s += lo * lo;
            s += hi * hi;
          }
        }
      }
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
      if (lane == 0) inv_rms[wave * 16 + rr] = 1.0f / sqrtf(s / (float)a.K + a.eps);
    }
    __syncthreads();
  }

  f32x4 acc[NB][2][2];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[b][i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int wm = (wave & 1) * 32, wn = (wave >> 1) * 32;
  const int arow = tid >> 2, akk = (tid & 3) * 8;  // A staging: 64 rows x 4 runs of 8
  const int bk = tid >> 3, bnn = (tid & 7) * 8;    // B staging: 32 k-rows x 8 runs of 8
  for (int k0 = 0; k0 < a.K; k0 += TK) {
    {
      Frag16 v = frag_zero();
      const int row = m0 + arow;
      if (row < a.M) v = load16(a.A + (size_t)row * a.K + k0 + akk);
      if (PRO == kProRmsnorm) {
        const float inv = inv_rms[arow];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float lo = __uint_as_float(v.u[j] << 16), hi = __uint_as_float(v.u[j] & 0xffff0000u);
          const float ylo = (lo * inv) * a.gamma[k0 + akk + 2 * j];
          const float yhi = (hi * inv) * a.gamma[k0 + akk + 2 * j + 1];
          v.u[j] = (uint32_t)f32_to_bf16(ylo) | ((uint32_t)f32_to_bf16(yhi) << 16);
        }
      }
      *reinterpret_cast<u32x4 *>(As + arow * LDK + akk) = v.u;
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const uint16_t *Bp = b == 0 ? B0 : B1;
      const Frag16 v = load16(Bp + (size_t)(k0 + bk) * a.Npart + n0 + bnn);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        Bs[b][(bnn + 2 * j) * LDK + bk] = (uint16_t)(v.u[j] & 0xffffu);
        Bs[b][(bnn + 2 * j + 1) * LDK + bk] = (uint16_t)(v.u[j] >> 16);
      }
    }
    __syncthreads();
    Frag16 af[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) af[i] = load16(As + (wm + 16 * i + r) * LDK + 8 * q);
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const Frag16 bf = load16(Bs[b] + (wn + 16 * j + r) * LDK + 8 * q);
#pragma unroll
        for (int i = 0; i < 2; ++i) MfmaBF16::mma(acc[b][i][j], af[i], bf);
      }
    __syncthreads();
  }

  // ---- epilogues: element (row m, column n) = acc[.][i][j][e]
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + wn + 16 * j + r;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + wm + 16 * i + 4 * q + e;
        const float v = acc[0][i][j][e];
        float y;
        if (EPI == kEpiQkvRope) {
          // RoPE pairs (2t, 2t+1) sit in adjacent lanes (columns r, r^1).
          const float partner = __shfl_xor(v, 1);
          y = v;
          if (part < 2 && m < a.M) {
            const int t = (n % a.Dh) >> 1;
            const float c = a.cos_t[m * (a.Dh / 2) + t], s = a.sin_t[m * (a.Dh / 2) + t];
            y = (n & 1) ? (partner * s + v * c) : (v * c - partner * s);
          }
        } else if (EPI == kEpiResidual) {
          y = m < a.M ? bf16_to_f32(a.res[(size_t)m * a.Npart + n]) + v : 0.0f;
        } else {
          y = silu(v) * acc[NB - 1][i][j][e];
        }
        if (m < a.M) a.out[part][(size_t)m * a.Npart + n] = f32_to_bf16(y);
      }
    }
}

// Causal attention for head dimension 64: one wave owns 16 query rows of one
// head and walks the key blocks of 32 up to its diagonal.
__global__ __launch_bounds__(64) void llama_attention_kernel(const uint16_t *__restrict__ Q,
                                                             const uint16_t *__restrict__ K,
                                                             const uint16_t *__restrict__ V,
                                                             uint16_t *__restrict__ O, int S,
                                                             int H, float scale) {
  constexpr int DH = 64;
  __shared__ __attribute__((aligned(16))) uint16_t Ps[16 * LDK];
  const int lane = threadIdx.x, r = lane & 15, q = lane >> 4;
  const int i0 = blockIdx.x * 16, h = blockIdx.y;
  const int D = H * DH;

  Frag16 qa[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
    qa[ks] = (i0 + r < S) ? load16(Q + (size_t)(i0 + r) * D + h * DH + 32 * ks + 8 * q) : frag_zero();

  float mrow[4], lrow[4];
  f32x4 o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    mrow[e] = -INFINITY;
    lrow[e] = 0.0f;
  }
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int kend = min(i0 + 16, S);
  for (int kb = 0; kb < kend; kb += 32) {
    f32x4 s[2];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      s[ct] = f32x4{0.f, 0.f, 0.f, 0.f};
      const int key = kb + 16 * ct + r;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const Frag16 kf = key < S ? load16(K + (size_t)key * D + h * DH + 32 * ks + 8 * q) : frag_zero();
        MfmaBF16::mma(s[ct], qa[ks], kf);
      }
    }
    float mx[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = i0 + 4 * q + e;
      mx[e] = -INFINITY;
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        const int key = kb + 16 * ct + r;
        const float v = (key <= row && key < S) ? s[ct][e] * scale : -INFINITY;
        s[ct][e] = v;
        mx[e] = fmaxf(mx[e], v);
      }
    }
#pragma unroll
    for (int off = 1; off < 16; off <<= 1)
#pragma unroll
      for (int e = 0; e < 4; ++e) mx[e] = fmaxf(mx[e], __shfl_xor(mx[e], off));
    float corr[4], sum[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float mnew = fmaxf(mrow[e], mx[e]);
      // rows past the end of the sequence see no key: keep them at zero
      corr[e] = (mnew == -INFINITY) ? 1.0f : expf(mrow[e] - mnew);
      sum[e] = 0.0f;
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        const float p = (mnew == -INFINITY) ? 0.0f : expf(s[ct][e] - mnew);
        s[ct][e] = p;
        sum[e] += p;
      }
      mrow[e] = mnew;
    }
#pragma unroll
    for (int off = 1; off < 16; off <<= 1)
#pragma unroll
      for (int e = 0; e < 4; ++e) sum[e] += __shfl_xor(sum[e], off);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      lrow[e] = lrow[e] * corr[e] + sum[e];
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) o[dt][e] *= corr[e];
    }
    // P (accumulator layout) -> LDS -> A-operand layout
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
      for (int e = 0; e < 4; ++e) Ps[(4 * q + e) * LDK + 16 * ct + r] = f32_to_bf16(s[ct][e]);
    __syncthreads();
    const Frag16 pa = load16(Ps + r * LDK + 8 * q);
    __syncthreads();
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      Frag16 vf;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int k0 = kb + 8 * q + 2 * jj;
        const uint32_t lo = k0 < S ? V[(size_t)k0 * D + h * DH + 16 * dt + r] : 0u;
        const uint32_t hi = k0 + 1 < S ? V[(size_t)(k0 + 1) * D + h * DH + 16 * dt + r] : 0u;
        vf.u[jj] = lo | (hi << 16);
      }
      MfmaBF16::mma(o[dt], pa, vf);
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int row = i0 + 4 * q + e;
    if (row >= S) continue;
    const float inv = 1.0f / lrow[e];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
      O[(size_t)row * D + h * DH + 16 * dt + r] = f32_to_bf16(o[dt][e] * inv);
  }
}

}  // namespace

hipError_t launch_llama_gemm(const LlamaGemmArgs &a, int pro, int epi, hipStream_t s) {
  const int tiles_n = (a.Npart / TN) * (epi == kEpiQkvRope ? a.nparts : 1);
  dim3 grid(tiles_n, (a.M + TM - 1) / TM);
  if (pro == kProRmsnorm && epi == kEpiQkvRope)
    hipLaunchKernelGGL((llama_gemm_kernel<kProRmsnorm, kEpiQkvRope>), grid, dim3(256), 0, s, a);
  else if (pro == kProPlain && epi == kEpiResidual)
    hipLaunchKernelGGL((llama_gemm_kernel<kProPlain, kEpiResidual>), grid, dim3(256), 0, s, a);
  else if (pro == kProRmsnorm && epi == kEpiSwiglu)
    hipLaunchKernelGGL((llama_gemm_kernel<kProRmsnorm, kEpiSwiglu>), grid, dim3(256), 0, s, a);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_llama_attention(const uint16_t *Q, const uint16_t *K, const uint16_t *V,
                                  uint16_t *O, int S, int H, float scale, hipStream_t s) {
  dim3 grid((S + 15) / 16, H);
  hipLaunchKernelGGL(llama_attention_kernel, grid, dim3(64), 0, s, Q, K, V, O, S, H, scale);
  return hipGetLastError();
}

}  // namespace npu
