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
// GEMM groups: one bf16 MFMA kernel (v_mfma_f32_16x16x32_bf16), 32x64
// workgroup tiles (the layer's M = 512 rows give 128-384 workgroups), K in
// chunks of 128 staged through double-buffered LDS: the next chunk's global
// loads are in flight while the current chunk is multiplied, one barrier per
// chunk.  Weights are row-major [K][N] as linalg.matmul takes them; each B
// chunk is transposed on its way into LDS, two k rows at a time, so that a
// lane's MFMA operand is one 16-byte k run.  RMSNorm is a prologue (row
// inverse-RMS, then the normalised bf16 A chunk is formed while staging);
// RoPE, residual and SiLU-gating are epilogues on the accumulators.
//
// Attention: causal flash attention, one workgroup per (head, 64 queries),
// four waves of 16 query rows.  Key blocks of 64 (K rows and V transposed)
// are staged once in LDS for the four waves, the next block prefetched into
// registers; online softmax in f32; P rounded to bf16 for its MFMA with V.
#include "kernels.hpp"
#include "npu_device.hpp"
#include "plans.hpp"

namespace npu {

namespace {

constexpr int TM = 32, TN = 64, TK = 128;
constexpr int LDA = TK + 16;  // LDS row stride (elements) of the [row][k] tiles: 288 bytes (32 mod 64)

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

__device__ __forceinline__ float bf_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

// Pack element j (0..7) of two 8-element bf16 runs into one 32-bit word:
// low half from run a, high half from run b.
__device__ __forceinline__ uint32_t pair_word(const u32x4 &a, const u32x4 &b, int j) {
  const uint32_t wa = a[j >> 1], wb = b[j >> 1];
  return (j & 1) ? ((wa >> 16) | (wb & 0xffff0000u)) : ((wa & 0xffffu) | (wb << 16));
}

__device__ __forceinline__ float sumsq8(const u32x4 &v) {
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float lo = bf_lo(v[j]), hi = bf_hi(v[j]);
    s += lo * lo;
    s += hi * hi;
  }
  return s;
}

template <int PRO, int EPI>
__global__ __launch_bounds__(256) void llama_gemm_kernel(const LlamaGemmArgs a) {
  constexpr int NB = (EPI == kEpiSwiglu) ? 2 : 1;
  constexpr int RPW = TM / 4;  // RMSNorm rows per wave
  __shared__ __attribute__((aligned(16))) uint16_t As[2][TM * LDA];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][NB][TN * LDA];
  __shared__ float inv_rms[TM];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int m0 = blockIdx.y * TM;
  const int tiles_per_part = a.Npart / TN;
  const int part = (EPI == kEpiQkvRope) ? blockIdx.x / tiles_per_part : 0;
  const int n0 = (blockIdx.x % tiles_per_part) * TN;
  const uint16_t *Bp[2] = {a.B[part], a.B[NB - 1]};

  if (PRO == kProRmsnorm) {
    // inverse RMS of the tile's rows, wave w owning rows RPW*w ..: all of a
    // wave's row loads are issued before any of them is reduced.
    float s[RPW];
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) s[rr] = 0.0f;
    for (int k = lane * 8; k < a.K; k += 512) {
      u32x4 v[RPW];
#pragma unroll
      for (int rr = 0; rr < RPW; ++rr) {
        const int row = m0 + wave * RPW + rr;
        v[rr] = row < a.M ? load16(a.A + (size_t)row * a.K + k).u : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int rr = 0; rr < RPW; ++rr) s[rr] += sumsq8(v[rr]);
    }
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) {
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) s[rr] += __shfl_xor(s[rr], off);
    }
    if (lane == 0) {
#pragma unroll
      for (int rr = 0; rr < RPW; ++rr)
        inv_rms[wave * RPW + rr] = 1.0f / sqrtf(s[rr] / (float)a.K + a.eps);
    }
    __syncthreads();
  }

  // staging: A chunk [32 rows][128 k] = two 8-element runs per thread;
  // B chunk [128 k][64 n] = four k rows (two pairs) x one 8-column run.
  const int arow = tid >> 3, akk = (tid & 7) * 8;
  const int bkp = (tid >> 3) * 2, bng = (tid & 7) * 8;
  u32x4 sa[2], sb[NB][4];
  auto fetch = [&](int k0) {
    const int row = m0 + arow;
    // K is a multiple of 64: the last chunk may hold only its first half,
    // the second half is zero-filled (and multiplies to zero).
    // (loads from clamped addresses, masked by selects: see masked())
    const int rowc = min(row, a.M - 1);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const bool ok = row < a.M && k0 + 64 * h < a.K;
      const int kc = min(k0 + 64 * h, a.K - 64);
      sa[h] = masked(load16(a.A + (size_t)rowc * a.K + kc + akk).u, ok);
    }
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const int k = k0 + bkp + (h & 1) + 64 * (h >> 1);
        sb[b][h] = masked(load16(Bp[b] + (size_t)min(k, a.K - 1) * a.Npart + n0 + bng).u,
                          k < a.K);
      }
  };
  auto commit = [&](int buf, int k0) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      u32x4 v = sa[h];
      const int kb = k0 + akk + 64 * h;
      if (PRO == kProRmsnorm && kb < a.K) {
        const float inv = inv_rms[arow];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float ylo = (bf_lo(v[j]) * inv) * a.gamma[kb + 2 * j];
          const float yhi = (bf_hi(v[j]) * inv) * a.gamma[kb + 2 * j + 1];
          v[j] = (uint32_t)f32_to_bf16(ylo) | ((uint32_t)f32_to_bf16(yhi) << 16);
        }
      }
      *reinterpret_cast<u32x4 *>(&As[buf][arow * LDA + akk + 64 * h]) = v;
    }
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int hp = 0; hp < 2; ++hp)
#pragma unroll
        for (int j = 0; j < 8; ++j)
          *reinterpret_cast<uint32_t *>(&Bs[buf][b][(bng + j) * LDA + bkp + 64 * hp]) =
              pair_word(sb[b][2 * hp], sb[b][2 * hp + 1], j);
  };

  f32x4 acc[NB][2];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[b][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // wave (wm, wn): rows 16*wm.., columns 32*wn.. (two 16-column tiles)
  const int wm = (wave & 1) * 16, wn = (wave >> 1) * 32;
  const int nchunks = (a.K + TK - 1) / TK;
  fetch(0);
  commit(0, 0);
  __syncthreads();
  for (int c = 0; c < nchunks; ++c) {
    if (c + 1 < nchunks) fetch((c + 1) * TK);
    const int buf = c & 1;
#pragma unroll
    for (int ks = 0; ks < TK / 32; ++ks) {
      const Frag16 af = load16(&As[buf][(wm + r) * LDA + 32 * ks + 8 * q]);
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const Frag16 bf = load16(&Bs[buf][b][(wn + 16 * j + r) * LDA + 32 * ks + 8 * q]);
          MfmaBF16::mma(acc[b][j], af, bf);
        }
    }
    if (c + 1 < nchunks) commit(buf ^ 1, (c + 1) * TK);
    __syncthreads();
  }

  // ---- epilogues: element (row m, column n) = acc[.][j][e]
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + wn + 16 * j + r;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = m0 + wm + 4 * q + e;
      const float v = acc[0][j][e];
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
        y = silu(v) * acc[NB - 1][j][e];
      }
      if (m < a.M) a.out[part][(size_t)m * a.Npart + n] = f32_to_bf16(y);
    }
  }
}

// Causal attention, head dimension 64.
constexpr int AQ = 64;          // queries per workgroup (4 waves x 16)
constexpr int AK = 64;          // keys per block
constexpr int LDK = 64 + 16;  // LDS row stride of K rows, V^T rows, P rows (elements): 160 bytes

__global__ __launch_bounds__(256) void llama_attention_kernel(const uint16_t *__restrict__ Q,
                                                              const uint16_t *__restrict__ K,
                                                              const uint16_t *__restrict__ V,
                                                              uint16_t *__restrict__ O, int S,
                                                              int H, float scale) {
  constexpr int DH = 64;
  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][AK * LDK];   // [key][d]
  __shared__ __attribute__((aligned(16))) uint16_t Vt[2][DH * LDK];   // [d][key]
  __shared__ __attribute__((aligned(16))) uint16_t Ps[4][16 * LDK];   // per wave [row][key]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int q0 = blockIdx.x * AQ, h = blockIdx.y;
  const int D = H * DH;
  const int i0 = q0 + wave * 16;  // this wave's first query row

  // query rows past S read row S-1: their outputs are never stored
  Frag16 qa[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
    qa[ks] = load16(Q + (size_t)min(i0 + r, S - 1) * D + h * DH + 32 * ks + 8 * q);

  // staging: K block [64 keys][64 d] = 2 runs of 8 per thread; V block
  // transposed: two keys x 8 d per thread.
  const int kr = tid >> 2, kd = (tid & 3) * 16;       // K: key kr, d kd..kd+15
  const int vk = (tid >> 3) * 2, vd = (tid & 7) * 8;  // V: keys vk, vk+1; d vd..vd+7
  u32x4 sk[2], sv[2];
  auto fetch = [&](int kb) {
    const int key = kb + kr;
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
      sk[s2] = masked(load16(K + (size_t)min(key, S - 1) * D + h * DH + kd + 8 * s2).u, key < S);
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const int vkey = kb + vk + s2;
      sv[s2] = masked(load16(V + (size_t)min(vkey, S - 1) * D + h * DH + vd).u, vkey < S);
    }
  };
  auto commit = [&](int buf) {
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
      *reinterpret_cast<u32x4 *>(&Ks[buf][kr * LDK + kd + 8 * s2]) = sk[s2];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      *reinterpret_cast<uint32_t *>(&Vt[buf][(vd + j) * LDK + vk]) = pair_word(sv[0], sv[1], j);
  };

  float mrow[4], lrow[4];
  f32x4 o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    mrow[e] = -INFINITY;
    lrow[e] = 0.0f;
  }
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int kend = min(q0 + AQ, S);  // keys beyond the block's last query are masked for all
  const int nblocks = (kend + AK - 1) / AK;
  fetch(0);
  commit(0);
  __syncthreads();
  for (int blk = 0; blk < nblocks; ++blk) {
    const int kb = blk * AK;
    if (blk + 1 < nblocks) fetch(kb + AK);
    const int buf = blk & 1;
    const bool active = kb <= i0 + 15;  // some key of the block is visible to this wave
    if (active) {
      f32x4 s[4];
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        s[ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const Frag16 kf = load16(&Ks[buf][(16 * ct + r) * LDK + 32 * ks + 8 * q]);
          MfmaBF16::mma(s[ct], qa[ks], kf);
        }
      }
      float mx[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = i0 + 4 * q + e;
        mx[e] = -INFINITY;
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
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
        corr[e] = (mnew == -INFINITY) ? 1.0f : expf(mrow[e] - mnew);
        sum[e] = 0.0f;
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
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
      // P (accumulator layout) -> this wave's LDS rows -> A-operand layout.
      // Only this wave touches Ps[wave]; LDS operations of a wave complete in
      // order, and the explicit wait makes the stores visible to the loads.
#pragma unroll
      for (int ct = 0; ct < 4; ++ct)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          Ps[wave][(4 * q + e) * LDK + 16 * ct + r] = f32_to_bf16(s[ct][e]);
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const Frag16 pa = load16(&Ps[wave][r * LDK + 32 * ks + 8 * q]);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          const Frag16 vf = load16(&Vt[buf][(16 * dt + r) * LDK + 32 * ks + 8 * q]);
          MfmaBF16::mma(o[dt], pa, vf);
        }
      }
    }
    if (blk + 1 < nblocks) commit(buf ^ 1);
    __syncthreads();
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

namespace {

// Launch plan of one GEMM variant: a TM x (NB*TN) output tile walks K in
// TK chunks (double-buffered: each chunk's loads overlap the previous
// chunk's MFMAs, so one exposed load phase plus the prologue's row loads).
template <class Kern>
void plan_gemm(const char *name, Kern kern, const LlamaGemmArgs &a, int grid, int nb, bool norm,
               int epi) {
  const int kchunks = (a.K + TK - 1) / TK;
  npu_launch_plan p = make_plan(name, grid, wg_per_cu(kern), grid, 16);
  p.load_phases = norm ? 2 : 1;
  p.tile_macs = (double)TM * TN * nb * kchunks * TK;
  p.tile_valu = (norm ? 3.0 * TM * a.K : 0.0) + (double)TM * TN * nb * (epi == kEpiResidual ? 3 : 8);
  p.tile_lds_bytes = 2.0 * ((double)TM + nb * TN) * kchunks * TK * 2;   // written once, read once
  p.tile_load_bytes = ((double)TM + nb * TN) * kchunks * TK * 2 + (norm ? 4.0 * a.K : 0.0);
  p.tile_store_bytes = (double)TM * TN * 2;
  const double parts = epi == kEpiQkvRope ? a.nparts : (epi == kEpiSwiglu ? 2 : 1);
  p.hbm_bytes = 2.0 * ((double)a.M * a.K + parts * a.K * a.Npart +
                       (double)a.M * a.Npart * (epi == kEpiQkvRope ? a.nparts : 1) +
                       (epi == kEpiResidual ? (double)a.M * a.Npart : 0.0)) +
                (norm ? 4.0 * a.K : 0.0) + (epi == kEpiQkvRope ? 2.0 * 4 * a.M * a.Dh / 2 : 0.0);
  plans_add(p);
}

}  // namespace

hipError_t launch_llama_gemm(const LlamaGemmArgs &a, int pro, int epi, hipStream_t s) {
  const int tiles_n = (a.Npart / TN) * (epi == kEpiQkvRope ? a.nparts : 1);
  dim3 grid(tiles_n, (a.M + TM - 1) / TM);
  const int g = grid.x * grid.y;
  if (pro == kProRmsnorm && epi == kEpiQkvRope) {
    plan_gemm("llama_rmsnorm_qkv_rope", llama_gemm_kernel<kProRmsnorm, kEpiQkvRope>, a, g, 1, true, epi);
    hipLaunchKernelGGL((llama_gemm_kernel<kProRmsnorm, kEpiQkvRope>), grid, dim3(256), 0, s, a);
  } else if (pro == kProPlain && epi == kEpiResidual) {
    plan_gemm("llama_matmul_residual", llama_gemm_kernel<kProPlain, kEpiResidual>, a, g, 1, false, epi);
    hipLaunchKernelGGL((llama_gemm_kernel<kProPlain, kEpiResidual>), grid, dim3(256), 0, s, a);
  } else if (pro == kProRmsnorm && epi == kEpiSwiglu) {
    plan_gemm("llama_rmsnorm_swiglu", llama_gemm_kernel<kProRmsnorm, kEpiSwiglu>, a, g, 2, true, epi);
    hipLaunchKernelGGL((llama_gemm_kernel<kProRmsnorm, kEpiSwiglu>), grid, dim3(256), 0, s, a);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_llama_attention(const uint16_t *Q, const uint16_t *K, const uint16_t *V,
                                  uint16_t *O, int S, int H, float scale, hipStream_t s) {
  dim3 grid((S + AQ - 1) / AQ, H);
  {
    // Causal: query block b sees key blocks 0..b, so the average tile walks
    // (nqb + 1) / 2 key blocks; every key block costs QK^T and PV MFMAs, the
    // online-softmax update, and one staged K and V^T block.
    const int nqb = grid.x;
    const double kblocks = (nqb + 1) / 2.0;
    npu_launch_plan p = make_plan("llama_causal_attention", grid.x * grid.y,
                                  wg_per_cu(llama_attention_kernel), grid.x * grid.y, 16);
    p.load_phases = 1;
    p.tile_macs = kblocks * 2.0 * AQ * AK * 64;
    p.tile_valu = kblocks * (double)AQ * AK * 12;
    p.tile_lds_bytes = kblocks * (2.0 * 2 * AK * 64 * 2 + 2.0 * AQ * AK * 2 + 4.0 * AQ * 64 * 2);
    p.tile_load_bytes = kblocks * 2.0 * AK * 64 * 2 + AQ * 64 * 2.0;
    p.tile_store_bytes = AQ * 64 * 2.0;
    p.hbm_bytes = 4.0 * S * H * 64 * 2;  // Q, K, V in, O out
    plans_add(p);
  }
  hipLaunchKernelGGL(llama_attention_kernel, grid, dim3(256), 0, s, Q, K, V, O, S, H, scale);
  return hipGetLastError();
}

}  // namespace npu
