// k_llama.hip -- the fused groups of one Llama decoder layer, bf16 storage,
// f32 accumulation (the Llama block the reference approximates in
// test/llama_attention.mlir:5-67, with the softmax, RMSNorm, RoPE and SwiGLU
// that it replaces by ReLU or omits, :39-52):
//
//   qkv   : xn = bf16(rmsnorm(x)*g1); Q,K = bf16(rope(xn@Wq|Wk)); V = bf16(xn@Wv)
//   attn  : A = bf16(softmax_causal(Q K^T * scale) V) per head
//   oproj : h = bf16(x + A@Wo)
//   swiglu: hn = bf16(rmsnorm(h)*g2); act = bf16(silu(hn@Wg) * (hn@Wu))
//   down  : out = bf16(h + act@Wd)
//
// GEMMs.  One bf16 MFMA kernel (v_mfma_f32_16x16x32_bf16) with the operands
// swapped: the weight fragment is the MFMA's A operand and the activation
// fragment its B operand, so an accumulator lane holds four consecutive
// output columns of one row -- RoPE pairs and the gate/up pair of SwiGLU are
// in one lane, and every store is 8 bytes.  The weights are row-major [K][N]
// as linalg.matmul takes them; their MFMA fragment needs eight consecutive k
// of one column, so they go through LDS untransposed, as 16-column strips of
// 32-byte rows, and come out with gfx950's transposing LDS read
// (ds_read_b64_tr_b16: in each 16-lane group, lane 4a+e receives element e
// of the 8-byte rows addressed by lanes 4j+a, j = 0..3).  The activation
// fragment is one 16-byte run of a row (row-major [M][K] in LDS).  Rows of a
// strip are stored permuted within each 32-row group (row 8g+4r+j at
// 16r+4g+j) so that the 32 lanes a transposing read serves per clock read
// 256 contiguous bytes.  The RMSNorm GEMMs stage their whole A panel (all of
// K, the layer's d_model) once, reduce each row in registers and write it
// back normalised; the others stream A and B in K chunks, double-buffered,
// the next chunk's loads in flight during the current chunk's MFMAs.
// Workgroups map to tiles XCD by XCD (workgroups are dispatched round-robin
// over the eight XCDs): the tiles of one XCD share their weight columns, so
// each XCD's L2 holds only its share of the weights.
//
// Attention.  One workgroup per (head, 16 queries): 256 workgroups at the
// layer's shape.  The four waves take 32-key blocks round-robin; each keeps
// an online-softmax state for the 16 queries (running max, partial sums,
// unnormalised O^T) and the states meet in LDS at the end.  S^T = K Q^T puts
// the keys on the accumulator's rows, so the probabilities P^T feed the
// P^T-side operand of O^T = V^T P^T straight from registers, and V^T is the
// transposing LDS read of the row-major V block.  P is rounded to bf16 for
// its MFMA (the oracle keeps it in f32).  All heads of one XCD's workgroups
// are the same, so the L2 of an XCD holds one head's K and V.
#include <cmath>

#include "kernels.hpp"
#include "npu_device.hpp"
#include "persistent.hpp"
#include "plans.hpp"

namespace npu {

namespace {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// Eight bf16 of one column, k = 8g .. 8g+7 of a 32-row k step, from a
// 16-column B strip in LDS (two transposing reads of four k each; the four
// 16-bit results of a read are the two dwords of the fragment half).
__device__ __forceinline__ Frag16 read_wfrag(const unsigned char *strip, int kstep, int lane) {
  const int g = lane >> 4, j = (lane >> 2) & 3, a = lane & 3;
  // physical row of logical row 8g + 4r + j (r = 0, 1) is 16r + 4g + j
  const unsigned char *p0 = strip + (kstep * 32 + 4 * g + j) * 32 + a * 8;
  const uint2 lo = __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(p0)));
  const uint2 hi = __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(p0 + 16 * 32)));
  Frag16 f;
  f.u = u32x4{lo.x, lo.y, hi.x, hi.y};
  return f;
}

// Physical row, within a chunk, of chunk row k (see read_wfrag).
__device__ __forceinline__ int strip_row(int k) {
  const int kl = k & 31;
  return (k & ~31) + 16 * ((kl >> 2) & 1) + 4 * (kl >> 3) + (kl & 3);
}

__device__ __forceinline__ uint2 pack4_bf16(float a, float b, float c, float d) {
  return make_uint2(cvt_pk_bf16(a, b), cvt_pk_bf16(c, d));
}

__device__ __forceinline__ float bf_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

// Tile of this workgroup among tiles_m x tiles_n tiles: with xm > 0 the 2-D
// XCD blocks of xcd_block_tile; else the N-major tile list cut into 8
// contiguous ranges, range x on XCD x (blockIdx.x % 8).  Returns false for
// the padding workgroups of a grid rounded up to a multiple of 8.
__device__ __forceinline__ bool xcd_tile(int tiles_m, int tiles_n, int xm, int &tm, int &tn) {
  if (xm > 0) {
    xcd_block_tile(tiles_m, tiles_n, xm, tm, tn);
    return true;
  }
  const int G = tiles_m * tiles_n, per = (G + 7) / 8;
  const int t = (blockIdx.x % 8) * per + blockIdx.x / 8;
  if (t >= G) return false;
  tn = t / tiles_m;
  tm = t % tiles_m;
  return true;
}

constexpr int APAD = 16;  // A row padding (elements): row stride = 32 mod 64 bytes
constexpr int GT = 1024;  // GEMM workgroup: 16 waves, four per SIMD

// BM x BN output tile (per weight: NB = 2 for gate and up) of 16 waves:
// WR row strips of 16 rows x WC column groups x WK parts of K.  Every global
// load of the tile is issued up front -- the RMSNorm A panel, then all of B
// (and A) in chunks of KC rows (at most NCH chunks), then the epilogue's own
// inputs -- and the chunks are stored to LDS as their loads arrive, into two
// buffers when there are several (one barrier per chunk).  With K split
// (WK > 1) the partial sums go to a dense [WK][BM][NB BN] array in LDS and
// every thread sums and finishes whole quads (four consecutive columns of one
// row) of the tile; with WK = 1 each lane finishes its own accumulator quads.
// kProRmsnorm keeps the whole A panel (K <= KMAX) in LDS.
template <int PRO, int EPI, int BM, int BN, int WR, int WC, int WK, int KC, int NCH, int KMAX>
struct GemmShape {
  static constexpr int kBM = BM, kBN = BN, kWK = WK, kWC = WC;
  static constexpr int PPL = KMAX / 512;  // RMSNorm panel: 8-element pieces per lane and row
  static constexpr int NB = EPI == kEpiSwiglu ? 2 : 1;
  static constexpr int TMW = BM / WR / 16, TNW = BN / WC / 16;  // MFMA tiles of a wave
  static constexpr int STRIPS = BN / 16;
  static constexpr int SB = KC * 32 + 64;                        // bytes of one 16-column strip
  static constexpr int BCHUNK = NB * STRIPS * SB;
  static constexpr int CPR = NB * BN / 8;                        // 16-byte pieces per B row
  static constexpr int BITEMS = KC * CPR, BPER = (BITEMS + GT - 1) / GT;
  static constexpr int ALD = KC + APAD;                          // plain A chunk row stride
  static constexpr int AITEMS = BM * KC / 8, APER = (AITEMS + GT - 1) / GT;
  static constexpr int RLD = NB * BN + 4;                        // partial-sum row stride (floats)
  static constexpr int RED = WK > 1 ? WK * BM * RLD * 4 : 0;     // bytes of the partial sums
  static constexpr int QUADS = BM * BN / 4, QPER = (QUADS + GT - 1) / GT;
  static_assert(WR * WC * WK == 16 && TMW >= 1 && TNW >= 1, "sixteen waves cover the tile");
  static_assert(BN % 16 == 0 && BM % 16 == 0 && KC % 32 == 0, "MFMA tiles");
  // K chunks staged in LDS: two buffers when there are several chunks (the
  // next chunk is written while the current one is multiplied)
  static constexpr int NBUF = NCH > 1 ? 2 : 1;
  static constexpr int ACHUNK = BM * ALD * 2;  // bytes of one plain A chunk
  __host__ __device__ static size_t abytes(int K) {
    return PRO == kProRmsnorm ? (size_t)BM * (K + APAD) * 2 : (size_t)NBUF * ACHUNK;
  }
  static size_t lds_bytes(int K) {
    const size_t main = abytes(K) + (size_t)NBUF * BCHUNK;
    return main > (size_t)RED ? main : (size_t)RED;
  }
};

// SiLU with the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32).
__device__ __forceinline__ float silu_fast(float g) {
  return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * g));
}

template <int PRO, int EPI, int BM, int BN, int WR, int WC, int WK, int KC, int NCH, int KMAX>
__global__ __launch_bounds__(GT) void llama_gemm_kernel(const LlamaGemmArgs a, int tiles_m,
                                                        int tiles_n, int xm) {
  using S = GemmShape<PRO, EPI, BM, BN, WR, WC, WK, KC, NCH, KMAX>;
  constexpr int NB = S::NB, TMW = S::TMW, TNW = S::TNW;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  int tm, tn;
  if (!xcd_tile(tiles_m, tiles_n, xm, tm, tn)) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int M = a.M, K = a.K, Np = a.Npart;
  const int m0 = tm * BM, n0 = tn * BN;  // n0: column over all parts (QKV: 3 Np)
  const int lda = PRO == kProRmsnorm ? K + APAD : S::ALD;
  unsigned char *const As = smem;
  unsigned char *const Bs = smem + S::abytes(K);
  const int nchunks = (K + KC - 1) / KC;  // <= NCH (checked at launch)

  // ---- RMSNorm A panel and gains first: the prologue waits for these only
  // (a wave's loads complete in order)
  constexpr int PPL = S::PPL, RPW = (BM + 15) / 16;
  const int pieces = K / 8;
  u32x4 x[PRO == kProRmsnorm ? RPW : 1][PPL];
  f32x4 g0[PPL], g1[PPL];  // gamma of this lane's pieces
  if constexpr (PRO == kProRmsnorm) {
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr)
#pragma unroll
      for (int p = 0; p < PPL; ++p) {
        const int row = min(m0 + min(wave + 16 * rr, BM - 1), M - 1);
        const int pc = min(lane + 64 * p, pieces - 1);
        x[rr][p] = *reinterpret_cast<const u32x4 *>(a.A + (size_t)row * K + pc * 8);
      }
#pragma unroll
    for (int p = 0; p < PPL; ++p) {
      const int pc = min(lane + 64 * p, pieces - 1);
      g0[p] = *reinterpret_cast<const f32x4 *>(a.gamma + pc * 8);
      g1[p] = *reinterpret_cast<const f32x4 *>(a.gamma + pc * 8 + 4);
    }
  }

  // ---- every chunk of B (and of a plain GEMM's A): 16-byte pieces
  const uint16_t *bsrc[S::BPER];
  int bdst[S::BPER], bk[S::BPER];
#pragma unroll
  for (int i = 0; i < S::BPER; ++i) {
    const int item = tid + GT * i;
    const bool ok = item < S::BITEMS;
    const int it = ok ? item : 0;
    const int k = it / S::CPR, c = it % S::CPR;
    const int nb = c / (BN / 8), cc = c % (BN / 8);
    const int gc = n0 + cc * 8;  // global column (over parts for QKV)
    const int part = EPI == kEpiQkvRope ? gc / Np : nb;
    const int col = EPI == kEpiQkvRope ? gc % Np : gc;
    bsrc[i] = a.B[part] + col;
    bdst[i] = ok ? (nb * S::STRIPS + cc / 2) * S::SB + strip_row(k) * 32 + (cc & 1) * 16 : -1;
    bk[i] = k;
  }
  u32x4 breg[NCH][S::BPER];
  // Rows of a chunk past K (the last chunk, or a chunk longer than K) load
  // row K - 1 instead: in bounds, and never read back (the k steps stop at K).
#pragma unroll
  for (int c = 0; c < NCH; ++c)
#pragma unroll
    for (int i = 0; i < S::BPER; ++i)
      if (c < nchunks)
        breg[c][i] = *reinterpret_cast<const u32x4 *>(bsrc[i] + (size_t)min(c * KC + bk[i], K - 1) * Np);

  const uint16_t *asrc[S::APER];
  int adst[S::APER], akc[S::APER];
  u32x4 areg[PRO == kProRmsnorm ? 1 : NCH][S::APER];
  if constexpr (PRO != kProRmsnorm) {
#pragma unroll
    for (int i = 0; i < S::APER; ++i) {
      const int item = tid + GT * i;
      const bool ok = item < S::AITEMS;
      const int it = ok ? item : 0;
      const int row = it / (KC / 8), kc = it % (KC / 8);
      asrc[i] = a.A + (size_t)min(m0 + row, M - 1) * K;
      adst[i] = ok ? (row * S::ALD + kc * 8) * 2 : -1;
      akc[i] = kc * 8;
    }
    // pieces past K load the row's last piece (K is a multiple of 8)
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int i = 0; i < S::APER; ++i)
        if (c < nchunks)
          areg[c][i] = *reinterpret_cast<const u32x4 *>(asrc[i] + min(c * KC + akc[i], K - 8));
  }

  // wave (wr, wc, wk): rows wr * BM/WR .., columns wc * BN/WC .., k steps wk, wk + WK, ...
  const int wr = wave % WR, wc = (wave / WR) % WC, wk = wave / (WR * WC);
  const int ml = lane & 15, ng = 4 * (lane >> 4);  // accumulator: row ml, columns ng .. ng+3

  // ---- the epilogue's quads (four consecutive columns of one row of the
  // tile).  With K split over the waves (WK > 1), quad q = tid + GT e of the
  // summed tile, row q / (BN / 4), columns 4 (q % (BN / 4)) .. +3; without
  // (WK = 1), the lane's own accumulator quads, one per 16 x 16 block (i, j)
  // with e = i TNW + j.  Their inputs are loaded here, before the K loop.
  constexpr int NQ = WK > 1 ? S::QPER : TMW * TNW;
  auto quad_of = [&](int e, int &row, int &col) __attribute__((always_inline)) {
    if constexpr (WK > 1) {
      const int q = min(tid + GT * e, S::QUADS - 1);
      row = q / (BN / 4);
      col = 4 * (q % (BN / 4));
    } else {
      row = wr * (BM / WR) + 16 * (e / TNW) + ml;
      col = wc * (BN / WC) + 16 * (e % TNW) + ng;
    }
  };
  uint2 res[NQ];
  float2 cs[NQ], sn[NQ];
#pragma unroll
  for (int e = 0; e < NQ; ++e) {
    int row, col;
    quad_of(e, row, col);
    const int m = min(m0 + row, M - 1), n = n0 + col;
    if constexpr (EPI == kEpiResidual)
      res[e] = *reinterpret_cast<const uint2 *>(a.res + (size_t)m * Np + n);
    if constexpr (EPI == kEpiQkvRope) {
      const int t = ((n % Np) % a.Dh) / 2;
      cs[e] = *reinterpret_cast<const float2 *>(a.cos_t + (size_t)m * (a.Dh / 2) + t);
      sn[e] = *reinterpret_cast<const float2 *>(a.sin_t + (size_t)m * (a.Dh / 2) + t);
    }
  }

  // ---- RMSNorm prologue: wave w normalises rows w, w + 16, ... of the panel
  if constexpr (PRO == kProRmsnorm) {
    const float invk = 1.0f / (float)K;
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) {
      const int row = wave + 16 * rr;
      if (row >= BM) break;  // wave-uniform
      float ss = 0.0f;
#pragma unroll
      for (int p = 0; p < PPL; ++p) {
        float part = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float lo = bf_lo(x[rr][p][e]), hi = bf_hi(x[rr][p][e]);
          part = fmaf(lo, lo, part);
          part = fmaf(hi, hi, part);
        }
        ss += lane + 64 * p < pieces ? part : 0.0f;
      }
      const float inv = __builtin_amdgcn_rsqf(wave_sum(ss) * invk + a.eps);
#pragma unroll
      for (int p = 0; p < PPL; ++p) {
        if (lane + 64 * p >= pieces) continue;
        const u32x4 v = x[rr][p];
        const f32x4 gl = g0[p], gh = g1[p];
        u32x4 o;
        o[0] = cvt_pk_bf16((bf_lo(v[0]) * inv) * gl[0], (bf_hi(v[0]) * inv) * gl[1]);
        o[1] = cvt_pk_bf16((bf_lo(v[1]) * inv) * gl[2], (bf_hi(v[1]) * inv) * gl[3]);
        o[2] = cvt_pk_bf16((bf_lo(v[2]) * inv) * gh[0], (bf_hi(v[2]) * inv) * gh[1]);
        o[3] = cvt_pk_bf16((bf_lo(v[3]) * inv) * gh[2], (bf_hi(v[3]) * inv) * gh[3]);
        *reinterpret_cast<u32x4 *>(As + ((size_t)row * lda + (lane + 64 * p) * 8) * 2) = o;
      }
    }
  }

  f32x4 acc[NB][TMW][TNW];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int i = 0; i < TMW; ++i)
#pragma unroll
      for (int j = 0; j < TNW; ++j) acc[b][i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // chunk c lives in buffer c % NBUF; with two buffers, chunk c + 2 is
  // written once every wave is done with chunk c, so each chunk costs one
  // barrier
  auto write_chunk = [&](int chunk, int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < S::BPER; ++i)
      if (bdst[i] >= 0) *reinterpret_cast<u32x4 *>(Bs + (size_t)buf * S::BCHUNK + bdst[i]) = breg[chunk][i];
    if constexpr (PRO != kProRmsnorm) {
#pragma unroll
      for (int i = 0; i < S::APER; ++i)
        if (adst[i] >= 0) *reinterpret_cast<u32x4 *>(As + (size_t)buf * S::ACHUNK + adst[i]) = areg[chunk][i];
    }
  };
  write_chunk(0, 0);
  if constexpr (S::NBUF == 2)
    if (nchunks > 1) write_chunk(1, 1);
  __syncthreads();
#pragma unroll
  for (int chunk = 0; chunk < NCH; ++chunk) {
    if (chunk >= nchunks) break;
    const int buf = chunk % S::NBUF;
    const unsigned char *abuf = PRO == kProRmsnorm ? As + (size_t)chunk * KC * 2 : As + (size_t)buf * S::ACHUNK;
    const unsigned char *bbuf = Bs + (size_t)buf * S::BCHUNK;
    const int steps = min(KC, K - chunk * KC) / 32;
    for (int s = wk; s < steps; s += WK) {
      Frag16 xf[TMW], wf[NB][TNW];
#pragma unroll
      for (int i = 0; i < TMW; ++i) {
        const int row = wr * (BM / WR) + 16 * i + ml;
        xf[i].u = *reinterpret_cast<const u32x4 *>(abuf + ((size_t)row * lda + s * 32 + 8 * (lane >> 4)) * 2);
      }
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int j = 0; j < TNW; ++j)
          wf[b][j] = read_wfrag(bbuf + (b * S::STRIPS + wc * TNW + j) * S::SB, s, lane);
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int i = 0; i < TMW; ++i)
#pragma unroll
          for (int j = 0; j < TNW; ++j)
            acc[b][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[b][j].h, xf[i].h, acc[b][i][j], 0, 0, 0);
    }
    if (chunk + 1 < nchunks) {
      __syncthreads();  // every wave is done with this chunk's buffer
      if constexpr (S::NBUF == 1) {
        write_chunk(chunk + 1, 0);
        __syncthreads();
      } else if (chunk + 2 < nchunks) {
        write_chunk(chunk + 2, buf);  // read after the next chunk's barrier
      }
    }
  }

  // ---- with K split, the partial sums -> LDS [WK][BM][NB BN], summed per quad
  [[maybe_unused]] float *red = reinterpret_cast<float *>(smem);
  if constexpr (WK > 1) {
    __syncthreads();  // LDS is free
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int i = 0; i < TMW; ++i)
#pragma unroll
        for (int j = 0; j < TNW; ++j) {
          const int row = wr * (BM / WR) + 16 * i + ml;
          const int col = b * BN + wc * (BN / WC) + 16 * j + ng;
          *reinterpret_cast<f32x4 *>(red + ((size_t)wk * BM + row) * S::RLD + col) = acc[b][i][j];
        }
    __syncthreads();
  }
#pragma unroll
  for (int e = 0; e < NQ; ++e) {
    if (WK > 1 && tid + GT * e >= S::QUADS) break;
    int row, col;
    quad_of(e, row, col);
    const int m = m0 + row, n = n0 + col;
    if (m >= M) continue;
    f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f}, u = f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (WK > 1) {
#pragma unroll
      for (int w = 0; w < WK; ++w) {
        v += *reinterpret_cast<const f32x4 *>(red + ((size_t)w * BM + row) * S::RLD + col);
        if constexpr (NB == 2) u += *reinterpret_cast<const f32x4 *>(red + ((size_t)w * BM + row) * S::RLD + BN + col);
      }
    } else {
      v = acc[0][e / TNW][e % TNW];
      if constexpr (NB == 2) u = acc[NB - 1][e / TNW][e % TNW];
    }
    uint2 o;
    uint16_t *dst;
    if constexpr (EPI == kEpiQkvRope) {
      const int part = n / Np, c = n % Np;
      if (part < 2) {
        // (2t, 2t+1) -> (x0 c - x1 s, x0 s + x1 c)
        const float2 cc = cs[e], ss = sn[e];
        o = pack4_bf16(v[0] * cc.x - v[1] * ss.x, v[0] * ss.x + v[1] * cc.x,
                       v[2] * cc.y - v[3] * ss.y, v[2] * ss.y + v[3] * cc.y);
      } else {
        o = pack4_bf16(v[0], v[1], v[2], v[3]);
      }
      dst = a.out[part] + (size_t)m * Np + c;
    } else if constexpr (EPI == kEpiResidual) {
      const uint2 r = res[e];
      o = pack4_bf16(bf_lo(r.x) + v[0], bf_hi(r.x) + v[1], bf_lo(r.y) + v[2], bf_hi(r.y) + v[3]);
      dst = a.out[0] + (size_t)m * Np + n;
    } else {
      o = pack4_bf16(silu_fast(v[0]) * u[0], silu_fast(v[1]) * u[1], silu_fast(v[2]) * u[2],
                     silu_fast(v[3]) * u[3]);
      dst = a.out[0] + (size_t)m * Np + n;
    }
    *reinterpret_cast<uint2 *>(dst) = o;
  }
}

// ---- attention ----------------------------------------------------------------
constexpr int AQ = 16;    // queries per workgroup
constexpr int AKB = 32;   // keys per block
constexpr int AWAVES = 4;
// Per head dim DH (64 or 128): Q / K fragments per row (8 dh per lane group,
// four groups), the V block's LDS row stride (DH + 16 elements: 32 mod 64
// bytes), 16-byte V pieces per lane of a 32-key block, 16-wide output tiles.
template <int DH>
struct AttnShape {
  static_assert(DH == 64 || DH == 128, "head dims 64 and 128");
  static constexpr int NQF = DH / 32, VLD = DH + 16, PPR = DH / 8, NVR = AKB * PPR / 64,
                       NDT = DH / 16;
};

// S^T tile (16 keys x 16 queries) of key tile t: lane holds keys 4g + r of the
// tile (g = lane / 16), query lane % 16.  P^T's fragment for the 32-key
// block then has, in lane (g, q), keys 4g + r and 16 + 4g + r (k slots 0..7):
// V^T's fragment must list the same keys, which the transposing read gives
// when lane (g, j, a) addresses V row (16 h + 4 g + j), columns 4a .. 4a+3
// of the dh tile, for halves h = 0, 1.
template <int VLD>
__device__ __forceinline__ Frag16 read_vfrag(const uint16_t *vs, int dtile, int lane) {
  const int g = lane >> 4, j = (lane >> 2) & 3, a = lane & 3;
  const uint16_t *p0 = vs + (4 * g + j) * VLD + dtile * 16 + 4 * a;
  const uint2 lo = __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(p0)));
  const uint2 hi = __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(p0 + 16 * VLD)));
  Frag16 f;
  f.u = u32x4{lo.x, lo.y, hi.x, hi.y};
  return f;
}

template <int DH>
__global__ __launch_bounds__(256) void llama_attention_kernel(const uint16_t *__restrict__ Q,
                                                              const uint16_t *__restrict__ Kg,
                                                              const uint16_t *__restrict__ V,
                                                              uint16_t *__restrict__ O, int S,
                                                              int H, float scale) {
  using Sh = AttnShape<DH>;
  constexpr int NQF = Sh::NQF, VLD = Sh::VLD, PPR = Sh::PPR, NVR = Sh::NVR, NDT = Sh::NDT;
  __shared__ __attribute__((aligned(16))) uint16_t vbuf[AWAVES][2][AKB * VLD];
  __shared__ float st_m[AWAVES][AQ], st_l[AWAVES][AQ];
  __shared__ float st_o[AWAVES][DH][AQ + 1];
  const int nqb = (S + AQ - 1) / AQ, G = nqb * H, per = (G + 7) / 8;
  const int t = (blockIdx.x % 8) * per + blockIdx.x / 8;
  if (t >= G) return;
  const int h = t / nqb, qb = t % nqb;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, ql = lane & 15;
  const int D = H * DH;
  const int q0 = qb * AQ;
  const int nkb = (q0 + AQ + AKB - 1) / AKB;  // key blocks 0 .. nkb-1 hold keys <= q0 + 15
  const float kscale = scale * 1.4426950408889634f;  // exp(x * scale) = exp2(x * kscale)

  // Rows past S (the last query or key block of a sequence that is not a
  // multiple of 16 or 32) are read from row S - 1: such keys lie above the
  // diagonal of every query that is stored, so the causal mask removes them,
  // and such queries are not stored.
  // Q^T fragments (B operand): query ql, dh 32 k + 8g .. +8
  Frag16 qf[NQF];
  {
    const uint16_t *qp = Q + (size_t)min(q0 + ql, S - 1) * D + h * DH + 8 * g;
#pragma unroll
    for (int k = 0; k < NQF; ++k) qf[k] = load16(qp + 32 * k);
  }
  float m_run = -__builtin_inff(), l_run = 0.0f;
  f32x4 o[NDT];
#pragma unroll
  for (int d = 0; d < NDT; ++d) o[d] = f32x4{0.f, 0.f, 0.f, 0.f};

  // block kb = wave, wave + 4, ...: K fragments (A operand: key 16 t + (lane % 16),
  // dh 32 k + 8g .. +8) and the V block (32 keys x DH, NVR x 16 bytes per lane)
  Frag16 kf[2][NQF];
  u32x4 vr[NVR];
  auto fetch = [&](int kb) {
    const int k0 = min(kb, nkb - 1) * AKB;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const uint16_t *kp = Kg + (size_t)min(k0 + 16 * tt + ql, S - 1) * D + h * DH + 8 * g;
#pragma unroll
      for (int k = 0; k < NQF; ++k) kf[tt][k] = load16(kp + 32 * k);
    }
#pragma unroll
    for (int i = 0; i < NVR; ++i) {
      const int item = lane + 64 * i;  // AKB * PPR pieces: key item / PPR, dh 8 (item % PPR)
      vr[i] = *reinterpret_cast<const u32x4 *>(V + (size_t)min(k0 + item / PPR, S - 1) * D + h * DH +
                                               (item % PPR) * 8);
    }
  };
  int buf = 0;
  if (wave < nkb) fetch(wave);
  for (int kb = wave; kb < nkb; kb += AWAVES) {
    uint16_t *vs = vbuf[wave][buf];
#pragma unroll
    for (int i = 0; i < NVR; ++i) {
      const int item = lane + 64 * i;
      *reinterpret_cast<u32x4 *>(vs + (item / PPR) * VLD + (item % PPR) * 8) = vr[i];
    }
    Frag16 kc[2][NQF];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int k = 0; k < NQF; ++k) kc[tt][k] = kf[tt][k];
    if (kb + AWAVES < nkb) fetch(kb + AWAVES);
    // S^T = K Q^T: two 16-key tiles
    f32x4 s[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      s[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kc[tt][0].h, qf[0].h, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
      for (int k = 1; k < NQF; ++k)
        s[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kc[tt][k].h, qf[k].h, s[tt], 0, 0, 0);
    }
    // causal mask on the block that reaches the diagonal: key > query
    const int k0 = kb * AKB, q = q0 + ql;
    if (k0 + AKB - 1 > q0) {
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (k0 + 16 * tt + 4 * g + r > q) s[tt][r] = -__builtin_inff();
    }
    // online softmax over this block's keys for query q
    float mx = fmaxf(fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3])),
                     fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3])));
    const LanePair p16 = lane_pair16(mx);
    mx = fmaxf(p16.lo, p16.hi);
    const LanePair p32 = lane_pair32(mx);
    mx = fmaxf(p32.lo, p32.hi);
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -__builtin_inff() ? 0.0f : m_new;
    const float alpha = __builtin_amdgcn_exp2f((m_run - m_use) * kscale);
    const float bias = -m_use * kscale;
    float p[2][4];
    float psum = 0.0f;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p[tt][r] = __builtin_amdgcn_exp2f(fmaf(s[tt][r], kscale, bias));
        psum += p[tt][r];
      }
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int d = 0; d < NDT; ++d) o[d] *= alpha;
    Frag16 pf;  // P^T, k slots: keys 4g + r (tile 0), 16 + 4g + r (tile 1)
    pf.u = u32x4{cvt_pk_bf16(p[0][0], p[0][1]), cvt_pk_bf16(p[0][2], p[0][3]),
                 cvt_pk_bf16(p[1][0], p[1][1]), cvt_pk_bf16(p[1][2], p[1][3])};
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
    for (int d = 0; d < NDT; ++d) {
      const Frag16 vf = read_vfrag<VLD>(vs, d, lane);
      o[d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf.h, pf.h, o[d], 0, 0, 0);
    }
    buf ^= 1;
  }
  // this wave's state: l summed over its four lane groups
  {
    const LanePair a16 = lane_pair16(l_run);
    const float l16 = a16.lo + a16.hi;
    const LanePair a32 = lane_pair32(l16);
    l_run = a32.lo + a32.hi;
  }
  if (g == 0) {
    st_m[wave][ql] = m_run;
    st_l[wave][ql] = l_run;
  }
#pragma unroll
  for (int d = 0; d < NDT; ++d)
#pragma unroll
    for (int r = 0; r < 4; ++r) st_o[wave][16 * d + 4 * g + r][ql] = o[d][r];
  __syncthreads();
  // merge: thread -> query tid / 16, dh 64 pass + 4 (tid % 16) .. +3
#pragma unroll
  for (int pass = 0; pass < DH / 64; ++pass) {
    const int qq = tid >> 4, d0 = 64 * pass + 4 * (tid & 15);
    float mw[AWAVES], mmax = -__builtin_inff();
#pragma unroll
    for (int w = 0; w < AWAVES; ++w) {
      mw[w] = st_m[w][qq];
      mmax = fmaxf(mmax, mw[w]);
    }
    float L = 0.0f, f[AWAVES];
#pragma unroll
    for (int w = 0; w < AWAVES; ++w) {
      f[w] = mw[w] == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f((mw[w] - mmax) * kscale);
      L += st_l[w][qq] * f[w];
    }
    const float invL = 1.0f / L;
    float out[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float acc = 0.0f;
#pragma unroll
      for (int w = 0; w < AWAVES; ++w) acc += st_o[w][d0 + e][qq] * f[w];
      out[e] = acc * invL;
    }
    if (q0 + qq < S)
      *reinterpret_cast<uint2 *>(O + (size_t)(q0 + qq) * D + h * DH + d0) =
          pack4_bf16(out[0], out[1], out[2], out[3]);
  }
}

// ---- launch plans ---------------------------------------------------------------
// Per-tile work of a GEMM launch, from the kernel's own loops.
template <class Sh, class Kern>
void plan_gemm(const char *name, Kern kern, const LlamaGemmArgs &a, int grid, int pro, int epi) {
  // A tile is one workgroup of 16 waves, planned as four 4-wave units side
  // by side (one wave per SIMD each).  Vector instructions per wave, counted
  // in the compiled code (gfx950 assembly, the path the layer's shapes take):
  // a straight-line part -- the loads' addresses, the RMSNorm of the A panel,
  // the chunk commits, the epilogue (RoPE, residual, SwiGLU) and the stores
  // -- plus a few per MFMA of the K loop (fragment addresses, loop control).
  // RMSNorm + QKV + RoPE: 440 + 2 per MFMA; RMSNorm + SwiGLU: 406 + 2 per
  // MFMA; residual GEMMs: 112 + 5 per MFMA with K in one chunk, 164 + 4.5
  // with several (the assembly's path counts 161 and 210 there; the
  // SQ_INSTS_VALU figures, 20 % lower, are used).  The wider-K instances
  // (K > 512 for the RMSNorm GEMMs) reuse these figures.
  const double BM = Sh::kBM, BN = Sh::kBN, units = 4.0;
  const double ksteps = a.K / 32.0;
  npu_launch_plan p = make_plan(name, grid * 4, wg_per_cu(kern, GT), grid * 4, 16);
  p.load_phases = a.K > (int)Sh::SB / 32 ? 2 : 1;  // one exposed load round trip per chunk beyond one
  p.tile_macs = BM * BN * Sh::NB * a.K / units;
  const double bpieces = a.K * BN * Sh::NB / 8.0, apieces = BM * a.K / 8.0;
  const double mfma_per_wave = p.tile_macs / 4.0 / (16.0 * 16.0 * 32.0);
  double base, per_mfma;
  if (pro == kProRmsnorm) {
    base = epi == kEpiQkvRope ? 440.0 : 406.0;
    per_mfma = 2.0;
  } else {
    base = Sh::NBUF > 1 ? 164.0 : 112.0;
    per_mfma = Sh::NBUF > 1 ? 4.5 : 5.0;
  }
  p.tile_valu = 4.0 * (base + per_mfma * mfma_per_wave);
  p.tile_lds_bytes = (2.0 * (bpieces + apieces) * 16 +
                      ksteps * 4.0 / Sh::kWK * (Sh::TNW * Sh::NB * 1024.0 * 4 / Sh::kWC + Sh::TMW * 1024.0 * 4) +
                      2.0 * Sh::RED) / units;
  p.tile_load_bytes = ((bpieces + apieces) * 16 + (pro == kProRmsnorm ? 4.0 * a.K : 0.0)) / units;
  p.tile_store_bytes = BM * BN * 2 / units;
  const double parts = epi == kEpiQkvRope ? a.nparts : (epi == kEpiSwiglu ? 2 : 1);
  p.hbm_bytes = 2.0 * ((double)a.M * a.K + parts * a.K * a.Npart +
                       (double)a.M * a.Npart * (epi == kEpiQkvRope ? a.nparts : 1) +
                       (epi == kEpiResidual ? (double)a.M * a.Npart : 0.0)) +
                (pro == kProRmsnorm ? 4.0 * a.K : 0.0) + (epi == kEpiQkvRope ? 2.0 * 4 * a.M * a.Dh / 2 : 0.0);
  plans_add(p);
}

template <int PRO, int EPI, int BM, int BN, int WR, int WC, int WK, int KC, int NCH, int KMAX = 512>
hipError_t run_gemm(const char *name, const LlamaGemmArgs &a, hipStream_t s) {
  using Sh = GemmShape<PRO, EPI, BM, BN, WR, WC, WK, KC, NCH, KMAX>;
  auto kern = llama_gemm_kernel<PRO, EPI, BM, BN, WR, WC, WK, KC, NCH, KMAX>;
  const int ncols = a.Npart * (EPI == kEpiQkvRope ? a.nparts : 1);
  if (ncols % BN != 0 || (PRO == kProRmsnorm && a.K > KMAX) || a.K > NCH * KC)
    return hipErrorInvalidValue;
  const int tiles_m = (a.M + BM - 1) / BM, tiles_n = ncols / BN;
  const int G = tiles_m * tiles_n, grid = (G + 7) / 8 * 8;
  const size_t lds = Sh::lds_bytes(a.K);
  if (lds > 160 * 1024) return hipErrorInvalidValue;
  // the dynamic LDS limit, raised once per device to the most a launch of
  // this kernel can ask for
  const int ok = cached_per_kernel(reinterpret_cast<const void *>(kern), [&](int) {
    return hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                               hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess
               ? 1 : 0;
  });
  if (!ok) return hipErrorInvalidValue;
  plan_gemm<Sh>(name, kern, a, G, PRO, EPI);
  const int xm = xcd_block_grid(tiles_m, tiles_n, BM, BN * Sh::NB, true);
  hipLaunchKernelGGL(kern, dim3(grid), dim3(GT), lds, s, a, tiles_m, tiles_n, xm);
  return hipGetLastError();
}

}  // namespace

// Tiles (16 waves each).  At d_model <= 512 the RMSNorm GEMMs give each wave
// one 16 x 16 block (per weight) over all of K, no K split: QKV 64 x 64 (192
// workgroups at the layer's 512 x 1536, K in one chunk), SwiGLU 64 x 64 per
// weight (176 workgroups, K in chunks of 128); beyond, K split four ways
// (QKV 64 x 48, SwiGLU 32 x 64, chunks of 128, K <= 1024: the whole A panel
// is in LDS).  Residual GEMMs 32 x 32 with K split four ways (256
// workgroups; K in chunks of 512, the down projection's 1408 in three, at
// most 2048).  Chunk sizes keep two chunk buffers within the 160 KiB of LDS.
hipError_t launch_llama_gemm(const LlamaGemmArgs &a, int pro, int epi, hipStream_t s) {
  if (pro == kProRmsnorm && epi == kEpiQkvRope) {
    if (a.K <= 512)
      return run_gemm<kProRmsnorm, kEpiQkvRope, 64, 64, 4, 4, 1, 512, 1, 512>("llama_rmsnorm_qkv_rope", a, s);
    return run_gemm<kProRmsnorm, kEpiQkvRope, 64, 48, 4, 1, 4, 128, 8, 1024>("llama_rmsnorm_qkv_rope", a, s);
  }
  if (pro == kProRmsnorm && epi == kEpiSwiglu) {
    if (a.K <= 512)
      return run_gemm<kProRmsnorm, kEpiSwiglu, 64, 64, 4, 4, 1, 128, 4, 512>("llama_rmsnorm_swiglu", a, s);
    return run_gemm<kProRmsnorm, kEpiSwiglu, 32, 64, 2, 2, 4, 128, 8, 1024>("llama_rmsnorm_swiglu", a, s);
  }
  if (pro == kProPlain && epi == kEpiResidual) {
    if (a.K <= 512)
      return run_gemm<kProPlain, kEpiResidual, 32, 32, 2, 2, 4, 512, 1>("llama_matmul_residual", a, s);
    return run_gemm<kProPlain, kEpiResidual, 32, 32, 2, 2, 4, 512, 4>("llama_matmul_residual", a, s);
  }
  return hipErrorInvalidValue;
}

template <int DH>
hipError_t launch_attention_dh(const uint16_t *Q, const uint16_t *K, const uint16_t *V,
                               uint16_t *O, int S, int H, float scale, hipStream_t s) {
  auto kern = llama_attention_kernel<DH>;
  const int G = (S + AQ - 1) / AQ * H, grid = (G + 7) / 8 * 8;
  {
    // The longest workgroup is the last query block's: ceil(S / AKB / 4)
    // key blocks per wave.  Per key block and wave: 8 MFMAs (S^T and O^T),
    // the online softmax and the next block's fetch (139 vector
    // instructions in the compiled code, 50 more on the diagonal block's
    // mask), one K and V block; 226 once (Q fetch, the merge and stores).
    const double kblocks = std::ceil(S / (double)AKB / AWAVES);
    npu_launch_plan p = make_plan("llama_causal_attention", G, wg_per_cu(kern, 256), G, 16);
    p.load_phases = 1;
    p.tile_macs = kblocks * AWAVES * 2.0 * AQ * AKB * DH;
    p.tile_valu = 4.0 * (226.0 + 139.0 * kblocks + 50.0) * (DH / 64);
    p.tile_lds_bytes = kblocks * AWAVES * (2.0 * AKB * DH * 2) + AWAVES * DH * AQ * 4 * 2;
    p.tile_load_bytes = kblocks * AWAVES * 2.0 * AKB * DH * 2 + AQ * DH * 2.0;
    p.tile_store_bytes = AQ * DH * 2.0;
    p.hbm_bytes = 4.0 * S * H * DH * 2;  // Q, K, V in, O out
    plans_add(p);
  }
  hipLaunchKernelGGL(kern, dim3(grid), dim3(256), 0, s, Q, K, V, O, S, H, scale);
  return hipGetLastError();
}

hipError_t launch_llama_attention(const uint16_t *Q, const uint16_t *K, const uint16_t *V,
                                  uint16_t *O, int S, int H, int dh, float scale, hipStream_t s) {
  if (dh == 64) return launch_attention_dh<64>(Q, K, V, O, S, H, scale, s);
  if (dh == 128) return launch_attention_dh<128>(Q, K, V, O, S, H, scale, s);
  return hipErrorInvalidValue;
}

}  // namespace npu
