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
// RoPE, residual and SiLU-gating are epilogues on the accumulators.  When K
// fits one 512-wide panel (the layer's d_model), the RMSNorm GEMMs run a
// variant that normalises the A rows it has just reduced straight into an
// LDS panel of all of K and has every B chunk in flight from the start.
//
// Attention: causal flash attention, one workgroup per (head, 64 queries),
// four key groups of four waves of 16 query rows.  Key blocks of 64 (K rows
// and V transposed) are staged once in LDS for a group's four waves, the
// next block prefetched into registers; online softmax in f32; P rounded to
// bf16 for its MFMA with V.
#include <cmath>
#include <type_traits>

#include "kernels.hpp"
#include "npu_device.hpp"
#include "plans.hpp"

namespace npu {

namespace {

constexpr int TN = 64, TK = 128;
constexpr int kNormGemmMaxK = 512;  // K of the single-panel RMSNorm GEMM
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

template <int N>
using Slot = std::integral_constant<int, N>;

// WAVES = 4: 32-row tiles; WAVES = 8: 64-row tiles (half the workgroups, each
// with twice the waves: the QKV and SwiGLU grids then fit one round of the CUs).
template <int PRO, int EPI, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void llama_gemm_kernel(const LlamaGemmArgs a) {
  constexpr int NB = (EPI == kEpiSwiglu) ? 2 : 1;
  constexpr int TM = 8 * WAVES;      // tile rows: 16 per wave pair
  constexpr int NT = 64 * WAVES;     // threads
  constexpr int RPW = TM / WAVES;    // RMSNorm rows per wave
  constexpr int KPT = 512 / NT;      // B k pairs per thread and chunk
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
  // wave (wm, wn): rows wm.. (16), columns wn.. (two 16-column tiles)
  const int wm = (wave % (WAVES / 2)) * 16, wn = (wave / (WAVES / 2)) * 32;
  const int nchunks = (a.K + TK - 1) / TK;

  // Latency, not arithmetic, bounds these small GEMMs: every dependent
  // memory round trip of a workgroup is on the critical path.  So the
  // epilogue's inputs are loaded first, the first two K chunks are in flight
  // together with the RMSNorm row loads, and the K loop keeps two chunks in
  // flight (register slots 0 and 1; chunk j lives in slot j % 2).
  //
  // staging: A chunk [TM rows][128 k] = two 8-element runs per thread;
  // B chunk [128 k][64 n] = 2 KPT k rows (KPT pairs) x one 8-column run.
  // fetch() only issues loads (raw, from clamped addresses); the zero fill,
  // the RMSNorm scaling and the B transpose happen in commit().
  // B lanes: item i = tid + NT hp is k pair i / 8 and 8-column group i % 8,
  // so eight consecutive lanes load one k row's 128 bytes (a wave loads
  // whole cache lines).  In LDS, B is [n][k] in 16-byte chunks of 8 k, chunk
  // c of column n stored at c ^ (n / 8): the transposed 4-byte writes of the
  // eight column groups then fall in eight different chunks (without it, in
  // one bank), and the MFMA reads undo the swizzle.
  const int arow = tid >> 3, akk = (tid & 7) * 8;
  const int bng = (tid & 7) * 8;  // this thread's 8-column group (the same for every hp)
  auto bkp = [&](int hp) { return 2 * ((tid + NT * hp) >> 3); };  // first k of its pair
  u32x4 sa[2][2], sb[2][NB][2 * KPT];
  f32x4 sg[2][2][2];  // gamma of this thread's two A runs (RMSNorm prologue)
  uint32_t okbits[2] = {0u, 0u};
  auto fetch = [&](auto slot, int chunk) {
    constexpr int S = decltype(slot)::value;
    const int k0 = min(chunk, nchunks - 1) * TK;
    const int row = m0 + arow;
    // K is a multiple of 64: the last chunk may hold only its first half,
    // the second half is zero-filled (and multiplies to zero).
    const int rowc = min(row, a.M - 1);
    uint32_t ok = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int kc = min(k0 + 64 * h, a.K - 64);
      sa[S][h] = load16(a.A + (size_t)rowc * a.K + kc + akk).u;
      if (PRO == kProRmsnorm) {
        sg[S][h][0] = *reinterpret_cast<const f32x4 *>(a.gamma + kc + akk);
        sg[S][h][1] = *reinterpret_cast<const f32x4 *>(a.gamma + kc + akk + 4);
      }
      ok |= (uint32_t)(row < a.M && k0 + 64 * h < a.K) << h;
    }
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int h = 0; h < 2 * KPT; ++h) {
        const int k = k0 + bkp(h >> 1) + (h & 1);
        sb[S][b][h] = load16(Bp[b] + (size_t)min(k, a.K - 1) * a.Npart + n0 + bng).u;
        ok |= (uint32_t)(k < a.K) << (2 + 4 * b + h);
      }
    okbits[S] = ok;
  };
  auto commit = [&](auto slot, int buf) {
    constexpr int S = decltype(slot)::value;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      u32x4 v = masked(sa[S][h], (okbits[S] >> h) & 1u);
      if (PRO == kProRmsnorm) {
        const float inv = inv_rms[arow];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float ylo = (bf_lo(v[j]) * inv) * sg[S][h][j >> 1][(2 * j) & 3];
          const float yhi = (bf_hi(v[j]) * inv) * sg[S][h][j >> 1][(2 * j + 1) & 3];
          v[j] = (uint32_t)f32_to_bf16(ylo) | ((uint32_t)f32_to_bf16(yhi) << 16);
        }
      }
      *reinterpret_cast<u32x4 *>(&As[buf][arow * LDA + akk + 64 * h]) = v;
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      u32x4 m[2 * KPT];
#pragma unroll
      for (int h = 0; h < 2 * KPT; ++h) m[h] = masked(sb[S][b][h], (okbits[S] >> (2 + 4 * b + h)) & 1u);
#pragma unroll
      for (int hp = 0; hp < KPT; ++hp) {
        const int kp = bkp(hp) >> 1;
        const int off = ((((kp >> 2) ^ (bng >> 3)) << 3) + 2 * (kp & 3));
#pragma unroll
        for (int j = 0; j < 8; ++j)
          *reinterpret_cast<uint32_t *>(&Bs[buf][b][(bng + j) * LDA + off]) = pair_word(m[2 * hp], m[2 * hp + 1], j);
      }
    }
  };

  // ---- epilogue inputs (cos/sin or the residual), from clamped addresses
  float ex0[2][4], ex1[2][4];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + wn + 16 * j + r;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int mc = min(m0 + wm + 4 * q + e, a.M - 1);
      ex0[j][e] = ex1[j][e] = 0.0f;
      if (EPI == kEpiQkvRope) {
        const int t = (n % a.Dh) >> 1;
        ex0[j][e] = a.cos_t[mc * (a.Dh / 2) + t];
        ex1[j][e] = a.sin_t[mc * (a.Dh / 2) + t];
      } else if (EPI == kEpiResidual) {
        ex0[j][e] = bf16_to_f32(a.res[(size_t)mc * a.Npart + n]);
      }
    }
  }
  fetch(Slot<0>{}, 0);
  fetch(Slot<1>{}, 1);

  if (PRO == kProRmsnorm) {
    // inverse RMS of the tile's rows, wave w owning rows RPW*w ..: all of a
    // wave's row loads are issued before any of them is reduced; rows past M
    // read row M-1 (their outputs are never stored).
    float s[RPW];
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) s[rr] = 0.0f;
    for (int k = lane * 8; k < a.K; k += 512) {
      u32x4 v[RPW];
#pragma unroll
      for (int rr = 0; rr < RPW; ++rr)
        v[rr] = load16(a.A + (size_t)min(m0 + wave * RPW + rr, a.M - 1) * a.K + k).u;
#pragma unroll
      for (int rr = 0; rr < RPW; ++rr) s[rr] += sumsq8(v[rr]);
    }
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) s[rr] = wave_sum(s[rr]);
    if (lane == 0) {
#pragma unroll
      for (int rr = 0; rr < RPW; ++rr)
        inv_rms[wave * RPW + rr] = 1.0f / sqrtf(s[rr] / (float)a.K + a.eps);
    }
    __syncthreads();
  }

  f32x4 acc[NB][2];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[b][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  commit(Slot<0>{}, 0);
  __syncthreads();
  // Iteration c: chunk c is in LDS buffer c % 2 and chunk c+1 in register
  // slot (c+1) % 2.  Fetch chunk c+2 into slot c % 2, multiply chunk c,
  // commit chunk c+1, barrier.  Fetch and commit are unconditional (past the
  // end they repeat the last chunk into the idle buffer, which is never
  // read): with a condition on either, the compiler's wait analysis would
  // drain every outstanding load at the loop head.  Unrolled by two so that
  // the register slots are compile-time.
  // B fragment of column n, k chunk 4 ks + q: stored at chunk (4 ks + q) ^ (n / 8)
  int bcol[2], bhi[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = wn + 16 * j + r, g = n >> 3;
    bcol[j] = n * LDA + ((q ^ g) & 3) * 8;
    bhi[j] = g & 4;
  }
  auto iteration = [&](auto slot, int c) {
    constexpr int S = decltype(slot)::value;  // = c % 2
    fetch(slot, c + 2);
    if (c < nchunks) {
#pragma unroll
      for (int ks = 0; ks < TK / 32; ++ks) {
        const Frag16 af = load16(&As[S][(wm + r) * LDA + 32 * ks + 8 * q]);
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const Frag16 bf = load16(&Bs[S][b][bcol[j] + ((4 * ks) ^ bhi[j]) * 8]);
            MfmaBF16::mma(acc[b][j], af, bf);
          }
      }
    }
    commit(Slot<1 - S>{}, 1 - S);
    __syncthreads();
  };
  for (int c = 0; c < nchunks; c += 2) {
    iteration(Slot<0>{}, c);
    iteration(Slot<1>{}, c + 1);
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
        // RoPE pairs (2t, 2t+1) sit in adjacent lanes (columns r, r^1); the
        // V part (part 2) is not rotated.
        const float partner = dpp_mov<0xb1>(v);  // lane ^ 1
        const float c = ex0[j][e], s = ex1[j][e];
        const float rot = (n & 1) ? (partner * s + v * c) : (v * c - partner * s);
        y = part < 2 ? rot : v;
      } else if (EPI == kEpiResidual) {
        y = ex0[j][e] + v;
      } else {
        y = silu(v) * acc[NB - 1][j][e];
      }
      if (m < a.M) a.out[part][(size_t)m * a.Npart + n] = f32_to_bf16(y);
    }
  }
}

// The RMSNorm GEMMs when K fits one panel (K <= 512, the layer's d_model):
// the loads that feed the RMSNorm are the whole A operand, so each wave
// normalises its own eight rows in registers right after reducing them
// (no second fetch of A, no barrier for the row statistics) and writes them
// into an LDS panel of all of K; every B chunk is in flight from the start
// (registers), and the K loop only moves B chunks into the double-buffered
// LDS tile and multiplies.  Eight waves, 64-row x 64-column tiles as the
// general kernel's eight-wave variant, the same B layout and epilogues.
template <int EPI>
__global__ __launch_bounds__(512) void llama_norm_gemm_kernel(const LlamaGemmArgs a) {
  constexpr int NB = (EPI == kEpiSwiglu) ? 2 : 1;
  constexpr int TM = 64, RPW = 8;  // tile rows; rows normalised per wave
  constexpr int NCH = kNormGemmMaxK / TK;
  __shared__ __attribute__((aligned(16))) uint16_t As[NCH][TM * LDA];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][NB][TN * LDA];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int m0 = blockIdx.y * TM;
  const int tiles_per_part = a.Npart / TN;
  const int part = (EPI == kEpiQkvRope) ? blockIdx.x / tiles_per_part : 0;
  const int n0 = (blockIdx.x % tiles_per_part) * TN;
  const uint16_t *Bp[2] = {a.B[part], a.B[NB - 1]};
  const int wm = (wave % 4) * 16, wn = (wave / 4) * 32;
  const int nchunks = (a.K + TK - 1) / TK;

  // A rows (this wave's eight, lane's 8 k) and the gamma of those k, first
  const int kk = lane * 8, kc = min(kk, a.K - 8);
  const bool kin = kk < a.K;
  u32x4 xr[RPW];
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr)
    xr[rr] = load16(a.A + (size_t)min(m0 + wave * RPW + rr, a.M - 1) * a.K + kc).u;
  const f32x4 g0 = *reinterpret_cast<const f32x4 *>(a.gamma + kc);
  const f32x4 g1 = *reinterpret_cast<const f32x4 *>(a.gamma + kc + 4);
  // every B chunk: item k pair tid / 8, 8-column group tid % 8 (eight lanes
  // load one k row's 128 bytes)
  const int bng = (tid & 7) * 8, bk = 2 * (tid >> 3);
  u32x4 sb[NCH][NB][2];
  static_for<NCH>([&](auto cc) __attribute__((always_inline)) {
    constexpr int c = decltype(cc)::value;
    const int k0 = min(c, nchunks - 1) * TK;
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        sb[c][b][h] = load16(Bp[b] + (size_t)min(k0 + bk + h, a.K - 1) * a.Npart + n0 + bng).u;
  });
  // epilogue inputs (cos/sin), from clamped addresses
  float ex0[2][4], ex1[2][4];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + wn + 16 * j + r;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int mc = min(m0 + wm + 4 * q + e, a.M - 1);
      ex0[j][e] = ex1[j][e] = 0.0f;
      if (EPI == kEpiQkvRope) {
        const int t = (n % a.Dh) >> 1;
        ex0[j][e] = a.cos_t[mc * (a.Dh / 2) + t];
        ex1[j][e] = a.sin_t[mc * (a.Dh / 2) + t];
      }
    }
  }

  // RMSNorm of this wave's rows: xn = bf16((x * inv_rms) * gamma) into the
  // panel (zero past K)
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) {
    const float ssq = wave_sum(kin ? sumsq8(xr[rr]) : 0.0f);
    const float inv = 1.0f / sqrtf(ssq / (float)a.K + a.eps);
    u32x4 v;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x4 &gg = j < 2 ? g0 : g1;
      const float ylo = (bf_lo(xr[rr][j]) * inv) * gg[(2 * j) & 3];
      const float yhi = (bf_hi(xr[rr][j]) * inv) * gg[(2 * j + 1) & 3];
      v[j] = (uint32_t)f32_to_bf16(ylo) | ((uint32_t)f32_to_bf16(yhi) << 16);
    }
    v = masked(v, kin);
    *reinterpret_cast<u32x4 *>(&As[kk / TK][(wave * RPW + rr) * LDA + kk % TK]) = v;
  }
  // B chunk c into LDS buffer c % 2: transposed to [n][k], 16-byte k chunk
  // of column n at chunk ^ (n / 8); k past K is zero
  auto commit_b = [&](auto cc) __attribute__((always_inline)) {
    constexpr int c = decltype(cc)::value;
    const int kp = bk >> 1, off = ((((kp >> 2) ^ (bng >> 3)) << 3) + 2 * (kp & 3));
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const u32x4 m0v = masked(sb[c][b][0], c * TK + bk < a.K);
      const u32x4 m1v = masked(sb[c][b][1], c * TK + bk + 1 < a.K);
#pragma unroll
      for (int j = 0; j < 8; ++j)
        *reinterpret_cast<uint32_t *>(&Bs[c & 1][b][(bng + j) * LDA + off]) = pair_word(m0v, m1v, j);
    }
  };
  f32x4 acc[NB][2];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[b][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  int bcol[2], bhi[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = wn + 16 * j + r, g = n >> 3;
    bcol[j] = n * LDA + ((q ^ g) & 3) * 8;
    bhi[j] = g & 4;
  }
  commit_b(std::integral_constant<int, 0>{});
  __syncthreads();
  static_for<NCH>([&](auto cc) __attribute__((always_inline)) {
    constexpr int c = decltype(cc)::value;
    if (c < nchunks) {
#pragma unroll
      for (int ks = 0; ks < TK / 32; ++ks) {
        const Frag16 af = load16(&As[c][(wm + r) * LDA + 32 * ks + 8 * q]);
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const Frag16 bf = load16(&Bs[c & 1][b][bcol[j] + ((4 * ks) ^ bhi[j]) * 8]);
            MfmaBF16::mma(acc[b][j], af, bf);
          }
      }
      if constexpr (c + 1 < NCH) {
        if (c + 1 < nchunks) commit_b(std::integral_constant<int, c + 1>{});
      }
      __syncthreads();
    }
  });

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
        const float partner = dpp_mov<0xb1>(v);  // lane ^ 1
        const float c = ex0[j][e], s = ex1[j][e];
        const float rot = (n & 1) ? (partner * s + v * c) : (v * c - partner * s);
        y = part < 2 ? rot : v;
      } else {
        y = silu(v) * acc[NB - 1][j][e];
      }
      if (m < a.M) a.out[part][(size_t)m * a.Npart + n] = f32_to_bf16(y);
    }
  }
}

// Causal attention, head dimension 64.
//
// Layout.  A wave owns 16 queries.  Scores are computed transposed,
// S^T = K Q^T (the K block is the MFMA's A operand, the queries its B
// operand), so lane (r, q) holds query r's scores for keys 4q..4q+3 of each
// 16-key column block: the online-softmax row statistics of query r live in
// lanes r, r+16, r+32, r+48 (two cross-lane steps), and the probabilities
// are already in the B-operand layout of O^T = V^T P^T.  An MFMA pairs the
// k slots of its two operands by position, and any assignment of keys to
// slots gives the same sum, so lane (r, q)'s eight slots of a 32-key step
// are its own keys {4q..4q+3, 16+4q..16+4q+3}, and the V^T operand is read
// in that same key order (two 8-byte LDS reads).  P never goes through LDS.
constexpr int AQ = 64;          // queries per workgroup (4 waves x 16, per key group)
constexpr int AK = 64;          // keys per block
constexpr int LDK = 64 + 16;  // LDS row stride of K rows and V^T rows (elements): 160 bytes

// AG key groups of four waves: group g takes key blocks g, g + AG, ... for
// the same 64 queries, each group with its own staged K/V blocks; at the end
// groups 1 .. AG-1 hand their online-softmax state (max, sum, unnormalised
// output) to group 0 through LDS, which merges them in order and stores.
// Against one group this divides the longest chain of key blocks (the last
// query block's) by AG; four groups put four waves on every SIMD and fill
// the CU's 160 KiB of LDS with their double-buffered K/V stages.
constexpr int AG = 4;
__global__ __launch_bounds__(256 * AG) void llama_attention_kernel(const uint16_t *__restrict__ Q,
                                                              const uint16_t *__restrict__ K,
                                                              const uint16_t *__restrict__ V,
                                                              uint16_t *__restrict__ O, int S,
                                                              int H, float scale) {
  constexpr int DH = 64;
  constexpr float kLog2e = 1.4426950408889634f;
  __shared__ __attribute__((aligned(16))) uint16_t Ks[AG][2][AK * LDK];  // [group][buf][key][d]
  __shared__ __attribute__((aligned(16))) uint16_t Vt[AG][2][DH * LDK];  // [group][buf][d][key]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kg = wave >> 2, qw = wave & 3, gt = tid & 255;  // key group, query wave, lane in group
  const int r = lane & 15, q = lane >> 4;
  const int q0 = blockIdx.x * AQ, h = blockIdx.y;
  const int D = H * DH;
  const int i0 = q0 + qw * 16;  // this wave's first query row
  const int row = i0 + r;         // this lane's query

  // query rows past S read row S-1: their outputs are never stored
  Frag16 qb[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
    qb[ks] = load16(Q + (size_t)min(row, S - 1) * D + h * DH + 32 * ks + 8 * q);

  // staging: K block [64 keys][64 d] and V block [64 keys][64 d], each two
  // 16-byte runs per thread, eight consecutive lanes on one key row's 128
  // bytes (a wave loads whole cache lines).  Raw loads in fetch(), the zero
  // fill of keys past S in commit(), so the loads overlap the block's MFMAs.
  // K: keys kr and kr + 32, d kc..kc+7.  V: keys vk and vk + 1, d vd..vd+7,
  // written transposed (V^T rows are d) as 4-byte key pairs.
  const int kr = gt >> 3, kc = (gt & 7) * 8;
  const int vk = (gt >> 3) * 2, vd = (gt & 7) * 8;
  // V^T rows keep each 32-key half in the order the PV operand reads it:
  // keys 4q..4q+3, 16+4q..16+4q+3 at 8q..8q+7, so a lane's eight keys are one
  // 16-byte read (a key pair stays adjacent); and the 16-byte key chunk c of
  // row d is stored at c ^ (d / 8 % 8), so the eight d groups' writes of one
  // key pair fall in eight different chunks (without it, in one bank).
  const int vkpos = (vk & ~31) + ((vk & 15) >> 2) * 8 + ((vk & 31) >> 4) * 4 + (vk & 3);
  const int vkw = (((vkpos >> 3) ^ (vd >> 3)) << 3) + (vkpos & 7);  // d group vd / 8 = row / 8
  // Two register slots: a group's block j lives in slot j % 2 from its
  // fetch (two steps ahead) to its commit into LDS buffer j % 2.
  u32x4 sk[2][2], sv[2][2];
  uint32_t okbits[2] = {0u, 0u};
  auto fetch = [&](auto slot, int kb) __attribute__((always_inline)) {
    constexpr int SL = decltype(slot)::value;
    uint32_t ok = 0;
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const int key = kb + kr + 32 * s2;
      sk[SL][s2] = load16(K + (size_t)min(key, S - 1) * D + h * DH + kc).u;
      ok |= (uint32_t)(key < S) << (3 + s2);
    }
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const int vkey = kb + vk + s2;
      sv[SL][s2] = load16(V + (size_t)min(vkey, S - 1) * D + h * DH + vd).u;
      ok |= (uint32_t)(vkey < S) << (1 + s2);
    }
    okbits[SL] = ok;
  };
  auto commit = [&](auto slot, int buf) __attribute__((always_inline)) {
    constexpr int SL = decltype(slot)::value;
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
      *reinterpret_cast<u32x4 *>(&Ks[kg][buf][(kr + 32 * s2) * LDK + kc]) =
          masked(sk[SL][s2], (okbits[SL] >> (3 + s2)) & 1u);
    const u32x4 v0 = masked(sv[SL][0], (okbits[SL] >> 1) & 1u), v1 = masked(sv[SL][1], (okbits[SL] >> 2) & 1u);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      *reinterpret_cast<uint32_t *>(&Vt[kg][buf][(vd + j) * LDK + vkw]) = pair_word(v0, v1, j);
  };

  int vsw[4];  // the chunk swizzle of V^T rows 16 dt + r
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) vsw[dt] = (2 * dt + (r >> 3)) & 7;
  // online softmax state of query `row`, in the log2 domain
  float m2 = -INFINITY, l = 0.0f;
  f32x4 o[4];  // o[dt][e] = O[row][16*dt + 4q + e] (unnormalised)
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  const float sc2 = scale * kLog2e;

  const int kend = min(q0 + AQ, S);  // keys beyond the block's last query are masked for all
  const int nblocks = (kend + AK - 1) / AK;
  const int nsteps = (nblocks + AG - 1) / AG;  // each step: one block per key group
  fetch(Slot<0>{}, min(kg, nblocks - 1) * AK);
  fetch(Slot<1>{}, min(kg + AG, nblocks - 1) * AK);
  commit(Slot<0>{}, 0);
  __syncthreads();
  // fetch and commit are unconditional (past its last block a group
  // refetches the last block into its idle buffer): with a condition on
  // either, the compiler's wait analysis drains every outstanding load at the
  // loop head.  Steps go in pairs so that the register slots are
  // compile-time; a step past nsteps has no visible block (blk >= nblocks).
  auto step_fn = [&](auto slot, int step) __attribute__((always_inline)) {
    constexpr int buf = decltype(slot)::value;  // = step % 2
    const int blk = AG * step + kg;
    const int kb = blk * AK;
    fetch(slot, min(blk + 2 * AG, nblocks - 1) * AK);  // this step's slot: its block is in LDS
    if (blk < nblocks && kb <= i0 + 15) {  // some key of the block is visible to this wave (uniform)
      f32x4 s[4];         // s[ct][e]: score of key kb + 16ct + 4q + e
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        s[ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const Frag16 kf = load16(&Ks[kg][buf][(16 * ct + r) * LDK + 32 * ks + 8 * q]);
          MfmaBF16::mma(s[ct], kf, qb[ks]);
        }
      }
      // Raw scores: the scale is folded into the exponent (sc2 > 0, so the
      // maximum of the scaled scores is the scaled maximum).  Keys past a
      // query or past S are masked only in a block that reaches either
      // (wave-uniform test).
      float mx = -INFINITY;
      if (kb + AK - 1 > i0 || kb + AK > S) {
#pragma unroll
        for (int ct = 0; ct < 4; ++ct)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int key = kb + 16 * ct + 4 * q + e;
            const float v = (key <= row && key < S) ? s[ct][e] : -INFINITY;
            s[ct][e] = v;
            mx = fmaxf(mx, v);
          }
      } else {
#pragma unroll
        for (int ct = 0; ct < 4; ++ct)
#pragma unroll
          for (int e = 0; e < 4; ++e) mx = fmaxf(mx, s[ct][e]);
      }
      // over the four lanes of query r (r, r+16, r+32, r+48)
      LanePair pr = lane_pair16(mx);
      mx = fmaxf(pr.lo, pr.hi);
      pr = lane_pair32(mx);
      mx = fmaxf(pr.lo, pr.hi);
      const float mnew = fmaxf(m2, mx * sc2);
      const float corr = (mnew == -INFINITY) ? 1.0f : __builtin_amdgcn_exp2f(m2 - mnew);
      float sum = 0.0f;
#pragma unroll
      for (int ct = 0; ct < 4; ++ct)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float p = (mnew == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(fmaf(s[ct][e], sc2, -mnew));
          s[ct][e] = p;
          sum += p;
        }
      pr = lane_pair16(sum);
      sum = pr.lo + pr.hi;
      pr = lane_pair32(sum);
      sum = pr.lo + pr.hi;
      l = l * corr + sum;
      m2 = mnew;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) o[dt] *= corr;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        // B operand: P^T, slots 0-3 = keys 32ks + 4q + e, slots 4-7 = 32ks + 16 + 4q + e
        Frag16 pb;
#pragma unroll
        for (int e2 = 0; e2 < 2; ++e2) {
          pb.u[e2] = cvt_pk_bf16(s[2 * ks][2 * e2], s[2 * ks][2 * e2 + 1]);
          pb.u[2 + e2] = cvt_pk_bf16(s[2 * ks + 1][2 * e2], s[2 * ks + 1][2 * e2 + 1]);
        }
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          // A operand: V^T rows d = 16dt + r, the same keys in the same slots
          const Frag16 va = load16(&Vt[kg][buf][(16 * dt + r) * LDK + (((4 * ks + q) ^ vsw[dt]) << 3)]);
          MfmaBF16::mma(o[dt], va, pb);
        }
      }
    }
    commit(Slot<1 - buf>{}, 1 - buf);
    __syncthreads();
  };
  for (int step = 0; step < nsteps; step += 2) {
    step_fn(Slot<0>{}, step);
    step_fn(Slot<1>{}, step + 1);
  }
  // merge: the states of groups 1 .. AG-1 go through LDS (the K stage is
  // free: every wave passed the loop's last barrier) to the group-0 wave with
  // the same rows, which folds them in group order; a state that saw no key
  // has max -inf and contributes nothing
  float *xch = reinterpret_cast<float *>(&Ks[0][0][0]);  // (AG-1) groups x 4 waves x 64 lanes x 18 floats
  static_assert((AG - 1) * 4 * 64 * 18 * 4 <= AG * 2 * AK * LDK * 2, "the exchange fits the K stage");
  if (kg != 0) {
    float *st = xch + (((kg - 1) * 4 + qw) * 64 + lane) * 18;
    st[0] = m2;
    st[1] = l;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int e = 0; e < 4; ++e) st[2 + 4 * dt + e] = o[dt][e];
  }
  __syncthreads();
  if (kg != 0) return;
#pragma unroll
  for (int g = 1; g < AG; ++g) {
    const float *st = xch + (((g - 1) * 4 + qw) * 64 + lane) * 18;
    const float m1 = st[0], l1 = st[1];
    const float mm = fmaxf(m2, m1);
    const float c0 = (m2 == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m2 - mm);
    const float c1 = (m1 == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m1 - mm);
    l = l * c0 + l1 * c1;
    m2 = mm;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int e = 0; e < 4; ++e) o[dt][e] = o[dt][e] * c0 + st[2 + 4 * dt + e] * c1;
  }
  if (row < S) {
    const float inv = 1.0f / l;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const uint32_t lo = (uint32_t)f32_to_bf16(o[dt][0] * inv) |
                          ((uint32_t)f32_to_bf16(o[dt][1] * inv) << 16);
      const uint32_t hi = (uint32_t)f32_to_bf16(o[dt][2] * inv) |
                          ((uint32_t)f32_to_bf16(o[dt][3] * inv) << 16);
      *reinterpret_cast<uint2 *>(O + (size_t)row * D + h * DH + 16 * dt + 4 * q) = make_uint2(lo, hi);
    }
  }
}

}  // namespace

namespace {

// Launch plan of one GEMM variant: a TM x (NB*TN) output tile walks K in
// TK chunks (double-buffered: each chunk's loads overlap the previous
// chunk's MFMAs, so one exposed load phase plus the prologue's row loads).
template <class Kern>
void plan_gemm(const char *name, Kern kern, const LlamaGemmArgs &a, int grid, int nb, bool norm,
               int epi, int waves, bool panel = false) {
  // The plan's unit is four waves (one per SIMD), as its occupancy is: an
  // eight-wave workgroup is two units that run side by side, each with half
  // of the workgroup's tile (its rows, and half of the B chunks it shares).
  const int units = waves / 4;
  const int kchunks = (a.K + TK - 1) / TK;
  const int TM = 8 * waves;
  npu_launch_plan p = make_plan(name, grid * units, wg_per_cu(kern, 64 * waves), grid * units, 16);
  p.load_phases = norm && !panel ? 2 : 1;  // the single-panel kernel issues every load up front
  p.tile_macs = (double)TM * TN * nb * kchunks * TK / units;
  // vector instructions per wave (SQ_INSTS_VALU less SQ_INSTS_MFMA): 225 + 98
  // per chunk (residual), 862 + 160 per chunk (RMSNorm + RoPE), 736 + 260 per
  // chunk (RMSNorm + SwiGLU, two B operands); the single-panel variants
  // count 1345 and 1563 at four chunks (705 and 523 fixed)
  const double fixed = epi == kEpiResidual ? 225
                       : epi == kEpiQkvRope ? (panel ? 705 : 862)
                                            : (panel ? 523 : 736);
  const double per = epi == kEpiResidual ? 98 : (epi == kEpiQkvRope ? 160 : 260);
  p.tile_valu = 4.0 * (fixed + per * kchunks);
  p.tile_lds_bytes = 2.0 * ((double)TM + nb * TN) * kchunks * TK * 2 / units;   // written once, read once
  p.tile_load_bytes = (((double)TM + nb * TN) * kchunks * TK * 2 + (norm ? 4.0 * a.K : 0.0) +
                       (norm && !panel ? (double)TM * a.K * 2 : 0.0)) / units;  // the general kernel reads A twice
  p.tile_store_bytes = (double)TM * TN * 2 / units;
  const double parts = epi == kEpiQkvRope ? a.nparts : (epi == kEpiSwiglu ? 2 : 1);
  p.hbm_bytes = 2.0 * ((double)a.M * a.K + parts * a.K * a.Npart +
                       (double)a.M * a.Npart * (epi == kEpiQkvRope ? a.nparts : 1) +
                       (epi == kEpiResidual ? (double)a.M * a.Npart : 0.0)) +
                (norm ? 4.0 * a.K : 0.0) + (epi == kEpiQkvRope ? 2.0 * 4 * a.M * a.Dh / 2 : 0.0);
  plans_add(p);
}

}  // namespace

// The QKV and SwiGLU GEMMs (RMSNorm prologue, 384 and 352 workgroups of 32
// rows at the layer's M = 512) run 64-row tiles of eight waves so the grid
// fits one round of the 256 CUs; the residual GEMMs (128 workgroups) keep
// 32-row tiles of four waves.
hipError_t launch_llama_gemm(const LlamaGemmArgs &a, int pro, int epi, hipStream_t s) {
  const int tiles_n = (a.Npart / TN) * (epi == kEpiQkvRope ? a.nparts : 1);
  const int waves = pro == kProRmsnorm ? 8 : 4, TM = 8 * waves;
  dim3 grid(tiles_n, (a.M + TM - 1) / TM);
  const int g = grid.x * grid.y;
  const bool panel = pro == kProRmsnorm && a.K <= kNormGemmMaxK;
  if (panel && epi == kEpiQkvRope) {
    plan_gemm("llama_rmsnorm_qkv_rope", llama_norm_gemm_kernel<kEpiQkvRope>, a, g, 1, true, epi, 8, true);
    hipLaunchKernelGGL((llama_norm_gemm_kernel<kEpiQkvRope>), grid, dim3(512), 0, s, a);
  } else if (panel && epi == kEpiSwiglu) {
    plan_gemm("llama_rmsnorm_swiglu", llama_norm_gemm_kernel<kEpiSwiglu>, a, g, 2, true, epi, 8, true);
    hipLaunchKernelGGL((llama_norm_gemm_kernel<kEpiSwiglu>), grid, dim3(512), 0, s, a);
  } else if (pro == kProRmsnorm && epi == kEpiQkvRope) {
    plan_gemm("llama_rmsnorm_qkv_rope", llama_gemm_kernel<kProRmsnorm, kEpiQkvRope, 8>, a, g, 1, true, epi, 8);
    hipLaunchKernelGGL((llama_gemm_kernel<kProRmsnorm, kEpiQkvRope, 8>), grid, dim3(512), 0, s, a);
  } else if (pro == kProPlain && epi == kEpiResidual) {
    plan_gemm("llama_matmul_residual", llama_gemm_kernel<kProPlain, kEpiResidual, 4>, a, g, 1, false, epi, 4);
    hipLaunchKernelGGL((llama_gemm_kernel<kProPlain, kEpiResidual, 4>), grid, dim3(256), 0, s, a);
  } else if (pro == kProRmsnorm && epi == kEpiSwiglu) {
    plan_gemm("llama_rmsnorm_swiglu", llama_gemm_kernel<kProRmsnorm, kEpiSwiglu, 8>, a, g, 2, true, epi, 8);
    hipLaunchKernelGGL((llama_gemm_kernel<kProRmsnorm, kEpiSwiglu, 8>), grid, dim3(512), 0, s, a);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_llama_attention(const uint16_t *Q, const uint16_t *K, const uint16_t *V,
                                  uint16_t *O, int S, int H, float scale, hipStream_t s) {
  dim3 grid((S + AQ - 1) / AQ, H);
  {
    // Causal: query block b sees key blocks 0..b; every key block costs QK^T
    // and PV MFMAs, the online-softmax update, and one staged K and V^T
    // block.  A workgroup is AG key groups of four waves, planned as AG
    // 4-wave units per query block, each walking 1/AG of its key blocks.
    // With no more workgroups than CUs the launch lasts as long as its
    // longest walk, the last query block's: ceil(nqb / AG) key blocks per
    // unit (the plan's tile is the busiest CU's).
    const int nqb = grid.x;
    const double kblocks = std::ceil(nqb / (double)AG);
    npu_launch_plan p = make_plan("llama_causal_attention", AG * grid.x * grid.y,
                                  wg_per_cu(llama_attention_kernel, 256 * AG), AG * grid.x * grid.y, 16);
    p.load_phases = 1;
    p.tile_macs = kblocks * 2.0 * AQ * AK * 64;
    p.tile_valu = 4.0 * (150.0 + 335.0 * kblocks);  // per wave; counted: 551 on average at 1.125 blocks
    p.tile_lds_bytes = kblocks * (2.0 * 2 * AK * 64 * 2 + 4.0 * 2 * AK * 64 * 2);
    p.tile_load_bytes = kblocks * 2.0 * AK * 64 * 2 + AQ * 64 * 2.0;
    p.tile_store_bytes = AQ * 64 * 2.0;
    p.hbm_bytes = 4.0 * S * H * 64 * 2;  // Q, K, V in, O out
    plans_add(p);
  }
  hipLaunchKernelGGL(llama_attention_kernel, grid, dim3(256 * AG), 0, s, Q, K, V, O, S, H, scale);
  return hipGetLastError();
}

}  // namespace npu
