// k_qbottleneck.hip -- int8 ResNet-50 bottleneck as ONE fused group:
//   y1  = clamp(requant(conv1x1(x, w1)), 0, 127)          [N,H,W,M1]
//   y2  = clamp(requant(conv3x3(pad(y1), w2)), 0, 127)    [N,H,W,M1]
//   out = clamp(requant(conv1x1(y2, w3)) + x, 0, 127)     [N,H,W,C]
// (the int8 restatement of test/resnet50_block.mlir:5-105; requant is TOSA
// apply_scale_32 with single rounding, per output channel).
//
// The reference cannot fuse across the tensor.pad that separates conv1 from
// conv2 (OutlineFusedGroupsPass.cpp:140-144 only unites linalg producers), so
// it would run three groups and round-trip y1 and y2 through DRAM.  Here the
// pad is folded into the halo: a tile is 7 output rows x 14 columns of one
// image, whose 9 x 16 halo is exactly nine 16-pixel MFMA blocks (one per halo
// row, lane = halo column); conv1 is recomputed on the halo and y1, y2 stay
// in LDS.  HBM sees x once (halo re-reads hit L2) and out once.
//
// The kernel is persistent: each wave loads its share of the three filters
// into registers once and the workgroup walks its tiles, prefetching the next
// tile's halo into registers while the current tile is computed.  A 56 x 56
// image is 32 such tiles, so 32 images are 1024 tiles: two per workgroup at
// two workgroups per CU, no CU carrying an extra tile.
//
// MFMA: v_mfma_i32_16x16x64_i8 with the filters as the A operand, so a lane's
// accumulator holds four consecutive output channels of one pixel.  Integer
// accumulation is exact, so any summation order gives the oracle's result bit
// for bit.
#include "kernels.hpp"
#include "npu_device.hpp"
#include "persistent.hpp"
#include "plans.hpp"

namespace npu {

namespace {

constexpr int TH = 7, TW = 14;                 // output tile
constexpr int HH = TH + 2, HW = 16;            // halo tile: HW = TW + 2 = one MFMA block
constexpr int HP = HH * HW;                    // 144 halo pixels = 9 blocks

// TOSA apply_scale_32, single rounding: (acc * m + 2^(s-1)) >> s in 64 bits,
// truncated to 32.  `rnd` is 2^(s-1), prepared once per channel.
__device__ __forceinline__ int requant(int acc, int m, long long rnd, int s) {
  return (int)(((long long)acc * (long long)m + rnd) >> s);
}
__device__ __forceinline__ int clamp_i(int v, int lo, int hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}

// Per-channel requant parameters of the four channels a lane's accumulator
// holds, read from the workgroup's LDS tables.
struct Scale4 {
  i32x4 m, s;
  long long r[4];
};
__device__ __forceinline__ Scale4 scale4(const int32_t *m, const int32_t *s, const long long *r,
                                         int c) {
  Scale4 q;
  q.m = *reinterpret_cast<const i32x4 *>(m + c);
  q.s = *reinterpret_cast<const i32x4 *>(s + c);
#pragma unroll
  for (int e = 0; e < 4; ++e) q.r[e] = r[c + e];
  return q;
}

// Requantize four accumulators (channels c..c+3 of one pixel), clamp to
// [0, 127] and pack them as four bytes, channel c in the low byte.
__device__ __forceinline__ uint32_t requant4(const i32x4 &acc, const Scale4 &q) {
  uint32_t packed = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    packed |= (uint32_t)clamp_i(requant(acc[e], q.m[e], q.r[e], q.s[e]), 0, 127) << (8 * e);
  return packed;
}

template <int C, int M1>
__global__ __launch_bounds__(256, 2) void qbottleneck_kernel(
    const int8_t *__restrict__ x, const int8_t *__restrict__ w1, const int8_t *__restrict__ w2,
    const int8_t *__restrict__ w3, const int32_t *__restrict__ m1, const int32_t *__restrict__ s1,
    const int32_t *__restrict__ m2, const int32_t *__restrict__ s2,
    const int32_t *__restrict__ m3, const int32_t *__restrict__ s3, int8_t *__restrict__ out,
    int H, int W, int tiles_w, int tiles_img, int ntiles) {
  static_assert(C % 64 == 0 && C <= 256 && M1 == 64, "C must be 64, 128 or 256 and M1 = 64");
  constexpr int XS = C + 32;    // LDS row strides: 32 mod 64 bytes keeps the 16-row
  constexpr int YS = M1 + 32;   // 16-byte operand reads free of bank conflicts
  constexpr int XCH = C / 16;   // 16-byte runs per pixel
  constexpr int NSEG = HP * XCH;
  constexpr int SEGS = (NSEG + 255) / 256;
  constexpr int FB3 = C / 64;   // conv3 filter blocks per wave
  __shared__ __attribute__((aligned(16))) int8_t xs[HP * XS];
  // conv2 reads three columns past a block's 16 lanes for lanes 14 and 15
  // (outputs that are never stored): one spare block keeps them in bounds.
  __shared__ __attribute__((aligned(16))) int8_t y1[(HP + 16) * YS];
  __shared__ __attribute__((aligned(16))) int8_t y2[TH * 16 * YS];
  // requant tables: conv1 channels 0..M1-1, conv2 M1..2M1-1, conv3 2M1..
  constexpr int NQ = 2 * M1 + C;
  __shared__ __attribute__((aligned(16))) int32_t qm[NQ], qs[NQ];
  __shared__ __attribute__((aligned(16))) long long qr[NQ];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q = lane >> 4;
  const TileWalk walk = tile_walk(ntiles);

  // Halo runs: with 256 threads and XCH 16-byte runs per pixel, thread t
  // loads run t % XCH of halo column (t / XCH) % 16 in every segment s, on
  // halo row t / (16 XCH) + s * 16 / XCH.  Runs outside the image are loaded
  // from a clamped address and zeroed when they are committed to LDS (bit s
  // of `keep`): masking at the load would make the wave wait for it there.
  constexpr int RSTEP = 16 / XCH;
  const int hx = (tid / XCH) % HW, hch = tid % XCH, hy0 = tid / (HW * XCH);
  auto halo_load = [&](int tile, u32x4 (&st)[SEGS], uint32_t &keep) {
    const int n = tile / tiles_img, tt = tile - n * tiles_img;
    const int iy0 = (tt / tiles_w) * TH - 1 + hy0, ix = (tt % tiles_w) * TW - 1 + hx;
    const bool col_in = (unsigned)ix < (unsigned)W;
    const int8_t *base = x + ((size_t)n * H * W + min(max(ix, 0), W - 1)) * C + hch * 16;
    keep = 0;
#pragma unroll
    for (int s = 0; s < SEGS; ++s) {
      const int iy = iy0 + s * RSTEP;
      keep |= (uint32_t)(col_in && (unsigned)iy < (unsigned)H) << s;
      st[s] = *reinterpret_cast<const u32x4 *>(base + (size_t)min(max(iy, 0), H - 1) * W * C);
    }
  };

  // requant tables: loads first, LDS writes after the other prologue loads
  // are issued
  int32_t tm[(NQ + 255) / 256], ts[(NQ + 255) / 256];
#pragma unroll
  for (int k = 0; k < (NQ + 255) / 256; ++k) {
    const int c = min(tid + 256 * k, NQ - 1);
    tm[k] = c < M1 ? m1[c] : c < 2 * M1 ? m2[c - M1] : m3[c - 2 * M1];
    ts[k] = c < M1 ? s1[c] : c < 2 * M1 ? s2[c - M1] : s3[c - 2 * M1];
  }

  u32x4 st[SEGS];
  uint32_t keep = 0;
  if (walk.first < walk.end) halo_load(walk.first, st, keep);

  // Filters as each MFMA's A operand: wave w owns conv1 / conv2 output
  // channels 16w..16w+15 and conv3 output blocks w, w + 4, ...
  const int f12 = wave * 16 + r;
  Frag16 b1[C / 64], b2[9], b3[FB3];
#pragma unroll
  for (int kc = 0; kc < C / 64; ++kc) b1[kc] = load16(w1 + f12 * C + kc * 64 + 16 * q);
#pragma unroll
  for (int t = 0; t < 9; ++t) b2[t] = load16(w2 + (f12 * 9 + t) * M1 + 16 * q);
#pragma unroll
  for (int j = 0; j < FB3; ++j) b3[j] = load16(w3 + ((wave + 4 * j) * 16 + r) * M1 + 16 * q);
  const int fq = wave * 16 + 4 * q;
#pragma unroll
  for (int k = 0; k < (NQ + 255) / 256; ++k) {
    const int c = tid + 256 * k;
    if (c < NQ) {
      qm[c] = tm[k];
      qs[c] = ts[k];
      qr[c] = 1LL << (ts[k] - 1);
    }
  }
#pragma unroll
  for (int kc = 0; kc < C / 64; ++kc) settle(b1[kc].u);
#pragma unroll
  for (int t = 0; t < 9; ++t) settle(b2[t].u);
#pragma unroll
  for (int j = 0; j < FB3; ++j) settle(b3[j].u);

  for (int tile = walk.first; tile < walk.end; tile += walk.step) {
    const int n = tile / tiles_img, tt = tile - n * tiles_img;
    const int ty0 = (tt / tiles_w) * TH, tx0 = (tt % tiles_w) * TW;
    // addressing recomputed per tile rather than held across the loop
    const int ti = opaque(tid);

    // ---- the halo of this tile into LDS; the next tile's loads go out
#pragma unroll
    for (int s = 0; s < SEGS; ++s) {
      const int hy = hy0 + s * RSTEP;
      if (hy < HH)
        *reinterpret_cast<u32x4 *>(xs + (hy * HW + hx) * XS + hch * 16) = masked(st[s], (keep >> s) & 1);
    }
    __syncthreads();
    if (tile + walk.step < walk.end) halo_load(tile + walk.step, st, keep);

    // ---- conv1 (1x1, C -> M1) on the 9 halo rows, requant + ReLU into y1
    //      (zero for halo pixels outside the image: the pad before conv2)
    const bool col_in = (unsigned)(tx0 - 1 + r) < (unsigned)W;
#pragma unroll
    for (int pb = 0; pb < HH; ++pb) {
      i32x4 acc = {0, 0, 0, 0};
#pragma unroll
      for (int kc = 0; kc < C / 64; ++kc)
        MfmaI8::mma(acc, b1[kc], load16(xs + (pb * 16 + r) * XS + kc * 64 + 16 * q));
      const bool inside = col_in && (unsigned)(ty0 - 1 + pb) < (unsigned)H;
      const uint32_t v = requant4(acc, scale4(qm, qs, qr, fq));
      *reinterpret_cast<uint32_t *>(y1 + (pb * 16 + r) * YS + fq) = inside ? v : 0u;
    }
    __syncthreads();

    // ---- conv2 (3x3, M1 -> M1): output row i, column r reads halo rows
    //      i..i+2, columns r..r+2
#pragma unroll
    for (int i = 0; i < TH; ++i) {
      i32x4 acc = {0, 0, 0, 0};
#pragma unroll
      for (int t = 0; t < 9; ++t)
        MfmaI8::mma(acc, b2[t], load16(y1 + ((i + t / 3) * 16 + r + t % 3) * YS + 16 * q));
      *reinterpret_cast<uint32_t *>(y2 + (i * 16 + r) * YS + fq) = requant4(acc, scale4(qm, qs, qr, M1 + fq));
    }
    __syncthreads();

    // ---- conv3 (1x1, M1 -> C), requant + residual + ReLU.  The result
    //      overwrites the residual's own slot in the halo tile (each element
    //      is read and written by the same lane); lanes 14, 15 hold no output.
#pragma unroll
    for (int j = 0; j < FB3; ++j) {
      const int f4 = (wave + 4 * j) * 16 + 4 * q;
      const Scale4 sc = scale4(qm, qs, qr, 2 * M1 + f4);
#pragma unroll
      for (int i = 0; i < TH; ++i) {
        i32x4 acc = {0, 0, 0, 0};
        MfmaI8::mma(acc, b3[j], load16(y2 + (i * 16 + r) * YS + 16 * q));
        if (r < TW) {
          uint32_t *slot = reinterpret_cast<uint32_t *>(xs + ((i + 1) * 16 + r + 1) * XS + f4);
          const uint32_t res = *slot;
          uint32_t packed = 0;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int v = requant(acc[e], sc.m[e], sc.r[e], sc.s[e]) + (int)(int8_t)(res >> (8 * e));
            packed |= (uint32_t)clamp_i(v, 0, 127) << (8 * e);
          }
          *slot = packed;
        }
      }
    }
    __syncthreads();

    // ---- coalesced 16-byte stores of the output tile, RPI rows per pass.
    //      Every thread stores unconditionally: a run past the tile or the
    //      image stores the clamped pixel's own bytes again (the same value
    //      to the same address), so the stores are straight-line code and
    //      the wait for the next halo, which was loaded before them, can
    //      leave them in flight (the vector-memory counter covers loads and
    //      stores).
    {
      constexpr int RUNS = TW * XCH, RPI = 256 / RUNS;
      const int u = min(ti % RUNS + (ti / RUNS >= RPI ? RUNS : 0), RUNS - 1);
      const int sr = min(ti / RUNS, RPI - 1);
      const int c = min(u / XCH, W - 1 - tx0), ch = u % XCH;
      const int rows = min(TH, H - ty0);
      int8_t *obase = out + ((size_t)(n * H + ty0) * W + tx0 + c) * C + ch * 16;
      const int8_t *lbase = xs + (16 + c + 1) * XS + ch * 16;
#pragma unroll
      for (int k = 0; k < (TH + RPI - 1) / RPI; ++k) {
        const int i = min(k * RPI + sr, rows - 1);
        *reinterpret_cast<u32x4 *>(obase + (size_t)i * W * C) =
            *reinterpret_cast<const u32x4 *>(lbase + i * 16 * XS);
      }
    }
    __syncthreads();
  }
}

template <int C, int M1>
hipError_t launch_qb(const QBottleneckArgs &a, hipStream_t s) {
  const int tiles_w = (a.W + TW - 1) / TW, tiles_h = (a.H + TH - 1) / TH;
  const int tiles_img = tiles_w * tiles_h, ntiles = a.N * tiles_img;
  auto kern = qbottleneck_kernel<C, M1>;
  const int full = persistent_grid(kern);
  if (full <= 0) return hipErrorInvalidValue;
  // one tile per workgroup when there are fewer tiles than resident slots
  // (rounded up to whole XCD rounds: the walk gives the spare ones nothing)
  const int grid = ntiles < full ? (ntiles + kXcds - 1) / kXcds * kXcds : full;
  {
    npu_launch_plan p = make_plan("int8_bottleneck", grid, wg_per_cu(kern), ntiles, 8);
    p.load_phases = 1;  // the halo of the next tile is fetched during this one
    p.tile_macs = (double)HP * M1 * C + (double)TH * 16 * M1 * 9 * M1 + (double)TH * 16 * C * M1;
    // per wave: 4.75 vector instructions per requantized channel value
    // (64-bit multiply-add, shift, clamp, packing), four values per lane and
    // block, over conv1's HH halo blocks, conv2's TH blocks and conv3's TH
    // blocks x C/64 filter blocks; 12 per halo run committed and per output
    // row stored (addresses)
    const double vals = 4.0 * (HH + TH + TH * C / 64);
    const int segs = (HP * C / 16 + 255) / 256;
    p.tile_valu = 4.0 * (vals * 4.75 + 12.0 * (segs + TH));
    // LDS: halo written; 1 KiB per wave and MFMA operand read (conv1 HH x
    // C/64, conv2 TH x 9 taps, conv3 TH x C/64); y1 and y2 written; the
    // residual read and overwritten; the output read for the stores; the
    // requant parameters (64 bytes per lane and scale set: conv1, conv2 and
    // one per conv3 filter block)
    p.tile_lds_bytes = HP * (double)C + 4.0 * 1024 * (HH * C / 64 + TH * 9 + TH * C / 64) +
                       (HP + TH * 16.0) * M1 + 2.0 * TH * TW * C + (double)TH * TW * C +
                       (2.0 + C / 64) * 256 * 64;
    // set-up: every workgroup loads the three filters (its waves' shares)
    // and the requant tables, and fills the tables (192 per wave)
    p.wg_setup_bytes = (double)M1 * C * 2 + 9.0 * M1 * M1 + 2.0 * 4 * (2 * M1 + C);
    p.wg_setup_valu = 4.0 * 192.0;
    p.tile_load_bytes = HP * (double)C;
    p.tile_store_bytes = (double)TH * TW * C;
    p.hbm_bytes = 2.0 * a.N * a.H * a.W * C + (double)M1 * C * 2 + 9.0 * M1 * M1 + 4.0 * 2 * (2 * M1 + C);
    plans_add(p);
  }
  hipLaunchKernelGGL(kern, dim3(grid), dim3(256), 0, s, a.x, a.w1, a.w2, a.w3, a.m1, a.s1, a.m2,
                     a.s2, a.m3, a.s3, a.out, a.H, a.W, tiles_w, tiles_img, ntiles);
  return hipGetLastError();
}

// Any C and M1 that are multiples of 64, C <= 2048 and M1 <= 512 (ResNet-50's
// later stages: 512/128, 1024/256, 2048/512), for the counts the tuned
// instances above do not cover.  Every filter block is read from L2 where it
// is used, so nothing scales the registers with the channel counts.  A
// workgroup walks 4 x 4 output tiles; per tile: the x halo (6 x 6 pixels, all
// C channels, zero outside the image) to LDS; conv1 on the halo, one unit =
// 16 output channels x 16 halo pixels, requant + ReLU clamp into y1 (zero
// outside the image: the pad before conv2); conv2, one unit = 16 channels of
// the 16 output pixels, into y2; conv3, one unit = 16 output channels, with
// requant, the residual from the halo and the clamp, stored.  The units of a
// phase are dealt round-robin over the four waves, one barrier per phase.
__global__ __launch_bounds__(256, 1) void qb_stream_kernel(
    const int8_t *__restrict__ x, const int8_t *__restrict__ w1, const int8_t *__restrict__ w2,
    const int8_t *__restrict__ w3, const int32_t *__restrict__ m1, const int32_t *__restrict__ s1,
    const int32_t *__restrict__ m2, const int32_t *__restrict__ s2,
    const int32_t *__restrict__ m3, const int32_t *__restrict__ s3, int8_t *__restrict__ out,
    int H, int W, int C, int M1, int tiles_w, int tiles_img, int ntiles) {
  constexpr int SHW = 6, SHP = 36, SHPB = 3, CMAX = 2048, MMAX = 512;
  __shared__ __attribute__((aligned(16))) int8_t xs[SHP * (CMAX + 32)];
  __shared__ __attribute__((aligned(16))) int8_t y1[SHPB * 16 * (MMAX + 32)];
  __shared__ __attribute__((aligned(16))) int8_t y2[16 * (MMAX + 32)];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int XS = C + 32, YS = M1 + 32;  // 16-byte row reads: 32 mod 64 bytes
  const int XV = C / 16;                // 16-byte runs per halo pixel
  const int py = r / 4, px = r - py * 4, hb = py * SHW + px;
  auto params = [&](const int32_t *m, const int32_t *sh, int c) {
    Scale4 sc;
    sc.m = *reinterpret_cast<const i32x4 *>(m + c);
    sc.s = *reinterpret_cast<const i32x4 *>(sh + c);
#pragma unroll
    for (int e = 0; e < 4; ++e) sc.r[e] = 1LL << (sc.s[e] - 1);
    return sc;
  };
  const TileWalk walk = tile_walk(ntiles);
  for (int t = walk.first; t < walk.end; t += walk.step) {
    const int n = t / tiles_img, tt = t - n * tiles_img;
    const int ty0 = (tt / tiles_w) * 4, tx0 = (tt - (tt / tiles_w) * tiles_w) * 4;
    for (int idx = tid; idx < SHP * XV; idx += 256) {
      const int hp = idx / XV, cv = idx - hp * XV, hy = hp / SHW, hx = hp - hy * SHW;
      const int iy = ty0 + hy - 1, ix = tx0 + hx - 1;
      const bool inside = (unsigned)iy < (unsigned)H && (unsigned)ix < (unsigned)W;
      const int8_t *src = x + ((size_t)(n * H + (inside ? iy : 0)) * W + (inside ? ix : 0)) * C + 16 * cv;
      *reinterpret_cast<u32x4 *>(xs + hp * XS + 16 * cv) = masked(*reinterpret_cast<const u32x4 *>(src), inside);
    }
    __syncthreads();
    // conv1: unit u = (filter block fb, halo block pb)
    for (int u = wave; u < (M1 / 16) * SHPB; u += 4) {
      const int fb = u / SHPB, pb = u - fb * SHPB;
      i32x4 acc = {0, 0, 0, 0};
      for (int c0 = 0; c0 < C; c0 += 64)
        MfmaI8::mma(acc, load16(w1 + (size_t)(fb * 16 + r) * C + c0 + 16 * q),
                    load16(xs + min(pb * 16 + r, SHP - 1) * XS + c0 + 16 * q));
      const int hp = pb * 16 + r, hy = hp / SHW, hx = hp - hy * SHW;
      const bool inside = hp < SHP && (unsigned)(ty0 + hy - 1) < (unsigned)H &&
                          (unsigned)(tx0 + hx - 1) < (unsigned)W;
      const uint32_t v = requant4(acc, params(m1, s1, fb * 16 + 4 * q));
      *reinterpret_cast<uint32_t *>(y1 + hp * YS + fb * 16 + 4 * q) = inside ? v : 0u;
    }
    __syncthreads();
    // conv2: unit = filter block fb on the 16 output pixels (pixel r: halo hb)
    for (int fb = wave; fb < M1 / 16; fb += 4) {
      i32x4 acc = {0, 0, 0, 0};
      for (int tap = 0; tap < 9; ++tap)
        for (int c0 = 0; c0 < M1; c0 += 64)
          MfmaI8::mma(acc, load16(w2 + ((size_t)(fb * 16 + r) * 9 + tap) * M1 + c0 + 16 * q),
                      load16(y1 + (hb + (tap / 3) * SHW + tap % 3) * YS + c0 + 16 * q));
      *reinterpret_cast<uint32_t *>(y2 + r * YS + fb * 16 + 4 * q) =
          requant4(acc, params(m2, s2, fb * 16 + 4 * q));
    }
    __syncthreads();
    // conv3 + requant + residual + clamp: unit = output channel block cb
    for (int cb = wave; cb < C / 16; cb += 4) {
      i32x4 acc = {0, 0, 0, 0};
      for (int c0 = 0; c0 < M1; c0 += 64)
        MfmaI8::mma(acc, load16(w3 + (size_t)(cb * 16 + r) * M1 + c0 + 16 * q),
                    load16(y2 + r * YS + c0 + 16 * q));
      const int c = cb * 16 + 4 * q;
      const Scale4 sc = params(m3, s3, c);
      const uint32_t res = *reinterpret_cast<const uint32_t *>(xs + (hb + SHW + 1) * XS + c);
      uint32_t packed = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int v = requant(acc[e], sc.m[e], sc.r[e], sc.s[e]) + (int)(int8_t)(res >> (8 * e));
        packed |= (uint32_t)clamp_i(v, 0, 127) << (8 * e);
      }
      if (ty0 + py < H && tx0 + px < W)
        *reinterpret_cast<uint32_t *>(out + ((size_t)(n * H + ty0 + py) * W + tx0 + px) * C + c) = packed;
    }
    __syncthreads();  // xs, y1 and y2 are the next tile's
  }
}

hipError_t launch_qb_stream(const QBottleneckArgs &a, hipStream_t s) {
  const int tiles_w = (a.W + 3) / 4, tiles_img = tiles_w * ((a.H + 3) / 4), ntiles = a.N * tiles_img;
  const int full = persistent_grid(qb_stream_kernel);
  if (full <= 0) return hipErrorInvalidValue;
  const int grid = ntiles < full ? (ntiles + kXcds - 1) / kXcds * kXcds : full;
  {
    npu_launch_plan p = make_plan("int8_bottleneck_stream", grid, wg_per_cu(qb_stream_kernel), ntiles, 8);
    p.load_phases = 4;  // the halo, then each phase's filters from L2
    p.tile_macs = 48.0 * a.M1 * a.C + 16.0 * 9 * a.M1 * a.M1 + 16.0 * a.C * a.M1;
    p.tile_valu = 4.0 * (40.0 + 30.0 * (3 * a.M1 / 16 + a.M1 / 16 + a.C / 16) / 4.0);
    p.tile_lds_bytes = 2.0 * 36 * a.C + 1024.0 * (3 * a.M1 / 16 * a.C / 64 + a.M1 / 16 * 9 * a.M1 / 64 +
                                                  a.C / 16 * a.M1 / 64);
    p.tile_load_bytes = 36.0 * a.C + 48.0 * a.M1 * a.C / 16 + 9.0 * a.M1 * a.M1 + (double)a.C * a.M1;
    p.tile_store_bytes = 16.0 * a.C;
    p.hbm_bytes = 2.0 * a.N * a.H * a.W * a.C + (double)a.M1 * a.C * 2 + 9.0 * a.M1 * a.M1 +
                  4.0 * 2 * (2 * a.M1 + a.C);
    plans_add(p);
  }
  hipLaunchKernelGGL(qb_stream_kernel, dim3(grid), dim3(256), 0, s, a.x, a.w1, a.w2, a.w3, a.m1,
                     a.s1, a.m2, a.s2, a.m3, a.s3, a.out, a.H, a.W, a.C, a.M1, tiles_w, tiles_img,
                     ntiles);
  return hipGetLastError();
}

bool qb_tuned(int C, int M1) {
  return (C == 256 && M1 == 64) || (C == 128 && M1 == 64) || (C == 64 && M1 == 64);
}

}  // namespace

bool qbottleneck_supported(int C, int M1) {
  return qb_tuned(C, M1) || (C >= 64 && C % 64 == 0 && C <= 2048 && M1 >= 64 && M1 % 64 == 0 && M1 <= 512);
}

hipError_t launch_qbottleneck_i8(const QBottleneckArgs &a, hipStream_t s) {
  if (a.C == 256 && a.M1 == 64) return launch_qb<256, 64>(a, s);
  if (a.C == 128 && a.M1 == 64) return launch_qb<128, 64>(a, s);
  if (a.C == 64 && a.M1 == 64) return launch_qb<64, 64>(a, s);
  if (!qbottleneck_supported(a.C, a.M1)) return hipErrorInvalidValue;
  return launch_qb_stream(a, s);
}

}  // namespace npu
