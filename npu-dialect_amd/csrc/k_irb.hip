// k_irb.hip -- MobileNetV2 inverted residual block as ONE fused group (f32):
//   e   = relu6(conv1x1(x, we))                 expand  C -> E   (MFMA)
//   d   = relu6(depthwise3x3(pad1(e), wdw))     E channels       (VALU)
//   out = conv1x1(d, wp) + x                    project E -> C   (MFMA)
// (NHWC restatement of test/mobilenet_block.mlir:8-94, with a true depthwise
// stage where the reference models it as a full conv, :45-53).
//
// Vertical fusion with the intermediates in LDS: a workgroup computes 8x8
// output tiles one at a time (persistent: filters loaded once, the next
// tile's x halo fetched while the current one is computed), stages the 10x10
// x halo, recomputes the expand conv on the
// halo (the tensor.pad before the depthwise conv becomes zeros written for
// out-of-image halo pixels), and keeps the E-channel tile in LDS.  The
// depthwise result is computed directly in the A-operand layout of the
// project MFMA (each lane produces the 4 consecutive channels of one pixel
// that it feeds), so d never leaves registers.  HBM sees x and out once: the
// E-channel intermediates (6x the block's own bytes) never reach it.
#include <type_traits>

#include "kernels.hpp"
#include "npu_device.hpp"
#include "persistent.hpp"
#include "plans.hpp"

namespace npu {

namespace {

// Output tile TH x TW: 8 x 8 when the batch has tiles enough for every CU,
// 4 x 4 below that (more workgroups, each with a shorter serial chain; the
// expand conv is recomputed on 36 halo pixels for 16 outputs instead of 100
// for 64, which idle CUs pay for).
template <int TH, int TW>
struct IrbTile {
  static constexpr int HW = TW + 2;           // halo tile width
  static constexpr int HP = HW * (TH + 2);    // halo pixels (100 for 8 x 8)
  static constexpr int HPB = (HP + 15) / 16;  // blocks of 16 halo pixels
  static constexpr int OP = TH * TW;          // output pixels
  static constexpr int OPB = OP / 16;         // blocks of 16 output pixels
  // the depthwise/project stage: wave w takes output block w % OPB and
  // channel group w / OPB of CS (CS > 1: partial projections summed in LDS)
  static constexpr int CS = 4 / OPB;
  static_assert(OP % 16 == 0 && 4 % OPB == 0, "one to four output blocks");
};

__device__ __forceinline__ float relu6(float v) { return act_clamp(v, ActBounds{0.0f, 6.0f}); }

template <int C, int E, int TH, int TW>
__global__ __launch_bounds__(256, E >= 192 ? 1 : 2) void irb_kernel(const float *__restrict__ x,
                                                  const float *__restrict__ we,
                                                  const float *__restrict__ wdw,
                                                  const float *__restrict__ wp,
                                                  float *__restrict__ out, int H, int W,
                                                  int tiles_w, int tiles_per_image, int ntiles) {
  using Tl = IrbTile<TH, TW>;
  constexpr int HW = Tl::HW, HP = Tl::HP, HPB = Tl::HPB, OPB = Tl::OPB, CS = Tl::CS;
  static_assert(C % 4 == 0 && E % 16 == 0, "C must be a multiple of 4, E of 16");
  constexpr int KC1 = (C + 15) / 16;  // expand reduction chunks (C padded to 16)
  // LDS row strides in floats.  A stride of 32 mod 64 bytes keeps the 16-lane
  // 16-byte row reads conflict-free; the E-channel rows (read nine times per
  // pixel by the depthwise stage) always get it, the x rows only if two
  // workgroups still fit in one CU's LDS.
  constexpr int ES = E + 8;
  constexpr int XS8 = KC1 * 16 + 8;
  constexpr int XS = (HP * XS8 + HP * ES + 9 * E) * 4 <= 81920 ? XS8 : KC1 * 16 + 4;
  constexpr int FB1 = E / 16;         // expand filter blocks
  constexpr int KC2 = E / 16;         // project reduction chunks
  constexpr int FB2 = (C + 15) / 16;  // project filter blocks
  constexpr int XV = KC1 * 4;         // 16-byte columns per staged x row
  constexpr int XSEG = HP * XV;
  constexpr int XSEGS = (XSEG + 255) / 256;
  __shared__ __attribute__((aligned(16))) float xs[HP * XS];
  __shared__ __attribute__((aligned(16))) float es[HP * ES];
  __shared__ __attribute__((aligned(16))) float wds[9 * E];
  // partial projections of channel groups 1 .. CS-1 (16 pixels x FB2*16)
  __shared__ __attribute__((aligned(16))) float part[CS > 1 ? (CS - 1) * 16 * FB2 * 16 : 4];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q = lane >> 4;
  const TileWalk walk = tile_walk(ntiles);
  if (walk.first >= walk.end) return;  // uniform over the workgroup

  // x halo fetch.  Run s of a thread is halo pixel hp = (tid + 256 s) / XV,
  // 16-byte column cv; its row and column in the halo and its offset from
  // the tile origin do not depend on the tile.  Out-of-image runs (and the
  // columns past C) load the tile origin instead and are zeroed on commit.
  int xrel[XSEGS], xhyx[XSEGS];  // xhyx: halo row | halo column << 16
  uint32_t xlds[XSEGS], cbits = 0;
#pragma unroll
  for (int s = 0; s < XSEGS; ++s) {
    const int idx = min(tid + 256 * s, XSEG - 1);
    const int hp = idx / XV, c = (idx - hp * XV) * 4;
    const int hy = hp / HW, hx = hp - hy * HW;
    xhyx[s] = hy | hx << 16;
    xrel[s] = ((hy - 1) * W + hx - 1) * C + min(c, C - 4);
    xlds[s] = (uint32_t)((hp * XS + c) * 4);
    cbits |= (uint32_t)(c < C && tid + 256 * s < XSEG) << s;
  }
  u32x4 st[XSEGS];
  uint32_t inside_bits = 0;
  auto tile_origin = [&](int t, int &n, int &ty0, int &tx0) {
    n = t / tiles_per_image;
    const int tt = t - n * tiles_per_image;
    ty0 = (tt / tiles_w) * TH;
    tx0 = (tt - (tt / tiles_w) * tiles_w) * TW;
  };
  // Raw loads now, zero fill when written to LDS (a select right after a
  // load would make the wave wait for it, serialising the prefetch).
  auto fetch = [&](int t) {
    int n, ty0, tx0;
    tile_origin(t, n, ty0, tx0);
    const float *base = x + ((size_t)(n * H + ty0) * W + tx0) * C;
    inside_bits = 0;
#pragma unroll
    for (int s = 0; s < XSEGS; ++s) {
      const bool inside = ((cbits >> s) & 1u) &&
                          (unsigned)(ty0 + (xhyx[s] & 0xffff) - 1) < (unsigned)H &&
                          (unsigned)(tx0 + (xhyx[s] >> 16) - 1) < (unsigned)W;
      st[s] = *reinterpret_cast<const u32x4 *>(base + (inside ? xrel[s] : 0));
      inside_bits |= (uint32_t)inside << s;
    }
  };
  char *const xsb = reinterpret_cast<char *>(xs);
  auto commit = [&]() {
#pragma unroll
    for (int s = 0; s < XSEGS; ++s)
      if (s + 1 < XSEGS || tid + 256 * s < XSEG)
        *reinterpret_cast<u32x4 *>(xsb + xlds[s]) = masked(st[s], (inside_bits >> s) & 1u);
  };

  // ---- once per workgroup: the first halo, every expand and project filter
  //      fragment (registers), the depthwise taps (LDS).
  fetch(walk.first);
  // Expand units (filter block fb, pixel block pb), filter-block major, are
  // split evenly over the four waves; a wave's units span at most NBW
  // consecutive filter blocks, whose fragments it keeps (A operand: filter
  // fb*16 + r, input channels kc*16 + 4q .. +3).
  constexpr int NU = FB1 * HPB;
  constexpr int NBW = (NU / 4 + 1 + HPB - 1) / HPB + 1;
  const int fb_lo = wave * NU / 4 / HPB;
  Frag16 be[NBW][KC1];
#pragma unroll
  for (int j = 0; j < NBW; ++j)
#pragma unroll
    for (int kc = 0; kc < KC1; ++kc) {
      const int k = kc * 16 + 4 * q;
      Frag16 b = load16(we + (min(fb_lo + j, FB1 - 1) * 16 + r) * C + min(k, C - 4));
      b.u = masked(b.u, k < C);
      be[j][kc] = b;
    }
  // Per-lane constants of the depthwise/project stage: wave w owns output
  // pixels 16 ob .. 16 ob + 15 (ob = w % OPB) and the expanded channels of
  // its channel group cg = w / OPB: 16-channel chunks [kc0, kc1) of KC2, at
  // most KCW; this lane's pixel p = 16 ob + r.
  const int ob = wave % OPB, cg = wave / OPB;
  constexpr int KCW = (KC2 + CS - 1) / CS;
  const int kc0 = CS == 1 ? 0 : cg * KC2 / CS, kc1 = CS == 1 ? KC2 : (cg + 1) * KC2 / CS;
  // project A operand of the wave's channel group: output channel fb*16 + r,
  // expanded channels kc*16 + 4q .. +3 (kc = kc0 + j)
  Frag16 bp[KCW][FB2];
#pragma unroll
  for (int j = 0; j < KCW; ++j)
#pragma unroll
    for (int fb = 0; fb < FB2; ++fb) {
      const int c = fb * 16 + r, kc = min(kc0 + j, KC2 - 1);
      Frag16 b = load16(wp + min(c, C - 1) * E + kc * 16 + 4 * q);
      b.u = masked(b.u, c < C);
      bp[j][fb] = b;
    }
  for (int i = tid; i < 9 * E / 4; i += 256)
    reinterpret_cast<f32x4 *>(wds)[i] = reinterpret_cast<const f32x4 *>(wdw)[i];
  commit();
#pragma unroll
  for (int j = 0; j < NBW; ++j)
#pragma unroll
    for (int kc = 0; kc < KC1; ++kc) settle(be[j][kc].u);
#pragma unroll
  for (int j = 0; j < KCW; ++j)
#pragma unroll
    for (int fb = 0; fb < FB2; ++fb) settle(bp[j][fb].u);
  __syncthreads();

  const int p = ob * 16 + r, py = p / TW, px = p - py * TW;
  const int hbase = py * HW + px;
  const uint32_t ooff = (uint32_t)(((py * W + px) * C + 4 * q) * 4);

  // Pipeline: the halo of tile t+step is in registers while tile t is
  // computed; once every wave is done with xs it goes to LDS and the fetch
  // of tile t+2*step is issued.  Fetch and commit are unconditional (past the
  // end the walk refetches a tile whose copy is never read): with a
  // condition on either, the compiler's wait analysis assumes a fetch can be
  // pending at the loop head and drains every outstanding load there.
  auto next_of = [&](int t) { return t + walk.step < walk.end ? t + walk.step : t; };
  fetch(next_of(walk.first));
  for (int t = walk.first; t < walk.end; t += walk.step) {
    int n, ty0, tx0;
    tile_origin(t, n, ty0, tx0);

    // ---- expand on the halo.  The filters are the A operand and the
    //      pixels the B operand: a lane's accumulator holds filters 4q..4q+3
    //      of the block for pixel pb*16 + r, written to LDS as one 16-byte
    //      store (zero for halo pixels outside the image: the tensor.pad
    //      before the depthwise).  The pixel blocks of one filter block are
    //      independent accumulators, interleaved step by step.
    auto expand = [&](auto wv) {
      constexpr int U0 = decltype(wv)::value * NU / 4, U1 = (decltype(wv)::value + 1) * NU / 4;
      constexpr int FLO = U0 / HPB;
      static_assert((U1 - 1) / HPB - FLO < NBW, "a wave's filter blocks fit its fragments");
#pragma unroll
      for (int fb = U0 / HPB; fb <= (U1 - 1) / HPB; ++fb) {
        const int p0 = max(U0 - fb * HPB, 0), p1 = min(U1 - fb * HPB, HPB);
        f32x4 acc[HPB];
#pragma unroll
        for (int pb = p0; pb < p1; ++pb) acc[pb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kc = 0; kc < KC1; ++kc) {
          Frag16 bx[HPB];
#pragma unroll
          for (int pb = p0; pb < p1; ++pb)
            bx[pb] = load16(xs + min(pb * 16 + r, HP - 1) * XS + kc * 16 + 4 * q);
#pragma unroll
          for (int s2 = 0; s2 < 4; ++s2)
#pragma unroll
            for (int pb = p0; pb < p1; ++pb) MfmaF32::step(acc[pb], be[fb - FLO][kc], bx[pb], s2);
        }
#pragma unroll
        for (int pb = p0; pb < p1; ++pb) {
          const int hp = pb * 16 + r, hy = hp / HW, hx = hp - hy * HW;
          const bool inside = (unsigned)(ty0 + hy - 1) < (unsigned)H &&
                              (unsigned)(tx0 + hx - 1) < (unsigned)W;
          if (pb * 16 + 15 < HP || hp < HP) {
            f32x4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = inside ? relu6(acc[pb][e]) : 0.0f;
            *reinterpret_cast<f32x4 *>(es + hp * ES + fb * 16 + 4 * q) = v;
          }
        }
      }
    };
    switch (wave) {
      case 0: expand(std::integral_constant<int, 0>{}); break;
      case 1: expand(std::integral_constant<int, 1>{}); break;
      case 2: expand(std::integral_constant<int, 2>{}); break;
      default: expand(std::integral_constant<int, 3>{}); break;
    }
    __syncthreads();

    // ---- depthwise (in registers) + project + residual.  The depthwise
    //      result of a lane is channels kc*16 + 4q .. +3 of its pixel: the B
    //      operand of the project MFMA (the project filters are A), so the
    //      accumulator holds output channels fb*16 + 4q .. +3 of the pixel.
    f32x4 acc2[FB2];
#pragma unroll
    for (int fb = 0; fb < FB2; ++fb) acc2[fb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KCW; ++j) {
      const int kc = kc0 + j;
      if (CS > 1 && kc >= kc1) break;  // a group of KCW - 1 chunks
      const int e0 = kc * 16 + 4 * q;
      f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int tap = 0; tap < 9; ++tap) {
        const f32x4 ev =
            *reinterpret_cast<const f32x4 *>(es + (hbase + (tap / 3) * HW + (tap % 3)) * ES + e0);
        const f32x4 wv = *reinterpret_cast<const f32x4 *>(wds + tap * E + e0);
        d += ev * wv;
      }
      Frag16 a;
      a.f = f32x4{relu6(d[0]), relu6(d[1]), relu6(d[2]), relu6(d[3])};
#pragma unroll
      for (int fb = 0; fb < FB2; ++fb) MfmaF32::mma(acc2[fb], bp[j][fb], a);
    }
    // residual added while x is still in LDS; the stores go out after the
    // next halo is committed and the one after it is fetched, so they are
    // the newest memory operations when the loop comes round.  With channel
    // groups, groups 1.. leave their partial projections in LDS and group 0
    // adds them, in group order, after the barrier.
    if (CS > 1 && cg > 0) {
#pragma unroll
      for (int fb = 0; fb < FB2; ++fb)
        *reinterpret_cast<f32x4 *>(part + ((cg - 1) * 16 + r) * FB2 * 16 + fb * 16 + 4 * q) = acc2[fb];
    } else {
#pragma unroll
      for (int fb = 0; fb < FB2; ++fb)
        acc2[fb] += *reinterpret_cast<const f32x4 *>(xs + (hbase + HW + 1) * XS + fb * 16 + 4 * q);
    }
    __syncthreads();  // every wave is done with xs and es of this tile
    if (CS > 1 && cg == 0) {
#pragma unroll
      for (int g2 = 1; g2 < CS; ++g2)
#pragma unroll
        for (int fb = 0; fb < FB2; ++fb)
          acc2[fb] += *reinterpret_cast<const f32x4 *>(part + ((g2 - 1) * 16 + r) * FB2 * 16 + fb * 16 + 4 * q);
    }
    commit();
    fetch(next_of(next_of(t)));
    if ((CS == 1 || cg == 0) && ty0 + py < H && tx0 + px < W) {
      char *ob = reinterpret_cast<char *>(out) + ((size_t)(n * H + ty0) * W + tx0) * C * 4;
#pragma unroll
      for (int fb = 0; fb < FB2; ++fb)
        if (fb * 16 + 4 * q < C)
          *reinterpret_cast<f32x4 *>(ob + ooff + fb * 64) = acc2[fb];
    }
    __syncthreads();
  }
}

template <int C, int E, int TH, int TW>
hipError_t launch_irb_tile(const IrbArgs &a, hipStream_t s) {
  using Tl = IrbTile<TH, TW>;
  constexpr int HP = Tl::HP, HPB = Tl::HPB, OP = Tl::OP;
  auto kern = irb_kernel<C, E, TH, TW>;
  const int tiles_w = (a.W + TW - 1) / TW, tiles_h = (a.H + TH - 1) / TH;
  const int per_image = tiles_w * tiles_h, ntiles = a.N * per_image;
  const int full = persistent_grid(kern);
  if (full == 0) return hipErrorInvalidDeviceFunction;
  // one tile per workgroup when there are fewer tiles than resident slots
  // (rounded up to whole XCD rounds: the walk gives the spare ones nothing)
  const int g = ntiles < full ? (ntiles + kXcds - 1) / kXcds * kXcds : full;
  {
    constexpr int KC1 = (C + 15) / 16, FB2 = (C + 15) / 16, FB1 = E / 16;
    npu_launch_plan p = make_plan("mbv2_inverted_residual", g, wg_per_cu(kern), ntiles, 32);
    p.load_phases = 0;  // the next tile's halo is fetched during this tile
    p.tile_macs = (double)E * HPB * 16 * KC1 * 16 + (double)OP * FB2 * 16 * E;
    // Vector instructions per wave and tile, counted in the compiled code
    // (gfx950 assembly, <24, 144, 8, 8>): 81 for the tile (halo commit and
    // fetch addresses, residual, stores, loop control); 13.4 per expand unit
    // (a filter block on 16 halo pixels, FB1 * HPB / 4 per wave: ReLU6, the
    // padding select, the store address); 46 per 16 depthwise channels of a
    // block of 16 output pixels (nine taps' FMAs, ReLU6, LDS addresses),
    // OP / 16 blocks over four waves: 706 per 8 x 8 tile at E = 144.
    // Set-up: 330 (the filter staging and the first halo's addresses; 254
    // for the 4 x 4 tile's 36-pixel halo, <24, 144, 4, 4>).
    p.tile_valu = 4.0 * (81.0 + FB1 * HPB / 4.0 * 13.4 + 46.0 * (E / 16) * (OP / 16) / 4.0);
    p.wg_setup_valu = 4.0 * (TH == 4 ? 254.0 : 330.0);
    p.tile_lds_bytes = HP * (KC1 * 16 + 8) * 4.0 +                // halo written
                       (E / 16.0) * KC1 * HPB * 1024 +            // expand A read
                       HP * E * 4.0 +                             // expanded tile written
                       2.0 * (OP / 16) * (E / 16) * 9 * 1024 +    // depthwise taps and weights read
                       OP * C * 4.0;                              // residual
    p.tile_load_bytes = HP * C * 4.0;
    p.tile_store_bytes = OP * C * 4.0;
    p.wg_setup_bytes = 4.0 * 1024 * ((E / 64.0) * KC1 + (E / 16.0) * FB2) + 9.0 * E * 4;
    p.hbm_bytes = 4.0 * (2.0 * a.N * a.H * a.W * C + 2.0 * C * E + 9.0 * E);
    plans_add(p);
  }
  hipLaunchKernelGGL(kern, dim3(g), dim3(256), 0, s, a.x, a.we, a.wdw, a.wp, a.out,
                     a.H, a.W, tiles_w, per_image, ntiles);
  return hipGetLastError();
}

// 8 x 8 tiles when there are at least as many as CUs, else 4 x 4.
template <int C, int E>
hipError_t launch_irb_t(const IrbArgs &a, hipStream_t s) {
  const long long tiles8 = (long long)a.N * ((a.H + 7) / 8) * ((a.W + 7) / 8);
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess)
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (tiles8 < cus) return launch_irb_tile<C, E, 4, 4>(a, s);
  return launch_irb_tile<C, E, 8, 8>(a, s);
}

// Any (C, E) with C % 4 == 0, C <= 16 CB and E % 16 == 0, for the channel
// counts the tuned instances above do not cover: the expanded channels are
// streamed in chunks of 16, so neither the filters nor the expanded tile
// need to fit in registers or LDS.  A workgroup walks 4 x 4 output tiles;
// per tile the x halo (6 x 6 pixels, all C channels, zero outside the image
// and past C) goes to LDS, then wave w takes chunks w, w + 4, ... of E / 16:
// the expand of the chunk on the halo (its 16 filters as the A operand, from
// L2), ReLU6 and the zero padding into the wave's own LDS slot, the
// depthwise of the 16 output pixels in the project MFMA's B layout, and the
// project of the chunk into the wave's CB accumulator blocks (its columns of
// wp as the A operand).  Waves 1..3 leave their partial projections in LDS
// and wave 0 adds them in wave order, then the residual, and stores.
template <int CB>
__global__ __launch_bounds__(256, 1) void irb_stream_kernel(
    const float *__restrict__ x, const float *__restrict__ we, const float *__restrict__ wdw,
    const float *__restrict__ wp, float *__restrict__ out, int H, int W, int C, int E,
    int tiles_w, int tiles_per_image, int ntiles) {
  constexpr int TW = 4, HW = 6, HP = 36, HPB = 3;
  constexpr int ESS = 24;  // a wave's expanded chunk: 16 channels per pixel + 8 (32 mod 64 bytes)
  __shared__ __attribute__((aligned(16))) float xs[HP * (16 * CB + 8)];
  __shared__ __attribute__((aligned(16))) float esw[4][HPB * 16 * ESS];
  __shared__ __attribute__((aligned(16))) float part[3 * 16 * CB * 16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int KC1 = (C + 15) / 16, XV = KC1 * 4, XS = KC1 * 16 + 8;  // x row: 32 mod 64 bytes
  const int py = r / TW, px = r - py * TW, hbase = py * HW + px;
  float *const ew = esw[wave];
  const TileWalk walk = tile_walk(ntiles);
  for (int t = walk.first; t < walk.end; t += walk.step) {
    const int n = t / tiles_per_image, tt = t - n * tiles_per_image;
    const int ty0 = (tt / tiles_w) * 4, tx0 = (tt - (tt / tiles_w) * tiles_w) * TW;
    for (int idx = tid; idx < HP * XV; idx += 256) {
      const int hp = idx / XV, cv = idx - hp * XV, hy = hp / HW, hx = hp - hy * HW;
      const int iy = ty0 + hy - 1, ix = tx0 + hx - 1;
      const bool inside = (unsigned)iy < (unsigned)H && (unsigned)ix < (unsigned)W && 4 * cv < C;
      const float *src = x + ((size_t)(n * H + (inside ? iy : 0)) * W + (inside ? ix : 0)) * C +
                         (inside ? 4 * cv : 0);
      *reinterpret_cast<u32x4 *>(xs + hp * XS + 4 * cv) = masked(*reinterpret_cast<const u32x4 *>(src), inside);
    }
    __syncthreads();
    f32x4 acc2[CB];
#pragma unroll
    for (int ob = 0; ob < CB; ++ob) acc2[ob] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int k = wave; k < E / 16; k += 4) {
      const int e0 = k * 16;
      // expand: filters e0 + r (A), halo pixels pb*16 + r (B), channels kc*16 + 4q + s
      f32x4 acc[HPB];
#pragma unroll
      for (int pb = 0; pb < HPB; ++pb) acc[pb] = f32x4{0.f, 0.f, 0.f, 0.f};
      for (int kc = 0; kc < KC1; ++kc) {
        const int c = kc * 16 + 4 * q;
        Frag16 a = load16(we + (size_t)(e0 + r) * C + min(c, C - 4));
        a.u = masked(a.u, c < C);
        Frag16 bx[HPB];
#pragma unroll
        for (int pb = 0; pb < HPB; ++pb) bx[pb] = load16(xs + min(pb * 16 + r, HP - 1) * XS + c);
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2)
#pragma unroll
          for (int pb = 0; pb < HPB; ++pb) MfmaF32::step(acc[pb], a, bx[pb], s2);
      }
      // ReLU6, then the zero padding of the expanded tensor outside the image
#pragma unroll
      for (int pb = 0; pb < HPB; ++pb) {
        const int hp = pb * 16 + r, hy = hp / HW, hx = hp - hy * HW;
        const bool inside = (unsigned)(ty0 + hy - 1) < (unsigned)H && (unsigned)(tx0 + hx - 1) < (unsigned)W;
        if (hp < HP) {
          f32x4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = inside ? relu6(acc[pb][e]) : 0.0f;
          *reinterpret_cast<f32x4 *>(ew + hp * ESS + 4 * q) = v;
        }
      }
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
      // depthwise: output pixel r, channels e0 + 4q .. +3
      f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int tap = 0; tap < 9; ++tap)
        d += *reinterpret_cast<const f32x4 *>(ew + (hbase + (tap / 3) * HW + (tap % 3)) * ESS + 4 * q) *
             *reinterpret_cast<const f32x4 *>(wdw + tap * E + e0 + 4 * q);
      Frag16 bd;
      bd.f = f32x4{relu6(d[0]), relu6(d[1]), relu6(d[2]), relu6(d[3])};
      // project: output channels ob*16 + r (A: wp rows), the chunk's channels
#pragma unroll
      for (int ob = 0; ob < CB; ++ob) {
        if (ob * 16 < C) {
          const int co = ob * 16 + r;
          Frag16 a = load16(wp + (size_t)min(co, C - 1) * E + e0 + 4 * q);
          a.u = masked(a.u, co < C);
          MfmaF32::mma(acc2[ob], a, bd);
        }
      }
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    }
    if (wave > 0) {
#pragma unroll
      for (int ob = 0; ob < CB; ++ob)
        if (ob * 16 < C)
          *reinterpret_cast<f32x4 *>(part + ((wave - 1) * 16 + r) * CB * 16 + ob * 16 + 4 * q) = acc2[ob];
    }
    __syncthreads();
    if (wave == 0 && ty0 + py < H && tx0 + px < W) {
      float *o = out + ((size_t)(n * H + ty0 + py) * W + tx0 + px) * C;
#pragma unroll
      for (int ob = 0; ob < CB; ++ob) {
        const int c = ob * 16 + 4 * q;
        if (ob * 16 < C) {
          f32x4 v = acc2[ob];
#pragma unroll
          for (int w2 = 0; w2 < 3; ++w2)
            v += *reinterpret_cast<const f32x4 *>(part + (w2 * 16 + r) * CB * 16 + ob * 16 + 4 * q);
          v += *reinterpret_cast<const f32x4 *>(xs + (hbase + HW + 1) * XS + c);
          if (c < C) *reinterpret_cast<f32x4 *>(o + c) = v;
        }
      }
    }
    __syncthreads();  // xs and part are the next tile's
  }
}

template <int CB>
hipError_t launch_irb_stream(const IrbArgs &a, hipStream_t s) {
  auto kern = irb_stream_kernel<CB>;
  const int tiles_w = (a.W + 3) / 4, tiles_h = (a.H + 3) / 4;
  const int per_image = tiles_w * tiles_h, ntiles = a.N * per_image;
  const int full = persistent_grid(kern);
  if (full == 0) return hipErrorInvalidDeviceFunction;
  const int g = ntiles < full ? (ntiles + kXcds - 1) / kXcds * kXcds : full;
  {
    const int KC1 = (a.C + 15) / 16, CBr = (a.C + 15) / 16, chunks = a.E / 16;
    npu_launch_plan p = make_plan("mbv2_inverted_residual_stream", g, wg_per_cu(kern), ntiles, 32);
    p.load_phases = 1 + (chunks + 3) / 4;  // the halo, then each chunk's filters from L2
    p.tile_macs = (double)a.E * 48 * KC1 * 16 + 16.0 * CBr * 16 * a.E;
    p.tile_valu = 4.0 * (40.0 + (chunks + 3) / 4 * (30.0 + 12.0 * KC1 + 8.0 * CBr));
    p.tile_lds_bytes = 36.0 * KC1 * 16 * 4 * 2 + chunks * (48.0 * 16 * 4 * KC1 + 36.0 * 16 * 4 + 9.0 * 16 * 16 * 4) +
                       3.0 * 16 * CBr * 16 * 4 * 2;
    p.tile_load_bytes = 36.0 * a.C * 4 + chunks * 4.0 * (16.0 * a.C + 9.0 * 16 + 16.0 * a.C);
    p.tile_store_bytes = 16.0 * a.C * 4;
    p.hbm_bytes = 4.0 * (2.0 * a.N * a.H * a.W * a.C + 2.0 * a.C * a.E + 9.0 * a.E);
    plans_add(p);
  }
  hipLaunchKernelGGL(kern, dim3(g), dim3(256), 0, s, a.x, a.we, a.wdw, a.wp, a.out, a.H, a.W, a.C,
                     a.E, tiles_w, per_image, ntiles);
  return hipGetLastError();
}

bool irb_tuned(int C, int E) {
  return (C == 24 && E == 144) || (C == 16 && E == 96) || (C == 32 && E == 192);
}

}  // namespace

bool irb_supported(int C, int E) {
  return irb_tuned(C, E) || (C >= 4 && C % 4 == 0 && C <= 320 && E >= 16 && E % 16 == 0);
}

hipError_t launch_irb_f32(const IrbArgs &a, hipStream_t s) {
  if (a.C == 24 && a.E == 144) return launch_irb_t<24, 144>(a, s);
  if (a.C == 16 && a.E == 96) return launch_irb_t<16, 96>(a, s);
  if (a.C == 32 && a.E == 192) return launch_irb_t<32, 192>(a, s);
  if (!irb_supported(a.C, a.E)) return hipErrorInvalidValue;
  if (a.C <= 32) return launch_irb_stream<2>(a, s);
  if (a.C <= 64) return launch_irb_stream<4>(a, s);
  if (a.C <= 128) return launch_irb_stream<8>(a, s);
  return launch_irb_stream<20>(a, s);
}

}  // namespace npu
