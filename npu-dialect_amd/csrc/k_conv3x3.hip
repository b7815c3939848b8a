// k_conv3x3.hip -- group `pad -> fill -> conv_2d_nhwc_fhwc(3x3, stride 1) ->
// generic(bias, act)` for images up to 64 pixels wide: the shape of the
// conv2d configurations (56x56x64 -> 64).
//
// A workgroup owns TR full image rows of one image and 64 (or 16) filters.
// The reduction runs over stages of NCH channel chunks (a chunk is one MFMA
// operand run: 16 f32 or 32 bf16 channels).  For each stage the zero-padded
// (TR+2) x (W+2) input halo is staged once into LDS and all nine taps read
// their A operands from it with shifted addressing, so each input element
// leaves HBM/L2 once per stage instead of once per tap.  With several stages
// the next stage's halo and filter fragments are fetched into registers
// while the current one is multiplied (double-buffered LDS, one barrier per
// stage); when one stage covers every channel (bf16, C = 64) the whole
// reduction runs after a single barrier.  Filters are read straight from L2
// as B operands (FHWC keeps each lane's channel run contiguous); the pad of
// tensor.pad is the zero fill of out-of-image halo records.
//
// Summation order is fixed (chunk by chunk, tap by tap within a chunk)
// whatever NCH is, so every variant returns the same bits.
//
// LDS record: one pixel's NCH*64 bytes of the stage plus 32 bytes of padding.
// On gfx950 a ds_read_b128 in which 16 lanes read 16 consecutive records runs
// conflict-free when the record stride is 32 mod 64 bytes (measured: 22
// cycles per wave instruction with four waves reading, against 32 for a
// stride of 16 mod 64 and 64 for an unpadded 128-byte stride).
//
// Workgroups are dispatched round-robin over the 8 XCDs, each with its own
// L2.  Consecutive block indices are remapped so that each XCD gets a
// contiguous range of row tiles: neighbouring tiles share two halo rows, and
// on one XCD the second read of those rows hits L2 instead of HBM.
#include "kernels.hpp"
#include "npu_device.hpp"
#include "persistent.hpp"
#include "plans.hpp"

namespace npu {

namespace {

template <class MM, typename T, int TR, int WF, int WMAX, int NCH, int NBUF, int WFIX>
__global__ __launch_bounds__(256) void conv3x3_rows_kernel(
    const T *__restrict__ x, const T *__restrict__ w, const float *__restrict__ bias,
    T *__restrict__ out, int H, int w_rt, int c_rt, int F, int act) {
  // a row width of WFIX (> 0) and the single stage's channel count are
  // compile-time, so the halo and output index arithmetic folds
  const int W = WFIX > 0 ? WFIX : w_rt;
  const int C = NBUF == 1 ? NCH * MM::kPerFrag : c_rt;
  constexpr int WP = 4 / WF;                  // waves along pixels
  constexpr int KPL = MM::kPerLane;           // elements of one lane's 16-byte run
  constexpr int KC = MM::kPerFrag;            // channels per chunk (64 bytes)
  constexpr int SEGP = NCH * 4;               // 16-byte segments per pixel and stage
  constexpr int REC = (NCH * 64 + 32) / sizeof(T);  // LDS record stride in elements
  constexpr int HR = TR + 2;
  constexpr int PBMAX = (TR * WMAX + 15) / 16;
  constexpr int PBW = (PBMAX + WP - 1) / WP;  // pixel blocks per wave
  constexpr int SEGS = (HR * (WMAX + 2) * SEGP + 255) / 256;
  static_assert(KC * sizeof(T) == 64, "a chunk is 64 bytes per pixel");
  static_assert(NBUF == 1 || NBUF == 2, "single or double buffered");
  // One stage (all of C): the workgroup's 16 filters (all four waves use the
  // same ones) are loaded once, coalesced, into LDS rather than by every
  // wave into registers as 16-byte pieces of 16 filter rows (on the critical
  // path of a one-tile workgroup: bf16 56x56x64 5.1 -> 3.7 us); a row
  // stride of 9 C channels plus 32 bytes (32 mod 64 bytes) keeps the 16
  // filters' fragment reads conflict-free.
  constexpr bool WLDS = NBUF == 1 && WF == 1;
  constexpr int WST = 9 * NCH * KC + 32 / sizeof(T);
  constexpr int EPR = 16 / sizeof(T);  // elements per 16-byte run
  __shared__ __attribute__((aligned(16))) T halo[NBUF][HR * (WMAX + 2) * REC];
  __shared__ __attribute__((aligned(16))) T wsm[WLDS ? 16 * WST : 4];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int tiles_h = (H + TR - 1) / TR;
  int tile = blockIdx.x;
  if (gridDim.x % kXcds == 0) tile = (tile % kXcds) * (gridDim.x / kXcds) + tile / kXcds;
  const int n = tile / tiles_h, h0 = (tile - n * tiles_h) * TR;
  const int f = (blockIdx.y * WF + (wave % WF)) * 16 + r;
  const bool fok = f < F;
  const int wp = wave / WF;
  const int HC = W + 2, nseg = HR * HC * SEGP;
  const int tile_px = TR * W;

  // Per-lane pixel rows of the A operand (pixel = pb*16 + r within the tile).
  // Rows past the tile read a valid (clamped) record: they only feed output
  // rows that are never stored, so they need no zeroing.
  int abase[PBW];
#pragma unroll
  for (int i = 0; i < PBW; ++i) {
    const int p = min((wp + i * WP) * 16 + r, tile_px - 1);
    const int pr = p / W, pc = p - pr * W;
    abase[i] = (pr * HC + pc) * REC + q * KPL;
  }

  // Halo staging: 16-byte segments, loads from clamped addresses, the zero
  // padding applied by a select.
  // The zero fill is applied when the segments are written to LDS, not when
  // they are loaded: a select on a loaded value right after the load would
  // make the wave wait for it, and the next stage's loads must stay in
  // flight while the current stage is multiplied.
  u32x4 stage[SEGS];
  uint32_t inside_bits = 0;
  auto fetch = [&](int c0) {
    inside_bits = 0;
#pragma unroll
    for (int s = 0; s < SEGS; ++s) {
      const int idx = min(tid + 256 * s, nseg - 1);
      const int rec = idx / SEGP, seg = idx % SEGP;
      const int hr = rec / HC, hc = rec - hr * HC;
      const int ih = h0 + hr - 1, iw = hc - 1;
      const bool inside = ih >= 0 && ih < H && iw >= 0 && iw < W;
      const int ihc = min(max(ih, 0), H - 1), iwc = min(max(iw, 0), W - 1);
      stage[s] = *reinterpret_cast<const u32x4 *>(
          x + ((size_t)(n * H + ihc) * W + iwc) * C + c0 + seg * (16 / sizeof(T)));
      inside_bits |= (uint32_t)inside << s;
    }
  };
  auto commit = [&](int buf) {
#pragma unroll
    for (int s = 0; s < SEGS; ++s) {
      const int idx = tid + 256 * s;
      if (idx < nseg)
        *reinterpret_cast<u32x4 *>(&halo[buf][(idx / SEGP) * REC + (idx % SEGP) * (16 / sizeof(T))]) =
            masked(stage[s], (inside_bits >> s) & 1u);
    }
  };
  // Filters past F read filter F-1: they only feed columns that are not stored.
  const T *wrow = w + (size_t)min(f, F - 1) * 9 * C + q * KPL;
  Frag16 b[NCH][9];
  auto fetch_b = [&](Frag16 (&dst)[NCH][9], int c0) {
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
      for (int t = 0; t < 9; ++t) dst[ch][t] = load16(wrow + t * C + c0 + ch * KC);
  };

  typename MM::acc_t acc[PBW];
#pragma unroll
  for (int i = 0; i < PBW; ++i) acc[i] = typename MM::acc_t{0, 0, 0, 0};

  fetch(0);
  if constexpr (WLDS) {
    // every load issued before the first LDS write (a loop that writes each
    // load's value before issuing the next would wait for every one in turn)
    constexpr int RPF = 9 * NCH * KC / EPR, NWR = 16 * RPF, NWL = (NWR + 255) / 256;
    const int f0 = blockIdx.y * 16;
    u32x4 wl[NWL];
#pragma unroll
    for (int i = 0; i < NWL; ++i) {
      const int idx = min(tid + 256 * i, NWR - 1), fl = idx / RPF, e = idx - fl * RPF;
      wl[i] = *reinterpret_cast<const u32x4 *>(w + (size_t)min(f0 + fl, F - 1) * 9 * C + EPR * e);
    }
#pragma unroll
    for (int i = 0; i < NWL; ++i) {
      const int idx = tid + 256 * i, fl = idx / RPF, e = idx - fl * RPF;
      if (idx < NWR) *reinterpret_cast<u32x4 *>(wsm + fl * WST + EPR * e) = wl[i];
    }
  } else {
    fetch_b(b, 0);
  }
  commit(0);
  __syncthreads();
  const int nstages = C / (KC * NCH);  // 1 when NBUF == 1 (checked by the launcher)
  for (int st = 0; st < nstages; ++st) {
    const bool more = NBUF == 2 && st + 1 < nstages;
    Frag16 bn[NCH][9];
    if (more) {
      fetch((st + 1) * NCH * KC);
      fetch_b(bn, (st + 1) * NCH * KC);
    }
    const T *hb = halo[NBUF == 2 ? (st & 1) : 0];
    // Two-deep pipeline over (chunk, tap): the A fragments of the next tap
    // are read from LDS while this tap's MFMAs run.  The scheduling barrier
    // keeps the compiler from hoisting every tap's reads (which would need
    // NCH*9*PBW fragments live at once).
    auto load_a = [&](Frag16 (&dst)[PBW], int j) {
      const int ch = j / 9, t = j % 9;
      const int toff = ((t / 3) * HC + (t % 3)) * REC + ch * KC;
#pragma unroll
      for (int i = 0; i < PBW; ++i) dst[i] = load16(hb + abase[i] + toff);
    };
    Frag16 a[2][PBW], bw[2];
    // filter fragment of (chunk ch, tap t) from LDS: filter r, channels ch*KC + 4q ..
    auto load_w = [&](int j) { return load16(wsm + r * WST + (j % 9) * NCH * KC + (j / 9) * KC + q * KPL); };
    load_a(a[0], 0);
    if constexpr (WLDS) bw[0] = load_w(0);
#pragma unroll
    for (int j = 0; j < NCH * 9; ++j) {
      if (j + 1 < NCH * 9) {
        load_a(a[(j + 1) & 1], j + 1);
        if constexpr (WLDS) bw[(j + 1) & 1] = load_w(j + 1);
      }
      // independent accumulators between the dependent steps of one fragment
#pragma unroll
      for (int s = 0; s < MM::kSteps; ++s)
#pragma unroll
        for (int i = 0; i < PBW; ++i) {
          if constexpr (WLDS)
            MM::step(acc[i], a[j & 1][i], bw[j & 1], s);
          else
            MM::step(acc[i], a[j & 1][i], b[j / 9][j % 9], s);
        }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (more) {
      commit((st + 1) & 1);
#pragma unroll
      for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
        for (int t = 0; t < 9; ++t) b[ch][t] = bn[ch][t];
    }
    if (NBUF == 2) __syncthreads();
  }

  if (!fok) return;
  const float bv = bias ? bias[f] : 0.0f;
  const ActBounds ab = act_bounds(act);
#pragma unroll
  for (int i = 0; i < PBW; ++i) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int p = (wp + i * WP) * 16 + 4 * q + e;
      if (p >= tile_px) continue;
      const int pr = p / W, pc = p - pr * W;
      if (h0 + pr >= H) continue;
      const float v = act_clamp(acc[i][e] + bv, ab);
      const size_t o = ((size_t)(n * H + h0 + pr) * W + pc) * F + f;
      if constexpr (sizeof(T) == 4) {
        out[o] = v;
      } else {
        out[o] = f32_to_bf16(v);
      }
    }
  }
}

// Persistent variant for reductions that fit one stage (C = NCH chunks):
// each workgroup loads its 64 filters' fragments into registers once, then
// walks a contiguous range of output rows in 2-row tiles (a 1-row tile where
// the range or an image ends), fetching the next tile's halo into registers
// while the current tile is multiplied, so loads, MFMAs and stores of
// different tiles overlap instead of every workgroup of a round waiting on
// its loads at the same time.  The ranges are balanced to within one row and
// those of one XCD are neighbours, so the halo rows two tiles share are read
// from HBM once.
//
// Per tile, only the tile's base addresses change: the rows of the halo and
// of the output are wave-uniform (scalar registers), and each lane's offset
// within a row is fixed for the whole walk.  So every global load and store
// is a scalar base plus one loop-invariant lane offset, and the LDS addresses
// are loop-invariant plus immediates: the per-tile vector-ALU work is the
// epilogue's clamp and conversion, not index arithmetic.
// Two workgroups per CU where their registers fit (two chunks, rows of up
// to 56 pixels), else one.
template <class MM, typename T, int WMAX, int NCH, int WFIX>
__global__ __launch_bounds__(256, NCH <= 2 && WMAX <= 56 ? 2 : 1) void conv3x3_stream_kernel(
    const T *__restrict__ x, const T *__restrict__ w, const float *__restrict__ bias,
    T *__restrict__ out, int H, int w_rt, int F, int act, int nrows) {
  const int W = WFIX > 0 ? WFIX : w_rt;
  constexpr int ES = sizeof(T);
  constexpr int C = NCH * MM::kPerFrag;
  constexpr int TR = 2, HR = TR + 2;
  constexpr int KPL = MM::kPerLane;
  constexpr int KC = MM::kPerFrag;
  constexpr int SEGP = C * ES / 16;                  // 16-byte runs per input pixel
  constexpr int REC = (NCH * 64 + 32) / ES;          // LDS halo record stride (elements)
  constexpr int HCMAX = WMAX + 2;
  constexpr int LPR = (HCMAX * SEGP + 255) / 256;    // loads per halo row
  constexpr int PBW = (TR * WMAX + 15) / 16;         // 16-pixel blocks of a 2-row tile
  constexpr int PB1 = (WMAX + 15) / 16;              // ... of a 1-row tile
  // Output tile staged in LDS (64 filters per pixel plus 32 bytes of
  // padding) so that it leaves in whole 16-byte runs per lane.
  constexpr int OREC = (64 * ES + 32) / ES;
  constexpr int OSEGP = 64 * ES / 16;                // 16-byte runs per output pixel
  constexpr int OPIX = 256 / OSEGP;                  // output pixels per store instruction
  constexpr int NST = (TR * WMAX + OPIX - 1) / OPIX; // store instructions per tile
  // Filter staging: a wave's 16 runs of one tap (C elements each), padded to
  // a stride of 32 mod 64 bytes so the fragment reads are conflict-free.
  constexpr int WRS = C * ES + 32;
  constexpr int FPI = 64 / SEGP;                     // filter runs per load instruction
  constexpr int NWI = 16 / FPI;                      // load instructions per tap
  static_assert(KC * ES == 64, "a chunk is 64 bytes per pixel");
  static_assert(4 * 16 * WRS <= HR * HCMAX * REC * ES, "filter staging fits the halo buffer");
  // halo rows, then one 16-byte slot per lane that takes the writes of lanes
  // with no halo record (past the row end, or a zero-padding column)
  constexpr int HALO = HR * HCMAX * REC;
  __shared__ __attribute__((aligned(16))) T halo[HALO + 64 * 16 / ES];
  __shared__ __attribute__((aligned(16))) T ostage[PBW * 16 * OREC];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q = lane >> 4;
  const RowRange range = row_range(nrows);
  const int HC = W + 2;
  const size_t row_bytes = (size_t)W * C * ES, orow_bytes = (size_t)W * F * ES;
  // rows of the tile that starts at row `g` (global over the batch)
  auto tile_rows = [&](int g) { return min(min(TR, range.end - g), H - g % H); };

  // B-operand (pixel) fragment addresses of the tile's 16-pixel blocks
  int abase[PBW];
#pragma unroll
  for (int i = 0; i < PBW; ++i) {
    const int p = min(i * 16 + r, TR * W - 1);
    const int pr = p / W, pc = p - pr * W;
    abase[i] = (pr * HC + pc) * REC + q * KPL;
  }
  // Halo fetch: load j of every halo row covers the row's 16-byte runs
  // tid + 256 j.  goff: byte offset in the input row (the column clamped
  // into the image); loff: byte address in the LDS halo, or the lane's slot
  // past the halo when the run has no record to fill (the zero-padding
  // columns are cleared once, before the walk, and never written again).
  uint32_t goff[LPR], loff[HR][LPR];
#pragma unroll
  for (int j = 0; j < LPR; ++j) {
    const int idx = tid + 256 * j, idxc = min(idx, HC * SEGP - 1);
    const int hc = idxc / SEGP, seg = idxc - hc * SEGP;
    const int iw = min(max(hc - 1, 0), W - 1);
    goff[j] = (uint32_t)(iw * C * ES + seg * 16);
    const bool rec = idx < HC * SEGP && hc >= 1 && hc <= W;
#pragma unroll
    for (int hr = 0; hr < HR; ++hr)
      loff[hr][j] = rec ? (uint32_t)((hr * HC + hc) * REC * ES + seg * 16)
                        : (uint32_t)(HALO * ES + lane * 16);
  }
  // Output stores: store s moves pixels s*OPIX + tid/OSEGP of the tile
  const int op = tid / OSEGP, osg = tid - op * OSEGP;
  const uint32_t ooff = (uint32_t)(op * F * ES + osg * 16);
  const uint32_t oloff = (uint32_t)(op * OREC * ES + osg * 16);

  // Raw loads now, zero rows chosen when written to LDS (a select right
  // after a load would make the wave wait for it, serialising the prefetch).
  u32x4 stage[HR][LPR];
  uint32_t rowok = 0;
  auto fetch = [&](int g) {
    const int n = g / H, h0 = g - n * H;
    rowok = 0;
#pragma unroll
    for (int hr = 0; hr < HR; ++hr) {
      const int ih = h0 + hr - 1;
      rowok |= (uint32_t)(ih >= 0 && ih < H) << hr;
      const char *rb = reinterpret_cast<const char *>(x) +
                       (size_t)(n * H + min(max(ih, 0), H - 1)) * row_bytes;
#pragma unroll
      for (int j = 0; j < LPR; ++j)
        stage[hr][j] = *reinterpret_cast<const u32x4 *>(rb + goff[j]);
    }
  };
  char *const hbytes = reinterpret_cast<char *>(halo);
  auto commit = [&]() {
    const u32x4 zero{0u, 0u, 0u, 0u};
#pragma unroll
    for (int hr = 0; hr < HR; ++hr) {
      if ((rowok >> hr) & 1u) {
#pragma unroll
        for (int j = 0; j < LPR; ++j) *reinterpret_cast<u32x4 *>(hbytes + loff[hr][j]) = stage[hr][j];
      } else {
#pragma unroll
        for (int j = 0; j < LPR; ++j) *reinterpret_cast<u32x4 *>(hbytes + loff[hr][j]) = zero;
      }
    }
  };

  if (range.first >= range.end) return;  // uniform over the workgroup
  fetch(range.first);
  // Filter fragments.  A fragment (filter r, 16-byte run q of a chunk) read
  // straight from global memory would touch 16 filters' 64-byte pieces per
  // instruction; instead each tap's 16 runs are loaded whole (SEGP lanes
  // per run, full cache lines) and turned into fragments through this
  // wave's slot of the halo buffer, before the first halo is written there.
  u32x4 wraw[9][NWI];
  {
    const char *wb = reinterpret_cast<const char *>(w) +
                     (size_t)(blockIdx.y * 4 + wave) * 16 * 9 * C * ES;
    const int fl = lane / SEGP, pc = lane - fl * SEGP;
#pragma unroll
    for (int t = 0; t < 9; ++t)
#pragma unroll
      for (int i = 0; i < NWI; ++i)
        wraw[t][i] = *reinterpret_cast<const u32x4 *>(
            wb + ((size_t)(fl + FPI * i) * 9 + t) * C * ES + pc * 16);
  }
  // The filters are the MFMA's A operand and the pixels its B operand, so
  // a lane's accumulator holds filters 4q..4q+3 (of its wave's 16) of one
  // pixel: the epilogue writes them to the output stage as one 8-byte (bf16)
  // or 16-byte (f32) LDS store.  The accumulators start at the bias.
  const int fq = (blockIdx.y * 4 + wave) * 16 + 4 * q;
  float bv[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) bv[e] = bias ? bias[fq + e] : 0.0f;
  const ActBounds ab = act_bounds(act);
  Frag16 b[NCH][9];
  {
    char *ws = reinterpret_cast<char *>(halo) + wave * 16 * WRS;
    const int fl = lane / SEGP, pc = lane - fl * SEGP;
#pragma unroll
    for (int t = 0; t < 9; ++t) {
#pragma unroll
      for (int i = 0; i < NWI; ++i)
        *reinterpret_cast<u32x4 *>(ws + (fl + FPI * i) * WRS + pc * 16) = wraw[t][i];
#pragma unroll
      for (int ch = 0; ch < NCH; ++ch)
        b[ch][t].u = *reinterpret_cast<const u32x4 *>(ws + r * WRS + ch * KC * ES + q * 16);
    }
  }
  __syncthreads();  // every wave's staging is read before the halo is written
  // zero-padding columns 0 and W+1 of the halo rows
  for (int i = tid; i < HR * 2 * SEGP; i += 256) {
    const int hr = i / (2 * SEGP), k = i - hr * 2 * SEGP, side = k / SEGP, seg = k - side * SEGP;
    *reinterpret_cast<u32x4 *>(hbytes + (hr * HC + side * (W + 1)) * REC * ES + seg * 16) =
        u32x4{0u, 0u, 0u, 0u};
  }
  commit();
#pragma unroll
  for (int e = 0; e < 4; ++e) settle(bv[e]);
  __syncthreads();

  // One halo buffer: the next tile's halo waits in registers until every
  // wave has finished reading the current one.
  // Pipeline: the halo of the next tile is in registers while this tile is
  // multiplied; after the epilogue it goes to LDS and the fetch of the tile
  // after it is issued before this tile's output stores, so no register that
  // feeds a pending store is a load destination (the in-order memory
  // counter would otherwise make the next fetch wait for those stores).
  // Fetch and commit are unconditional (past the end the walk refetches a
  // tile whose copy is never read): with a condition on either, the
  // compiler's wait analysis assumes a fetch can be pending at the loop head
  // and drains every outstanding load there.
  auto next_of = [&](int g) {
    const int n = g + tile_rows(g);
    return n < range.end ? n : g;
  };
  fetch(next_of(range.first));
  for (int g = range.first; g < range.end; g += tile_rows(g)) {
    const int rows = tile_rows(g);
    const T *hb = halo;
    typename MM::acc_t acc[PBW];
#pragma unroll
    for (int i = 0; i < PBW; ++i) acc[i] = typename MM::acc_t{bv[0], bv[1], bv[2], bv[3]};
    // Two-deep pipeline over taps: the next tap's B fragments are read from
    // LDS while this tap's MFMAs run; the scheduling barrier keeps each
    // tap's reads and MFMAs in their own region.  A 1-row tile multiplies
    // only its own pixel blocks.
    auto multiply = [&](auto nblk) {
      constexpr int NB = decltype(nblk)::value;
      auto load_a = [&](Frag16 (&dst)[PBW], int j) {
        const int toff = ((j % 9 / 3) * HC + (j % 3)) * REC + (j / 9) * KC;
#pragma unroll
        for (int i = 0; i < NB; ++i) dst[i] = load16(hb + abase[i] + toff);
      };
      Frag16 a[2][PBW];
      load_a(a[0], 0);
#pragma unroll
      for (int j = 0; j < NCH * 9; ++j) {
        if (j + 1 < NCH * 9) load_a(a[(j + 1) & 1], j + 1);
#pragma unroll
        for (int s = 0; s < MM::kSteps; ++s)
#pragma unroll
          for (int i = 0; i < NB; ++i) MM::step(acc[i], b[j / 9][j % 9], a[j & 1][i], s);
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    if (rows == TR)
      multiply(std::integral_constant<int, PBW>{});
    else
      multiply(std::integral_constant<int, PB1>{});
    // Every 16-pixel block is staged (the stage has room for PBW*16 pixels);
    // the stores below move only the tile's pixels.
#pragma unroll
    for (int i = 0; i < PBW; ++i) {
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = act_clamp(acc[i][e], ab);
      T *dst = ostage + (i * 16 + r) * OREC + wave * 16 + 4 * q;
      if constexpr (sizeof(T) == 4) {
        *reinterpret_cast<f32x4 *>(dst) = f32x4{v[0], v[1], v[2], v[3]};
      } else {
        const uint32_t lo = f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16);
        const uint32_t hi = f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16);
        *reinterpret_cast<uint2 *>(dst) = make_uint2(lo, hi);
      }
    }
    __syncthreads();
    commit();
    fetch(next_of(next_of(g)));
    {
      const int npx = rows * W;
      char *ob = reinterpret_cast<char *>(out) + (size_t)g * orow_bytes + blockIdx.y * 64 * ES;
      const char *ol = reinterpret_cast<const char *>(ostage) + oloff;
#pragma unroll
      for (int s = 0; s < NST; ++s)
        if (op + s * OPIX < npx)
          *reinterpret_cast<u32x4 *>(ob + (size_t)s * OPIX * F * ES + ooff) =
              *reinterpret_cast<const u32x4 *>(ol + s * OPIX * OREC * ES);
    }
    __syncthreads();
  }
}

// Output rows [first, end) of the 3x3 / pad-1 conv for 64 filters from f0,
// computed the way the sequential f32 loops compute them: the accumulator
// starts at +0, every tap row, tap column and channel in that order adds
// the rounded product of the padded input (zero outside the image) and the
// filter value as a separate f32 multiply and add, then the bias and the
// activation.  Bit-identical to those loops, so +-Inf, NaN and values the
// bf16 split cannot carry come out as they do there.  The x6 kernel runs it
// over its rows when a split value fell outside the split's domain.
template <int C>
__device__ __forceinline__ void conv3x3_exact_rows(
    const float *__restrict__ x, const float *__restrict__ w, const float *__restrict__ bias,
    float *__restrict__ out, int H, int W, int F, int act, int f0, int first, int end) {
#pragma clang fp contract(off)
  const int f = f0 + (threadIdx.x & 63);
  const float *const wf = w + (size_t)f * 9 * C;
  const ActBounds ab = act_bounds(act);
  const float b = bias ? bias[f] : 0.0f;
  for (int p = first * W + (int)(threadIdx.x >> 6); p < end * W; p += (int)(blockDim.x >> 6)) {
    const int g = p / W, ow = p - g * W;  // g = n * H + oh
    const int n = g / H, oh = g - n * H;
    float acc = 0.0f;
    for (int kh = 0; kh < 3; ++kh) {
      const int ih = oh + kh - 1;
      for (int kw = 0; kw < 3; ++kw) {
        const int iw = ow + kw - 1;
        const bool in = ih >= 0 && ih < H && iw >= 0 && iw < W;
        const float *xp = x + ((size_t)(n * H + (in ? ih : 0)) * W + (in ? iw : 0)) * C;
        const float *wp = wf + (kh * 3 + kw) * C;
#pragma unroll 4
        for (int c = 0; c < C; ++c) {
          const float a = in ? xp[c] : 0.0f;
          const float prod = a * wp[c];
          acc = acc + prod;
        }
      }
    }
    const float v = bias ? acc + b : acc;
    out[(size_t)p * F + f] = act_clamp(v, ab);
  }
}

// f32 variant of the persistent walk on the bf16 matrix pipe.  Every input
// and filter value is split into its three bf16 parts (split_parts) and each
// 32-channel run is multiplied with the six part products (mma_x6): 6 x 16
// MFMA clocks where the f32 MFMA takes 8 x 32.
//
// Eight waves, two per SIMD: with one wave per SIMD every LDS read and
// vector instruction of the wave would stall its own MFMAs; with two, one
// wave's reads and splits issue while the other's MFMAs run.  Waves w and
// w + 4 share filter group w & 3 (16 of the workgroup's 64 filters) and
// split the rest of the work: with 64 channels, wave half c takes channel
// run c and the two partial sums meet in LDS; with 32 channels, it takes the
// 16-pixel blocks c, c + 2, ... of the tile.  A wave's filter fragments
// (nine taps, three parts, its run) stay in registers for the whole walk.
//
// The halo is a ring of NSLOT row slots in LDS (a slot: W + 2 records of a
// pixel's three parts, C bf16 each, then 32 bytes of padding, a record
// stride of 32 mod 64 bytes).  A tile of TR rows reads TR + 2 slots; the
// next tile of the same image shares two of them and needs TR new rows,
// which are fetched into registers a tile ahead, split during this tile's
// multiply and written straight into the TR slots this tile does not read.
// So each input row is fetched and split once per workgroup, plus the two
// rows a range or image starts with.  A tile that starts an image has all
// of its rows written after the previous tile has finished.  Outputs leave
// straight from the accumulators: a lane holds filters 4q..4q+3 of pixel r
// of a 16-pixel block, one 16-byte buffer store per block, the buffer's
// extent ending at the tile so stores past it are dropped.
template <int WMAX, int NCX, int WFIX>
__global__ __launch_bounds__(512, 1) void conv3x3_x6_kernel(
    const float *__restrict__ x, const float *__restrict__ w, const float *__restrict__ bias,
    float *__restrict__ out, int H, int w_rt, int F, int act, int nrows) {
  const int W = WFIX > 0 ? WFIX : w_rt;
  constexpr int C = 32 * NCX;                        // channels: NCX runs of 32
  constexpr bool KSPLIT = NCX == 2;                  // wave halves split the channel runs (else blocks)
  constexpr int TR = WMAX <= 56 ? 2 : 1;             // output rows per tile (LDS bounds the ring)
  constexpr int NSLOT = 2 * TR + 2;                  // a tile's TR + 2 halo rows and the next tile's TR
  constexpr int SEGP = C / 4;                        // 16-byte f32 runs per input pixel
  constexpr int PST = 2 * C;                         // bytes from one part of a record to the next
  constexpr int RECB = 3 * PST + 32;                 // LDS halo record (bytes)
  constexpr int HCMAX = WMAX + 2;
  constexpr int SLOTB = HCMAX * RECB;                // bytes per row slot
  constexpr int NT = 512;                            // threads
  constexpr int LPR = (HCMAX * SEGP + NT - 1) / NT;  // loads per halo row
  constexpr int NBT = (TR * WMAX + 15) / 16;         // 16-pixel blocks of a full tile
  constexpr int NB1 = (WMAX + 15) / 16;              // ... of a 1-row tile
  constexpr int NBW = KSPLIT ? NBT : (NBT + 1) / 2;  // blocks per wave, full tile
  constexpr int NBW1 = KSPLIT ? NB1 : (NB1 + 1) / 2; // ... 1-row tile
  constexpr int NXB = (NBW + 1) / 2;                 // blocks per partial-sum exchange round
  constexpr int FPI = 8, NWI = 2;                    // filter loads: 8 filters' 128-byte runs per instruction, 2 per tap
  constexpr int WSR = 64 + 32;                       // filter staging record: one part of one filter's run
  constexpr int HALOB = NSLOT * SLOTB;
  constexpr int TRASHB = 64 * 8 + 2 * PST;           // lanes' 8-byte trash slots plus the part offsets
  constexpr int XB_SUM = KSPLIT ? 4 * NXB * 64 * 16 : 0;
  constexpr int XB_STAGE = 8 * 16 * WSR;
  constexpr int XB = XB_SUM > XB_STAGE ? XB_SUM : XB_STAGE;  // partial sums, or filter staging (before the walk)
  constexpr int FLAGB = 16;                          // set when a value fell outside the split's domain
  static_assert(HALOB + TRASHB + XB + FLAGB <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(16))) char lds[HALOB + TRASHB + XB + FLAGB];
  char *const halo = lds;
  char *const xch = lds + HALOB + TRASHB;
  int *const miss_flag = reinterpret_cast<int *>(lds + HALOB + TRASHB + XB);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int fg = wave & 3, half = wave >> 2;         // filter group; wave half
  const int run = KSPLIT ? half : 0;                 // this wave's channel run
  const RowRange range = row_range(nrows);
  const size_t row_bytes = (size_t)W * C * 4;
  auto tile_rows = [&](int g) __attribute__((always_inline)) { return min(min(TR, range.end - g), H - g % H); };

  // This wave's blocks: b = ii (channel split) or half + 2 ii (block split);
  // pixel b*16 + r of the tile lies in tile row bit ii of prow, halo
  // column pcol + 1 (the +1 and the tap's column shift are folded into the
  // read offsets, and so is the channel run).
  uint32_t colb[NBW];
  uint32_t prow = 0;
#pragma unroll
  for (int ii = 0; ii < NBW; ++ii) {
    const int b = KSPLIT ? ii : half + 2 * ii;
    const int p = min(b * 16 + r, TR * W - 1);
    const int pr = p / W, pc = p - pr * W;
    colb[ii] = (uint32_t)(pc * RECB + run * 64 + q * 16);
    prow |= (uint32_t)pr << ii;
  }
  // Halo row fetch: load j covers the row's 16-byte runs tid + NT j.
  // goff: byte offset in the input row (column clamped into the image);
  // loff: byte offset of the run's h part within a slot, or ~0u for a lane
  // with no record (past the row, or a zero-padding column).
  uint32_t goff[LPR], loff[LPR];
#pragma unroll
  for (int j = 0; j < LPR; ++j) {
    const int idx = tid + NT * j, idxc = min(idx, (W + 2) * SEGP - 1);
    const int hc = idxc / SEGP, seg = idxc - hc * SEGP;
    goff[j] = (uint32_t)(min(max(hc - 1, 0), W - 1) * C * 4 + seg * 16);
    const bool rec = idx < (W + 2) * SEGP && hc >= 1 && hc <= W;
    loff[j] = rec ? (uint32_t)(hc * RECB + seg * 8) : ~0u;
  }
  const uint32_t trash = (uint32_t)(HALOB + lane * 8);
  auto waddr = [&](int slot, int j) __attribute__((always_inline)) {
    return loff[j] == ~0u ? trash : (uint32_t)(slot * SLOTB) + loff[j];
  };
  auto load_row = [&](u32x4 (&dst)[LPR], int grow) __attribute__((always_inline)) {  // grow: an input row
    const char *rb = reinterpret_cast<const char *>(x) + (size_t)grow * row_bytes;
#pragma unroll
    for (int j = 0; j < LPR; ++j) dst[j] = *reinterpret_cast<const u32x4 *>(rb + goff[j]);
  };
  auto put_run = [&](uint32_t a, const Parts4 &p) __attribute__((always_inline)) {
    char *d = halo + a;
    *reinterpret_cast<uint2 *>(d) = p.h;
    *reinterpret_cast<uint2 *>(d + PST) = p.m;
    *reinterpret_cast<uint2 *>(d + 2 * PST) = p.l;
  };
  auto zero_run = [&](uint32_t a) __attribute__((always_inline)) {
    const uint2 z = make_uint2(0u, 0u);
    char *d = halo + a;
    *reinterpret_cast<uint2 *>(d) = z;
    *reinterpret_cast<uint2 *>(d + PST) = z;
    *reinterpret_cast<uint2 *>(d + 2 * PST) = z;
  };
  // All halo rows of the tile at g (fetch_tile), written to slots b, b+1,
  // ... (mod NSLOT) by put_tile; rows outside the image are zero.  Used where
  // no prefetch could run: the first tile, and a tile that starts an image.
  // Lanes whose split values fell outside the split's domain (Inf, NaN, or
  // magnitudes the split does not carry), over the whole walk: such a
  // workgroup recomputes its rows on the exact path at the end.
  uint64_t miss = 0;
  u32x4 fraw[TR + 2][LPR];
  auto fetch_tile = [&](int g) __attribute__((always_inline)) {
    const int n = g / H, h0 = g - n * H;
#pragma unroll
    for (int hr = 0; hr < TR + 2; ++hr) load_row(fraw[hr], n * H + min(max(h0 + hr - 1, 0), H - 1));
  };
  // run j of halo row hr of the tile at g, into slot b + hr
  auto put_fraw = [&](int g, int b, int hr, int j, SplitDomainBounds &bd) __attribute__((always_inline)) {
    const int rows = tile_rows(g), ih = g % H + hr - 1, slot = (b + hr) % NSLOT;
    if (hr > rows + 1) {
      // not a halo row of a short tile
    } else if (ih >= 0 && ih < H) {
      put_run(waddr(slot, j), split_parts(fraw[hr][j]));
      bd.fold(fraw[hr][j]);
    } else {
      zero_run(waddr(slot, j));
    }
  };
  auto put_tile = [&](int g, int b, int hr0, int hr1, SplitDomainBounds &bd) __attribute__((always_inline)) {
#pragma unroll
    for (int hr = hr0; hr < hr1; ++hr)
#pragma unroll
      for (int j = 0; j < LPR; ++j) put_fraw(g, b, hr, j, bd);
  };
  // The next tile's new rows (its halo rows 2..TR+1: image rows gn+1..gn+TR
  // for a tile starting at gn), fetched a tile ahead.  Unconditional (rows
  // clamped into the input): a fetch under a condition would make the
  // compiler drain every outstanding load at the loop head.
  u32x4 nraw[TR][LPR];
  auto prefetch = [&](int gn) __attribute__((always_inline)) {
    gn = min(gn, nrows - 1);
    const int n = gn / H, h0 = gn - n * H;
#pragma unroll
    for (int k = 0; k < TR; ++k) load_row(nraw[k], n * H + min(h0 + 1 + k, H - 1));
  };

  if (range.first >= range.end) return;  // uniform over the workgroup
  // Issue order matters (the counter of outstanding loads is in order):
  // the filters (from L2, split while the rest arrives), the first tile's
  // rows, the bias, then the next tile's new rows, each waited for in that
  // order.
  // Filters: this wave's 16 filters, its channel run, every tap: 128-byte
  // runs loaded whole, split, and turned into A fragments one part at a time
  // through this wave's staging slot (record stride WSR).
  u32x4 wraw[9][NWI];
  {
    const char *wb = reinterpret_cast<const char *>(w) + ((size_t)(blockIdx.y * 4 + fg) * 16 * 9 * C + run * 32) * 4;
    const int fl = lane / 8, pc = lane - fl * 8;
#pragma unroll
    for (int t = 0; t < 9; ++t)
#pragma unroll
      for (int i = 0; i < NWI; ++i)
        wraw[t][i] = *reinterpret_cast<const u32x4 *>(wb + ((size_t)(fl + FPI * i) * 9 + t) * C * 4 + pc * 16);
  }
  fetch_tile(range.first);
  const int fq = (blockIdx.y * 4 + fg) * 16 + 4 * q;
  float bv[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) bv[e] = bias && (!KSPLIT || half == 0) ? bias[fq + e] : 0.0f;
  const ActBounds ab = act_bounds(act);
  // (past the range: the first tile's own rows again, already in L2)
  const int g1 = range.first + tile_rows(range.first);
  prefetch(g1 < range.end ? g1 : range.first);
  Frag16 fr[9][3];  // [tap][part]
  SplitDomainBounds wbd;  // this wave's filter values (and the first tile's first rows)
  {
    char *const wslot = xch + wave * 16 * WSR;
    const int fl = lane / 8, pc = lane - fl * 8;
#pragma unroll
    for (int t = 0; t < 9; ++t) {
      Parts4 p[NWI];
#pragma unroll
      for (int i = 0; i < NWI; ++i) {
        p[i] = split_parts(wraw[t][i]);
        wbd.fold(wraw[t][i]);
      }
#pragma unroll
      for (int k = 0; k < 3; ++k) {
#pragma unroll
        for (int i = 0; i < NWI; ++i)
          *reinterpret_cast<uint2 *>(wslot + (fl + FPI * i) * WSR + pc * 8) = k == 0 ? p[i].h : k == 1 ? p[i].m : p[i].l;
        fr[t][k] = load16(wslot + r * WSR + q * 16);
      }
    }
  }
  // The first tile's halo rows 0 and 1 now; rows 2 and up during the first
  // third of its multiply (the taps of tap row 0 read rows 0 and 1 only).
  // With the row width known at compile time only: the run-time width's
  // index registers and those rows held over would not fit without spills.
  constexpr bool EARLY = WFIX > 0;
  int base = 0;  // slot of the current tile's halo row 0
  put_tile(range.first, base, 0, EARLY ? 2 : TR + 2, wbd);
  // zero-padding columns 0 and W+1 of every slot (lanes write no record there)
  constexpr int ZR = 3 * PST / 16;  // 16-byte runs of a record's parts
  for (int i = tid; i < NSLOT * 2 * ZR; i += NT) {
    const int s = i / (2 * ZR), k = i - s * 2 * ZR, side = k / ZR, seg = k - side * ZR;
    *reinterpret_cast<u32x4 *>(halo + s * SLOTB + side * (W + 1) * RECB + seg * 16) = u32x4{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) settle(bv[e]);
#pragma unroll
  for (int t = 0; t < 9; ++t)
#pragma unroll
    for (int k = 0; k < 3; ++k) settle(fr[t][k].u);
  // The accumulators start at the bias: a subnormal bias is carried by the
  // exact path (the MFMA's treatment of it is not the f32 add's).
  {
    bool sub = false;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t t = __float_as_uint(bv[e]) << 1;
      sub |= (t != 0u) & (t < (1u << 24));
    }
    miss |= __builtin_amdgcn_ballot_w64(sub);
  }
  miss |= __builtin_amdgcn_ballot_w64(wbd.miss());
  if (tid == 0) *miss_flag = 0;
  __syncthreads();  // halo, padding and every wave's filter staging done (staging shares the exchange area)

  auto tile = [&](int g, auto first) __attribute__((always_inline)) {
    constexpr bool FIRST = decltype(first)::value;
    const int rows = tile_rows(g);
    const int bnext = (base + rows) % NSLOT;  // the next tile's halo row 0
    // read bases: block ii, tap row dy -> slot of halo row (its row + dy)
    uint32_t rb[NBW][3];
#pragma unroll
    for (int dy = 0; dy < 3; ++dy) {
      const uint32_t s0 = (uint32_t)((base + dy) % NSLOT * SLOTB), s1 = (uint32_t)((base + dy + 1) % NSLOT * SLOTB);
#pragma unroll
      for (int ii = 0; ii < NBW; ++ii) rb[ii][dy] = ((prow >> ii) & 1u ? s1 : s0) + colb[ii];
    }
    // the next tile's new rows go to its slots 2..TR+1 (slots this tile does
    // not read); rows past the image are zero
    const int gn = g + rows, hn = gn % H;
    uint32_t nok = 0;
#pragma unroll
    for (int k = 0; k < TR; ++k) nok |= (uint32_t)(hn + 1 + k < H) << k;
    f32x4 acc[NBW];
#pragma unroll
    for (int ii = 0; ii < NBW; ++ii) acc[ii] = f32x4{bv[0], bv[1], bv[2], bv[3]};
    SplitDomainBounds nb;  // the new rows split during this tile
    // Steps s = (tap t, block ii) in order; each reads its block's three
    // pixel parts from LDS D steps ahead and issues six MFMAs.  From a third
    // of the way in, one new-row run is split and written every SPS steps.
    // The scheduling barrier keeps each step's work in its own region.
    auto multiply = [&](auto nblk) __attribute__((always_inline)) {
      constexpr int NB = decltype(nblk)::value;
      constexpr int NS = 9 * NB, D = 2, RB = D + 1;
      constexpr int NSPL = TR * LPR, S0 = NS / 3;
      constexpr int SPS = (NS - S0 - 2) / NSPL > 0 ? (NS - S0 - 2) / NSPL : 1;
      static_assert(S0 + SPS * (NSPL - 1) < NS, "every new-row run is written within the multiply");
      Frag16 px[RB][3];
      auto load_px = [&](Frag16 (&dst)[3], int s) __attribute__((always_inline)) {
        const int t = s / NB, ii = s - t * NB;
        const char *src = halo + rb[ii][t / 3] + (t % 3) * RECB;
#pragma unroll
        for (int k = 0; k < 3; ++k) dst[k] = load16(src + k * PST);
      };
#pragma unroll
      for (int s = 0; s < D; ++s) load_px(px[s], s);
      static_for<NS>([&](auto sc) __attribute__((always_inline)) {
        constexpr int s = decltype(sc)::value;
        if constexpr (s + D < NS) load_px(px[(s + D) % RB], s + D);
        mma_x6(acc[s % NB], fr[s / NB], px[s % RB]);
        if constexpr (FIRST) {
          // the first tile's halo rows 2 and 3, then a barrier before tap row 1
          constexpr int NF = TR * LPR, SPF = (3 * NB - 1) / NF > 0 ? (3 * NB - 1) / NF : 1;
          static_assert(SPF * (NF - 1) < 3 * NB - 1, "the first tile's last rows are written before tap row 1");
          if constexpr (s % SPF == 0 && s / SPF < NF) put_fraw(g, 0, 2 + (s / SPF) / LPR, (s / SPF) % LPR, nb);
          if constexpr (s == 3 * NB - 1) __syncthreads();
        }
        if constexpr (s >= S0 && (s - S0) % SPS == 0 && (s - S0) / SPS < NSPL) {
          // Branch-free, so the split's vector work stays in this step's
          // region beside its MFMAs: a row past the image is written as
          // zeros by a uniform select.
          constexpr int e = (s - S0) / SPS, k = e / LPR, j = e % LPR;
          const bool ok = (nok >> k) & 1u;
          Parts4 p = split_parts(nraw[k][j]);
          nb.fold(nraw[k][j]);  // (a row past the image is the clamped last row: checked anyway)
          const uint2 z = make_uint2(0u, 0u);
          p.h = ok ? p.h : z;
          p.m = ok ? p.m : z;
          p.l = ok ? p.l : z;
          put_run(waddr((bnext + 2 + k) % NSLOT, j), p);
        }
        __builtin_amdgcn_sched_barrier(0);
      });
    };
    if constexpr (TR == 1)
      multiply(std::integral_constant<int, NBW>{});
    else if (rows == TR)
      multiply(std::integral_constant<int, NBW>{});
    else
      multiply(std::integral_constant<int, NBW1>{});
    // outputs: the buffer ends at the tile, so stores of pixels past it drop
    const int npx = rows * W;
    const __amdgpu_buffer_rsrc_t o = __builtin_amdgcn_make_buffer_rsrc(
        reinterpret_cast<char *>(out) + ((size_t)g * W * F + blockIdx.y * 64 + fg * 16) * 4, (short)0,
        (npx - 1) * F * 4 + 64, 0x00020000);
    auto store = [&](int b, f32x4 a) __attribute__((always_inline)) {
      f32x4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = act_clamp(a[e], ab);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), o,
                                             (uint32_t)((b * 16 + r) * F * 4 + q * 16), 0, 0);
    };
    if constexpr (KSPLIT) {
      // The two partial sums of a block meet in LDS: blocks [0, NXB) are
      // finished by half 0, [NXB, NBW) by half 1, in two rounds through an
      // exchange area of NXB blocks per filter group.
      char *const xg = xch + fg * NXB * 1024 + lane * 16;
      miss |= __builtin_amdgcn_ballot_w64(nb.miss());
      if (miss != 0 && lane == 0) *miss_flag = 1;  // read after the walk
      if (half == 1) {
#pragma unroll
        for (int ii = 0; ii < NXB; ++ii) *reinterpret_cast<f32x4 *>(xg + ii * 1024) = acc[ii];
      }
      __syncthreads();
      if (half == 0) {
#pragma unroll
        for (int ii = 0; ii < NXB; ++ii) acc[ii] += *reinterpret_cast<const f32x4 *>(xg + ii * 1024);
#pragma unroll
        for (int ii = NXB; ii < NBW; ++ii) *reinterpret_cast<f32x4 *>(xg + (ii - NXB) * 1024) = acc[ii];
      }
      __syncthreads();
      if (half == 0) {
#pragma unroll
        for (int ii = 0; ii < NXB; ++ii) store(ii, acc[ii]);
      } else {
#pragma unroll
        for (int ii = NXB; ii < NBW; ++ii) store(ii, acc[ii] + *reinterpret_cast<const f32x4 *>(xg + (ii - NXB) * 1024));
      }
    } else {
#pragma unroll
      for (int ii = 0; ii < NBW; ++ii) store(half + 2 * ii, acc[ii]);
      miss |= __builtin_amdgcn_ballot_w64(nb.miss());
      if (miss != 0 && lane == 0) *miss_flag = 1;  // read after the walk
      __syncthreads();  // every wave's multiply (halo reads) and new-row writes are done
    }
    // The tile after next: fetched now, written during the next tile.  With
    // the channel split no further barrier is needed here: the exchange
    // barriers already follow every wave's multiply and new-row writes, and
    // a wave's next exchange writes come after its own reads of this one.
    // (past the range: this tile's rows again, fetched a tile ago and still in L2)
    const int g2 = gn + tile_rows(min(gn, range.end - 1));
    prefetch(g2 < range.end ? g2 : g);
    if (gn < range.end && hn == 0) {  // the next tile starts an image: its rows were not prefetched
      fetch_tile(gn);
      SplitDomainBounds ib;
      put_tile(gn, bnext, 0, TR + 2, ib);
      miss |= __builtin_amdgcn_ballot_w64(ib.miss());
      if (miss != 0 && lane == 0) *miss_flag = 1;
      __syncthreads();
    }
    base = bnext;
  };
  tile(range.first, std::integral_constant<bool, EARLY>{});
  for (int g = range.first + tile_rows(range.first); g < range.end; g += tile_rows(g))
    tile(g, std::integral_constant<bool, false>{});
  // A value outside the split's domain anywhere in the walk (every split
  // precedes the last tile's barrier, which also published the flag): once
  // every wave's stores have completed, the range is computed again on the
  // exact path, whose stores then land after them.
  if (*miss_flag != 0) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    conv3x3_exact_rows<C>(x, w, bias, out, H, W, F, act, blockIdx.y * 64, range.first, range.end);
  }
}

// Vector-ALU instructions per wave of the persistent kernel, counted in its
// compiled code (gfx950 assembly, vector instructions other than MFMAs per
// basic block): per 2-row tile 105 (the epilogue's bias, activation and
// bf16 packing, slot and loop control) plus 20 per 64-byte input chunk (the
// next rows' commit and halo writes): 145 at two chunks, 185 at four; 196
// once (the filter fragments' staging and the first halo).
constexpr double STREAM_VALU_TILE_FIXED = 105.0;
constexpr double STREAM_VALU_TILE_PER_CHUNK = 20.0;
constexpr double STREAM_VALU_SETUP = 196.0;

template <class MM, typename T, int WMAX, int NCH, int WFIX>
hipError_t launch_stream(const ConvArgs &a, int wgs, hipStream_t s) {
  if (a.W > WMAX || (WFIX > 0 && a.W != WFIX) || a.C != MM::kPerFrag * NCH || a.F % 64 != 0 ||
      wgs % kXcds != 0)
    return hipErrorInvalidValue;
  const int nrows = a.N * a.H;
  dim3 grid(wgs, (a.F + 63) / 64);
  {
    // The plan's work unit is one output row (half a 2-row tile): the walk
    // gives each workgroup a contiguous range of rows.
    constexpr int TR = 2, PBW = (TR * WMAX + 15) / 16, REC = NCH * 64 + 32;
    const double es = sizeof(T);
    npu_launch_plan p =
        make_plan("conv3x3_persistent", wgs * grid.y,
                  wg_per_cu(conv3x3_stream_kernel<MM, T, WMAX, NCH, WFIX>), nrows * grid.y, 8 * sizeof(T));
    p.load_phases = 0;  // the next tile's halo is fetched during this tile
    p.tile_macs = 4.0 * (PBW / 2.0) * 256 * 9 * a.C;
    // vector-ALU instructions per row, summed over the four waves
    p.tile_valu = 4.0 * (STREAM_VALU_TILE_FIXED + STREAM_VALU_TILE_PER_CHUNK * NCH) / TR;
    p.wg_setup_valu = 4.0 * STREAM_VALU_SETUP;
    p.tile_lds_bytes = 2.0 * (a.W + 2) * REC +                  // halo written
                       2.0 * PBW * 9 * NCH * 1024 +             // B fragments read
                       2.0 * a.W * (64 * es + 32);              // output staged and read
    p.tile_load_bytes = 2.0 * (a.W + 2) * a.C * es;
    p.tile_store_bytes = a.W * 64 * es;
    p.wg_setup_bytes = 4.0 * 16 * 9 * a.C * es;
    p.hbm_bytes = es * ((double)a.N * a.H * a.W * a.C + 9.0 * a.F * a.C + (double)a.N * a.H * a.W * a.F) +
                  (a.bias ? 4.0 * a.F : 0.0);
    plans_add(p);
  }
  hipLaunchKernelGGL((conv3x3_stream_kernel<MM, T, WMAX, NCH, WFIX>), grid, dim3(256), 0, s,
                     static_cast<const T *>(a.x), static_cast<const T *>(a.w), a.bias,
                     static_cast<T *>(a.out), a.H, a.W, a.F, a.act, nrows);
  return hipGetLastError();
}

// Vector-ALU instructions per wave of the f32 walk on the bf16 pipe, from
// its compiled loops: per tile 34 per 16-byte new-row run split into three
// parts, written and folded into the split-domain bounds (TR x LPR runs),
// 20 per 16-pixel block (activation, store address, the partial-sum
// exchange), 64 for slots, read bases and the prefetch; once, 34 per
// filter run split (9 taps x 2 runs), 160 for the first tile's rows and the
// addresses, 20 for the bias check and the end-of-walk domain test.
constexpr double X6_VALU_SPLIT_RUN = 34.0;
constexpr double X6_VALU_BLOCK = 20.0;
constexpr double X6_VALU_TILE = 64.0;
constexpr double X6_VALU_SETUP = 9 * 2 * 34.0 + 160.0 + 20.0;

template <int WMAX, int NCX, int WFIX>
hipError_t launch_x6(const ConvArgs &a, hipStream_t s) {
  const int wgs = persistent_grid(conv3x3_x6_kernel<WMAX, NCX, WFIX>, 512);
  if (wgs == 0) return hipErrorInvalidDeviceFunction;
  if (a.W > WMAX || (WFIX > 0 && a.W != WFIX) || a.C != 32 * NCX || a.F % 64 != 0 || wgs % kXcds != 0)
    return hipErrorInvalidValue;
  const int nrows = a.N * a.H;
  dim3 grid(wgs, a.F / 64);
  {
    // One output row is the plan's work unit; 6 bf16 MACs per f32 MAC.
    // Each input row is fetched, split and written to the halo ring once.
    constexpr int TR = WMAX <= 56 ? 2 : 1, NBT = (TR * WMAX + 15) / 16, RECB = 6 * 32 * NCX + 32;
    constexpr double BLOCKS_ROW = (double)NBT / TR;  // 16-pixel blocks per output row
    npu_launch_plan p = make_plan("conv3x3_f32_bf16x6", wgs * grid.y,
                                  wg_per_cu(conv3x3_x6_kernel<WMAX, NCX, WFIX>, 512), nrows * grid.y, 16);
    p.load_phases = 0;  // the next tile's new rows are fetched a tile ahead
    p.unit_waves = 8;   // one grid unit is a whole eight-wave workgroup
    p.tile_macs = 6.0 * 4.0 * BLOCKS_ROW * 256 * 9 * a.C;
    constexpr int LPR = ((WMAX + 2) * 8 * NCX + 511) / 512;  // 16-byte runs per lane and input row
    constexpr int NBW = NCX == 2 ? NBT : (NBT + 1) / 2;           // blocks per wave
    // per row, eight waves
    p.tile_valu = 8.0 * (X6_VALU_SPLIT_RUN * TR * LPR + X6_VALU_BLOCK * NBW + X6_VALU_TILE) / TR;
    p.wg_setup_valu = 8.0 * X6_VALU_SETUP;
    p.tile_lds_bytes = (a.W + 2.0) * RECB +                           // halo row written
                       4.0 * BLOCKS_ROW * 9 * NCX * 3 * 1024 +        // pixel parts read (four filter groups)
                       (NCX == 2 ? 2.0 * 4.0 * BLOCKS_ROW / 2 * 1024 : 0.0);  // partial sums exchanged
    p.tile_load_bytes = (a.W + 2.0) * a.C * 4;
    p.tile_store_bytes = a.W * 64 * 4;
    p.wg_setup_bytes = 4.0 * 16 * 9 * a.C * 4;
    p.hbm_bytes = 4.0 * ((double)a.N * a.H * a.W * a.C + 9.0 * a.F * a.C + (double)a.N * a.H * a.W * a.F) +
                  (a.bias ? 4.0 * a.F : 0.0);
    plans_add(p);
  }
  hipLaunchKernelGGL((conv3x3_x6_kernel<WMAX, NCX, WFIX>), grid, dim3(512), 0, s,
                     static_cast<const float *>(a.x), static_cast<const float *>(a.w), a.bias,
                     static_cast<float *>(a.out), a.H, a.W, a.F, a.act, nrows);
  return hipGetLastError();
}

template <class MM, typename T, int TR, int WF, int WMAX, int NCH, int NBUF, int WFIX>
hipError_t launch_rows(const ConvArgs &a, hipStream_t s) {
  if (a.W > WMAX || (WFIX > 0 && a.W != WFIX) || a.C % (MM::kPerFrag * NCH) != 0 ||
      (NBUF == 1 && a.C != MM::kPerFrag * NCH))
    return hipErrorInvalidValue;
  const int tiles_h = (a.H + TR - 1) / TR;
  dim3 grid(a.N * tiles_h, (a.F + 16 * WF - 1) / (16 * WF));
  {
    constexpr int WP = 4 / WF, PBW = ((TR * WMAX + 15) / 16 + WP - 1) / WP;
    constexpr int REC = NCH * 64 + 32;
    const int nstages = a.C / (MM::kPerFrag * NCH);
    const double es = sizeof(T);
    npu_launch_plan p = make_plan("conv3x3_rows", grid.x * grid.y,
                                  wg_per_cu(conv3x3_rows_kernel<MM, T, TR, WF, WMAX, NCH, NBUF, WFIX>),
                                  grid.x * grid.y, 8 * sizeof(T));
    p.load_phases = 1;  // later stages are fetched while the previous one computes
    p.tile_macs = 4.0 * PBW * 256 * 9 * a.C;
    // Vector instructions per wave, from the compiled loops.  With the row
    // width compiled in (WFIX, 56), a one-row, single-stage kernel runs
    // straight-line code, the filters staged in LDS (the halo's addresses
    // and commit, the staging's loads and writes, the epilogue): 478 for
    // f32 at 64 channels, 300 for 2304-byte filter rows (f32 32 channels,
    // bf16 64).
    // Otherwise: the first stages' halo and filter staging (260 f32, 400
    // bf16: twice the 16-byte runs), 41 per stage, the epilogue (bias,
    // activation, conversion and the stores of the tile's pixel blocks) 137.
    constexpr bool WLDS = NBUF == 1 && WF == 1;
    p.tile_valu = 4.0 * (WFIX > 0 && NBUF == 1 && TR == 1
                             ? (WLDS ? (sizeof(T) == 4 && NCH == 4 ? 478.0 : 300.0) : 235.0)
                             : (sizeof(T) == 4 ? 260.0 : 400.0) + 41.0 * nstages + 137.0);
    p.tile_lds_bytes = (TR + 2.0) * (a.W + 2) * REC * nstages + 4.0 * PBW * 9 * NCH * 1024 * nstages +
                       (WLDS ? 2.0 * 16 * 9 * a.C * es : 0.0);  // filters staged and read
    p.tile_load_bytes = (TR + 2.0) * (a.W + 2) * a.C * es + (WLDS ? 1.0 : 4.0) * 16 * 9 * a.C * es;
    p.tile_store_bytes = (double)TR * a.W * 16 * WF * es;
    p.hbm_bytes = es * ((double)a.N * a.H * a.W * a.C + 9.0 * a.F * a.C + (double)a.N * a.H * a.W * a.F) +
                  (a.bias ? 4.0 * a.F : 0.0);
    plans_add(p);
  }
  hipLaunchKernelGGL((conv3x3_rows_kernel<MM, T, TR, WF, WMAX, NCH, NBUF, WFIX>), grid, dim3(256), 0, s,
                     static_cast<const T *>(a.x), static_cast<const T *>(a.w), a.bias,
                     static_cast<T *>(a.out), a.H, a.W, a.C, a.F, a.act);
  return hipGetLastError();
}

template <class MM, typename T, int WMAX, int NCH, int WFIX>
hipError_t launch_persistent(const ConvArgs &a, hipStream_t s) {
  const int g = persistent_grid(conv3x3_stream_kernel<MM, T, WMAX, NCH, WFIX>);
  if (g == 0) return hipErrorInvalidDeviceFunction;
  return launch_stream<MM, T, WMAX, NCH, WFIX>(a, g, s);
}

// Launch shapes.  With C of two or four chunks, F a multiple of 64 and at
// least 48 row pairs (two 56-row images), a persistent kernel (filter
// fragments held in registers): for f32 the one on the bf16 pipe (32 or 64
// channels), for bf16 the stream kernel.  Its per-workgroup set-up (filters
// loaded, for f32 split) costs about 2.5 us once, where the one-workgroup-per-
// tile kernels refetch the filters and re-stage the halo per tile: on
// 56x56x64 -> 64 those take 5.4 (f32) and 2.3 us (bf16) per further image,
// the persistent kernels 1.1 and 0.3.  Else one workgroup per tile: 2 rows x
// 64 filters (waves split the filters) when tiles are many, 1 row x 16
// filters (waves split the row) when few, so the grid still spreads over the
// CUs.  Rows of up to 56 pixels use tiles sized for 56 (7 pixel blocks for 2
// rows, none wasted); a row width of exactly 56 is also compiled in, so
// index arithmetic folds.
template <class MM, typename T, int WMAX, int WFIX>
hipError_t launch_w(const ConvArgs &a, hipStream_t s) {
  const int pairs = a.N * ((a.H + 1) / 2);
  const bool big = pairs >= 512;
  if (pairs >= 48 && a.F % 64 == 0) {
    if constexpr (sizeof(T) == 4) {  // f32: on the bf16 pipe
      if (a.C == 32) return launch_x6<WMAX, 1, WFIX>(a, s);
      if (a.C == 64) return launch_x6<WMAX, 2, WFIX>(a, s);
    } else {
      if (a.C == 2 * MM::kPerFrag) return launch_persistent<MM, T, WMAX, 2, WFIX>(a, s);
      if (a.C == 4 * MM::kPerFrag) return launch_persistent<MM, T, WMAX, 4, WFIX>(a, s);
    }
  }
  if (a.C == 2 * MM::kPerFrag)
    return big ? launch_rows<MM, T, 2, 4, WMAX, 2, 1, WFIX>(a, s) : launch_rows<MM, T, 1, 1, WMAX, 2, 1, WFIX>(a, s);
  if constexpr (sizeof(T) == 4)
    if (!big && a.C == 4 * MM::kPerFrag) return launch_rows<MM, T, 1, 1, WMAX, 4, 1, WFIX>(a, s);
  return big ? launch_rows<MM, T, 2, 4, WMAX, 1, 2, WFIX>(a, s) : launch_rows<MM, T, 1, 1, WMAX, 1, 2, WFIX>(a, s);
}

template <class MM, typename T>
hipError_t launch_conv3x3(const ConvArgs &a, hipStream_t s) {
  if (a.W == 56) return launch_w<MM, T, 56, 56>(a, s);
  return a.W < 56 ? launch_w<MM, T, 56, 0>(a, s) : launch_w<MM, T, 64, 0>(a, s);
}

}  // namespace

bool conv3x3_rows_supported(const ConvArgs &a, int elem_bytes) {
  const int kc = 64 / elem_bytes;
  return a.KH == 3 && a.KW == 3 && a.pad == 1 && a.W <= 64 && a.C % kc == 0 && a.F % 16 == 0;
}

hipError_t launch_conv3x3_f32(const ConvArgs &a, hipStream_t s) {
  return launch_conv3x3<MfmaF32, float>(a, s);
}
hipError_t launch_conv3x3_bf16(const ConvArgs &a, hipStream_t s) {
  return launch_conv3x3<MfmaBF16, uint16_t>(a, s);
}

}  // namespace npu
