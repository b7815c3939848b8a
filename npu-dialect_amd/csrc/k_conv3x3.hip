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

template <class MM, typename T, int TR, int WF, int WMAX, int NCH, int NBUF>
__global__ __launch_bounds__(256) void conv3x3_rows_kernel(
    const T *__restrict__ x, const T *__restrict__ w, const float *__restrict__ bias,
    T *__restrict__ out, int H, int W, int C, int F, int act) {
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
  __shared__ __attribute__((aligned(16))) T halo[NBUF][HR * (WMAX + 2) * REC];

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
  fetch_b(b, 0);
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
    Frag16 a[2][PBW];
    load_a(a[0], 0);
#pragma unroll
    for (int j = 0; j < NCH * 9; ++j) {
      if (j + 1 < NCH * 9) load_a(a[(j + 1) & 1], j + 1);
      // independent accumulators between the dependent steps of one fragment
#pragma unroll
      for (int s = 0; s < MM::kSteps; ++s)
#pragma unroll
        for (int i = 0; i < PBW; ++i) MM::step(acc[i], a[j & 1][i], b[j / 9][j % 9], s);
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
template <class MM, typename T, int WMAX, int NCH, int WFIX>
__global__ __launch_bounds__(256, NCH <= 2 ? 2 : 1) void conv3x3_stream_kernel(
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

// Vector-ALU instructions per wave and output row of the persistent kernel
// (counted with SQ_INSTS_VALU less SQ_INSTS_MFMA): a fixed part (epilogue,
// loop control) and a part per 64-byte input chunk (halo commit, fetch).
constexpr double STREAM_VALU_ROW_FIXED = 127.6;
constexpr double STREAM_VALU_ROW_PER_CHUNK = 0.45;

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
    p.tile_valu = 4.0 * (STREAM_VALU_ROW_FIXED + STREAM_VALU_ROW_PER_CHUNK * NCH);
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

template <class MM, typename T, int TR, int WF, int WMAX, int NCH, int NBUF>
hipError_t launch_rows(const ConvArgs &a, hipStream_t s) {
  if (a.W > WMAX || a.C % (MM::kPerFrag * NCH) != 0 ||
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
                                  wg_per_cu(conv3x3_rows_kernel<MM, T, TR, WF, WMAX, NCH, NBUF>),
                                  grid.x * grid.y, 8 * sizeof(T));
    p.load_phases = 1;  // later stages are fetched while the previous one computes
    p.tile_macs = 4.0 * PBW * 256 * 9 * a.C;
    // counted per wave: 570 (f32, one chunk per stage, four stages), 554 (bf16, one stage)
    p.tile_valu = 4.0 * (540.0 + 8.0 * nstages * PBW);
    p.tile_lds_bytes = (TR + 2.0) * (a.W + 2) * REC * nstages + 4.0 * PBW * 9 * NCH * 1024 * nstages;
    p.tile_load_bytes = (TR + 2.0) * (a.W + 2) * a.C * es + 4.0 * 16 * 9 * a.C * es;
    p.tile_store_bytes = (double)TR * a.W * 16 * WF * es;
    p.hbm_bytes = es * ((double)a.N * a.H * a.W * a.C + 9.0 * a.F * a.C + (double)a.N * a.H * a.W * a.F) +
                  (a.bias ? 4.0 * a.F : 0.0);
    plans_add(p);
  }
  hipLaunchKernelGGL((conv3x3_rows_kernel<MM, T, TR, WF, WMAX, NCH, NBUF>), grid, dim3(256), 0, s,
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

// Launch shapes.  With many row tiles (batched images) and C of two or four
// chunks, the persistent kernel (filter fragments held in registers); else
// one workgroup per tile: 2 rows x 64 filters (waves split the filters) when
// tiles are many, 1 row x 16 filters (waves split the row) when few (batch
// 1), so the grid still spreads over the CUs.  Rows of up to 56 pixels use
// tiles sized for 56 (7 pixel blocks for 2 rows, none wasted); a row width
// of exactly 56 is also compiled in, so index arithmetic folds.
template <class MM, typename T, int WMAX, int WFIX>
hipError_t launch_w(const ConvArgs &a, hipStream_t s) {
  const bool big = a.N * ((a.H + 1) / 2) >= 512;
  if (big && a.F % 64 == 0) {
    if (a.C == 2 * MM::kPerFrag) return launch_persistent<MM, T, WMAX, 2, WFIX>(a, s);
    if (a.C == 4 * MM::kPerFrag) return launch_persistent<MM, T, WMAX, 4, WFIX>(a, s);
  }
  if (a.C == 2 * MM::kPerFrag)
    return big ? launch_rows<MM, T, 2, 4, WMAX, 2, 1>(a, s) : launch_rows<MM, T, 1, 1, WMAX, 2, 1>(a, s);
  return big ? launch_rows<MM, T, 2, 4, WMAX, 1, 2>(a, s) : launch_rows<MM, T, 1, 1, WMAX, 1, 2>(a, s);
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
