// npu_device.hpp -- shared gfx950 device helpers: MFMA fragment types, the
// 16x16 output-tile lane layout, bf16 rounding, buffer predicates.
//
// MFMA tiles used throughout (CDNA4, wave64):
//   v_mfma_f32_16x16x4_f32    A: 1 f32 / lane   B: 1 f32 / lane
//   v_mfma_f32_16x16x32_bf16  A: 8 bf16 / lane  B: 8 bf16 / lane
//   v_mfma_i32_16x16x64_i8    A: 16 i8 / lane   B: 16 i8 / lane
// For all three, lane l feeds row (l % 16) of A and column (l % 16) of B,
// and the k slots it feeds are a fixed function of (l / 16).  Because a dot
// product does not depend on the order of its k terms, any bijection between
// k slots and reduction indices works as long as A and B use the same one;
// we pick the one that makes every lane's operand a single 16-byte run of
// the reduction dimension (4 f32, 8 bf16 or 16 i8 consecutive channels).
// The f32 case covers 16 reduction indices with four back-to-back MFMAs: step
// s uses index 4*(l/16) + s.
//
// Accumulator layout of a 16x16 output tile: lane l holds rows
// 4*(l/16) + r, r = 0..3, of column l % 16.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

namespace npu {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// A 16-byte operand fragment, reinterpreted per element type.
union Frag16 {
  u32x4 u;
  f32x4 f;
  bf16x8 h;
  i32x4 i;
};

__device__ __forceinline__ Frag16 frag_zero() {
  Frag16 z;
  z.u = u32x4{0u, 0u, 0u, 0u};
  return z;
}

// acc += A_frag (16 rows x 16-byte k run) * B_frag, per element type.
// A fragment pair is kSteps MFMA instructions; step(s) issues the s-th, so a
// caller can interleave independent accumulators between dependent steps.
struct MfmaF32 {
  using acc_t = f32x4;
  static constexpr int kPerFrag = 16;  // reduction indices covered per frag pair (4 lanes groups x 4)
  static constexpr int kPerLane = 4;   // consecutive elements per lane in 16 bytes
  static constexpr int kSteps = 4;
  __device__ __forceinline__ static void step(acc_t &acc, const Frag16 &a, const Frag16 &b, int s) {
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.f[s], b.f[s], acc, 0, 0, 0);
  }
  __device__ __forceinline__ static void mma(acc_t &acc, const Frag16 &a, const Frag16 &b) {
#pragma unroll
    for (int s = 0; s < kSteps; ++s) step(acc, a, b, s);
  }
};

struct MfmaBF16 {
  using acc_t = f32x4;
  static constexpr int kPerFrag = 32;
  static constexpr int kPerLane = 8;
  static constexpr int kSteps = 1;
  __device__ __forceinline__ static void step(acc_t &acc, const Frag16 &a, const Frag16 &b, int) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.h, b.h, acc, 0, 0, 0);
  }
  __device__ __forceinline__ static void mma(acc_t &acc, const Frag16 &a, const Frag16 &b) {
    step(acc, a, b, 0);
  }
};

struct MfmaI8 {
  using acc_t = i32x4;
  static constexpr int kPerFrag = 64;
  static constexpr int kPerLane = 16;
  static constexpr int kSteps = 1;
  __device__ __forceinline__ static void step(acc_t &acc, const Frag16 &a, const Frag16 &b, int) {
    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a.i, b.i, acc, 0, 0, 0);
  }
  __device__ __forceinline__ static void mma(acc_t &acc, const Frag16 &a, const Frag16 &b) {
    step(acc, a, b, 0);
  }
};

// Loads are issued unconditionally from an always-valid address and masked
// afterwards with a select: a load under a divergent branch makes the
// compiler wait for every outstanding load (vmcnt(0)) before its first use,
// which defeats prefetching.
__device__ __forceinline__ u32x4 masked(u32x4 v, bool keep) {
  const uint32_t m = keep ? 0xffffffffu : 0u;
  return u32x4{v[0] & m, v[1] & m, v[2] & m, v[3] & m};
}

// ---- bf16 <-> f32, round to nearest even (arith.truncf) -------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(((uint32_t)h) << 16);
}
// gfx950 converts in hardware (v_cvt_pk_bf16_f32): round to nearest even,
// NaN stays NaN.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  const __bf16 h = (__bf16)f;
  return __builtin_bit_cast(uint16_t, h);
}

// arith.maximumf / minimumf semantics (NaN propagates).
__device__ __forceinline__ float act_apply(float v, int act) {
  if (act == 1) return (v != v) ? v : (v > 0.0f ? v : 0.0f);
  if (act == 2) {
    if (v != v) return v;
    v = v > 0.0f ? v : 0.0f;
    return v < 6.0f ? v : 6.0f;
  }
  return v;
}

// The same activations without a branch per element: the activation is
// resolved once into clamp bounds (none: [-inf, inf], ReLU: [0, inf],
// ReLU6: [0, 6]) and a NaN passes through the select.
struct ActBounds {
  float lo, hi;
};
__device__ __forceinline__ ActBounds act_bounds(int act) {
  const float inf = __builtin_inff();
  return ActBounds{act == 0 ? -inf : 0.0f, act == 2 ? 6.0f : inf};
}
// IEEE maximum/minimum (NaN in, NaN out; -0 < +0): gfx950's v_maximum3_f32
// and v_minimum3_f32, one instruction each.
__device__ __forceinline__ float act_clamp(float v, ActBounds b) {
  return __builtin_elementwise_minimum(__builtin_elementwise_maximum(v, b.lo), b.hi);
}

// f(std::integral_constant<int, 0>{}) ... f(std::integral_constant<int, N-1>{}),
// in order: a loop whose body indexes register arrays by its counter, unrolled
// whatever its length (a `#pragma unroll` loop that the compiler declines to
// unroll moves such arrays to scratch memory).
template <class Fn, int... I>
__device__ __forceinline__ void static_for_impl(Fn &&f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class Fn>
__device__ __forceinline__ void static_for(Fn &&f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Sum of a float over the 64 lanes of a wave, the same in every lane: DPP
// within each row of 16 lanes (quad permutes xor 1 and xor 2, then the
// half-row and row mirrors, each pairing a lane with one that holds the other
// half of its group), then the four rows' sums read out and added.  Vector-
// ALU work only, where a __shfl_xor ladder is six dependent LDS-crossbar
// round trips.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_mov<0xb1>(v);   // quad_perm [1,0,3,2]
  v += dpp_mov<0x4e>(v);   // quad_perm [2,3,0,1]
  v += dpp_mov<0x141>(v);  // row_half_mirror
  v += dpp_mov<0x140>(v);  // row_mirror
  const int u = __float_as_int(v);
  return ((__int_as_float(__builtin_amdgcn_readlane(u, 0)) + __int_as_float(__builtin_amdgcn_readlane(u, 16))) +
          __int_as_float(__builtin_amdgcn_readlane(u, 32))) +
         __int_as_float(__builtin_amdgcn_readlane(u, 48));
}

// A lane's value and that of lane ^ 16 (or ^ 32), in vector registers:
// gfx950's v_permlane16_swap (v_permlane32_swap) of (x, x) leaves, in every
// lane, the value of the even 16-lane row (lower 32-lane half) of its pair
// in .lo and that of the odd one in .hi.  lo op hi is then the pair's
// reduction, the same in both lanes, with no LDS-crossbar round trip.
struct LanePair {
  float lo, hi;
};
__device__ __forceinline__ LanePair lane_pair16(float x) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return LanePair{__uint_as_float(p[0]), __uint_as_float(p[1])};
}
__device__ __forceinline__ LanePair lane_pair32(float x) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return LanePair{__uint_as_float(p[0]), __uint_as_float(p[1])};
}

__device__ __forceinline__ Frag16 load16(const void *p) {
  Frag16 r;
  r.u = *reinterpret_cast<const u32x4 *>(p);
  return r;
}

// ---- f32 products on the bf16 matrix pipe ----------------------------------
// An f32 value a splits exactly into three bf16 parts, a = h + m + l: h is a
// with its low 16 bits cleared (its top 8 significant bits; never rounds up
// to Inf), m is r = a - h rounded to nearest even, and l = r - m, which has
// at most 8 significant bits and so is a bf16 exactly.  |m| < 2^-7 |a| and
// |l| <= 2^-8 |m|.  A product a*b is summed from the six part products
// mm, lh, hl, mh, hm, hh (smallest first); the three left out (ml, lm, ll)
// add up to less than 2^-21 |a b|.  This is the bf16x6 scheme of Henry,
// Tang and Heinecke, "Leveraging the bfloat16 Artificial Intelligence
// Datatype For Higher-Precision Computations" (ARITH 2019), with a
// truncating first split.  On gfx950 a bf16 MFMA (16 clocks for 16x16x32)
// does the 16x work of an f32 MFMA (32 clocks for 16x16x4), so the six
// products take 6 * 16 clocks where the f32 instructions take 8 * 32.
//
// The split's domain: zero, or a finite magnitude in [2^-E, 2^E) with
// E = kSplitDomainLog2.  There every part is exact (a's low part keeps its
// bits far above bf16's subnormals), every part product that mma_x6 keeps
// is exact in f32 or rounds at f32's subnormal spacing (the MFMA keeps f32
// subnormals), every product of two such values is at least 2^-2E, and no
// sum of products comes near the f32 range: the six products give the
// f32 sum to f32 accuracy.  Outside it the split is not used: an infinite
// a gives h = a and r = Inf - Inf = NaN (and splitting it into (a, 0, 0)
// would not help: its products with the zero parts of a finite b are
// Inf * 0), a value below 2^-102 loses its low part under bf16's
// subnormals, and products of tiny values round differently from the f32
// products.  A kernel that splits tests every value (SplitDomainBounds) and
// computes the outputs such values reach without the split.
constexpr int kSplitDomainLog2 = 55;
struct Parts4 {  // parts of four f32 values, two bf16 per dword
  uint2 h, m, l;
};
__device__ __forceinline__ uint32_t pack_high_halves(uint32_t lo, uint32_t hi) {
  return __builtin_amdgcn_perm(hi, lo, 0x07060302u);  // (lo >> 16) | (hi & 0xffff0000)
}
__device__ __forceinline__ uint32_t cvt_pk_bf16(float a, float b) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  bf16x2 v;
  v[0] = (__bf16)a;
  v[1] = (__bf16)b;
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ Parts4 split_parts(u32x4 v) {
  float r[4];
  uint32_t hb[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    hb[e] = v[e] & 0xffff0000u;
    r[e] = __uint_as_float(v[e]) - __uint_as_float(hb[e]);  // exact
  }
  Parts4 p;
  p.h = make_uint2(pack_high_halves(hb[0], hb[1]), pack_high_halves(hb[2], hb[3]));
  p.m = make_uint2(cvt_pk_bf16(r[0], r[1]), cvt_pk_bf16(r[2], r[3]));
  const float s0 = r[0] - __uint_as_float(p.m.x << 16), s1 = r[1] - __uint_as_float(p.m.x & 0xffff0000u);
  const float s2 = r[2] - __uint_as_float(p.m.y << 16), s3 = r[3] - __uint_as_float(p.m.y & 0xffff0000u);
  p.l = make_uint2(cvt_pk_bf16(s0, s1), cvt_pk_bf16(s2, s3));
  return p;
}
// The domain test, spread over the runs a lane splits: fold() takes a
// 16-byte run into two running bounds, the largest magnitude by IEEE
// maximum (NaN in, NaN out, so NaN and Inf fail `< 2^E`) and the smallest
// 2|bits| - 1 (the sign shifted out; zero wraps to 0xffffffff, above every
// nonzero value); miss() compares them once with 2^E and 2 bits(2^-E) - 1.
// Four values cost four shifts, a min3 and two maximum3.
struct SplitDomainBounds {
  uint32_t umin = 0xffffffffu;
  float amax = 0.0f;
  __device__ __forceinline__ void fold(u32x4 v) {
    uint32_t u[4];
    float a[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      u[e] = (v[e] << 1) + 0xffffffffu;
      a[e] = __builtin_fabsf(__uint_as_float(v[e]));
    }
    umin = min(min(umin, u[0]), min(min(u[1], u[2]), u[3]));
    amax = __builtin_elementwise_maximum(__builtin_elementwise_maximum(amax, a[0]),
                                         __builtin_elementwise_maximum(a[1], __builtin_elementwise_maximum(a[2], a[3])));
  }
  __device__ __forceinline__ bool miss() const {
    constexpr uint32_t LO2 = (uint32_t)(127 - kSplitDomainLog2) << 24;
    const float big = __uint_as_float((uint32_t)(127 + kSplitDomainLog2) << 23);
    return (umin < LO2 - 1u) | !(amax < big);
  }
};

// acc += A * B over one 32-long k run, A and B given as their three parts.
__device__ __forceinline__ void mma_x6(f32x4 &acc, const Frag16 (&a)[3], const Frag16 (&b)[3]) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[1].h, b[1].h, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[2].h, b[0].h, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0].h, b[2].h, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[1].h, b[0].h, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0].h, b[1].h, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0].h, b[0].h, acc, 0, 0, 0);
}

}  // namespace npu
