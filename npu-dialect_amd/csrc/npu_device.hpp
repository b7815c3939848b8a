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

__device__ __forceinline__ Frag16 load16(const void *p) {
  Frag16 r;
  r.u = *reinterpret_cast<const u32x4 *>(p);
  return r;
}

}  // namespace npu
