// abi.hip -- the extern "C" boundary: descriptor validation, error
// reporting, dispatch to the kernel launchers.
//
// Every entry point checks its memref descriptors against the group's shape
// and dtype contract before launching anything, and reports the first
// mismatch through npu_last_error() (thread-local), so a bad call returns a
// status instead of faulting the GPU.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/npu_amd.h"
#include "kernels.hpp"
#include "plans.hpp"

#include <vector>

namespace npu {

namespace {
thread_local std::vector<npu_launch_plan> g_plans;
}

void plans_reset() { g_plans.clear(); }
void plans_add(const npu_launch_plan &p) { g_plans.push_back(p); }

}  // namespace npu

namespace {

thread_local std::string g_last_error;

}  // namespace

namespace npu {
void set_last_error(const char *msg) { g_last_error = msg ? msg : ""; }
}  // namespace npu

namespace {

npu_status fail(npu_status code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

npu_status ok() {
  g_last_error.clear();
  return NPU_OK;
}

int64_t dtype_size(int32_t dt) {
  switch (dt) {
    case NPU_F32: return 4;
    case NPU_BF16: return 2;
    case NPU_I8: return 1;
    case NPU_I32: return 4;
    default: return 0;
  }
}

const char *dtype_name(int32_t dt) {
  switch (dt) {
    case NPU_F32: return "f32";
    case NPU_BF16: return "bf16";
    case NPU_I8: return "i8";
    case NPU_I32: return "i32";
    default: return "?";
  }
}

constexpr int64_t kMaxElems = (int64_t(1) << 31) - 1;

// Checks rank, dtype, row-major contiguity, 16-byte alignment and the
// element-count limit; returns the base device pointer in *ptr.
npu_status check_memref(const npu_memref *m, const char *name, int32_t rank, int32_t dtype,
                        const void **ptr) {
  if (!m) return fail(NPU_ERR_INVALID_ARG, "%s: null descriptor", name);
  if (m->rank != rank)
    return fail(NPU_ERR_INVALID_ARG, "%s: rank %d, expected %d", name, m->rank, rank);
  if (m->dtype != dtype)
    return fail(NPU_ERR_INVALID_ARG, "%s: dtype %s, expected %s", name, dtype_name(m->dtype),
                dtype_name(dtype));
  if (!m->aligned) return fail(NPU_ERR_INVALID_ARG, "%s: null data pointer", name);
  if (m->offset < 0) return fail(NPU_ERR_INVALID_ARG, "%s: negative offset", name);
  int64_t elems = 1, expect_stride = 1;
  for (int d = rank - 1; d >= 0; --d) {
    if (m->sizes[d] <= 0)
      return fail(NPU_ERR_INVALID_ARG, "%s: size[%d] = %lld must be positive", name, d,
                  (long long)m->sizes[d]);
    if (m->sizes[d] > 1 && m->strides[d] != expect_stride)
      return fail(NPU_ERR_UNSUPPORTED, "%s: stride[%d] = %lld, only row-major contiguous is "
                  "supported (expected %lld)", name, d, (long long)m->strides[d],
                  (long long)expect_stride);
    expect_stride *= m->sizes[d];
    elems *= m->sizes[d];
    if (elems > kMaxElems)
      return fail(NPU_ERR_UNSUPPORTED, "%s: more than 2^31-1 elements", name);
  }
  const char *base = static_cast<const char *>(m->aligned) + m->offset * dtype_size(dtype);
  if (reinterpret_cast<uintptr_t>(base) % 16 != 0)
    return fail(NPU_ERR_UNSUPPORTED, "%s: data pointer is not 16-byte aligned", name);
  *ptr = base;
  return NPU_OK;
}

}  // namespace

namespace npu {
npu_status memref_check(const npu_memref *m, const char *name, int32_t rank, int32_t dtype) {
  const void *p;
  return check_memref(m, name, rank, dtype, &p);
}
}  // namespace npu

namespace {

// An optional operand: a null descriptor or a null data pointer means absent.
bool absent(const npu_memref *m) { return !m || !m->aligned; }

npu_status check_act(int32_t act) {
  if (act < NPU_ACT_NONE || act > NPU_ACT_RELU6)
    return fail(NPU_ERR_INVALID_ARG, "act %d is not one of NONE/RELU/RELU6", act);
  return NPU_OK;
}

npu_status hip_status(hipError_t e, const char *what) {
  if (e != hipSuccess) return fail(NPU_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return ok();
}

#define NPU_TRY(expr)                 \
  do {                                \
    npu_status _s = (expr);           \
    if (_s != NPU_OK) return _s;      \
  } while (0)

}  // namespace

extern "C" {

const char *npu_version(void) { return "npu-mi355x 0.1 (gfx950)"; }

const char *npu_last_error(void) { return g_last_error.c_str(); }

const char *npu_status_string(npu_status s) {
  switch (s) {
    case NPU_OK: return "ok";
    case NPU_ERR_INVALID_ARG: return "invalid argument";
    case NPU_ERR_UNSUPPORTED: return "unsupported";
    case NPU_ERR_HIP: return "HIP error";
    case NPU_ERR_OOM: return "out of memory";
    default: return "unknown status";
  }
}

int32_t npu_last_launch_plans(npu_launch_plan *plans, int32_t max_plans) {
  const int32_t n = (int32_t)npu::g_plans.size();
  for (int32_t i = 0; i < n && i < max_plans && plans; ++i) plans[i] = npu::g_plans[i];
  return n;
}

int32_t npu_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return -1;
  return n;
}

npu_status fused_matmul_bias_act(const npu_memref *A, const npu_memref *B,
                                 const npu_memref *bias, const npu_memref *out, int32_t act,
                                 npu_stream stream) {
  npu::plans_reset();
  const void *pa, *pb, *pbias = nullptr, *po;
  NPU_TRY(check_memref(A, "A", 2, NPU_F32, &pa));
  NPU_TRY(check_memref(B, "B", 2, NPU_F32, &pb));
  NPU_TRY(check_memref(out, "out", 2, NPU_F32, &po));
  NPU_TRY(check_act(act));
  const int64_t M = A->sizes[0], K = A->sizes[1], N = B->sizes[1];
  if (B->sizes[0] != K)
    return fail(NPU_ERR_INVALID_ARG, "B: sizes[0] = %lld, expected K = %lld",
                (long long)B->sizes[0], (long long)K);
  if (out->sizes[0] != M || out->sizes[1] != N)
    return fail(NPU_ERR_INVALID_ARG, "out: [%lld,%lld], expected [%lld,%lld]",
                (long long)out->sizes[0], (long long)out->sizes[1], (long long)M, (long long)N);
  if (!absent(bias)) {
    NPU_TRY(check_memref(bias, "bias", 1, NPU_F32, &pbias));
    if (bias->sizes[0] != N)
      return fail(NPU_ERR_INVALID_ARG, "bias: size %lld, expected N = %lld",
                  (long long)bias->sizes[0], (long long)N);
  }
  if (K % 4 != 0) return fail(NPU_ERR_UNSUPPORTED, "K = %lld must be a multiple of 4", (long long)K);
  npu::MatmulArgs a{static_cast<const float *>(pa), static_cast<const float *>(pb),
                    static_cast<const float *>(pbias), const_cast<float *>(static_cast<const float *>(po)),
                    (int)M, (int)N, (int)K, act};
  return hip_status(npu::launch_matmul_bias_act_f32(a, static_cast<hipStream_t>(stream)),
                    "fused_matmul_bias_act launch");
}

npu_status npu_planned_matmul_bias_act(const npu_memref *A, const npu_memref *B,
                                       const npu_memref *bias, const npu_memref *out,
                                       int32_t act, const npu_tile_plan *plan, void *lds_dump,
                                       npu_stream stream) {
  npu::plans_reset();
  const void *pa, *pb, *pbias = nullptr, *po;
  NPU_TRY(check_memref(A, "A", 2, NPU_F32, &pa));
  NPU_TRY(check_memref(B, "B", 2, NPU_F32, &pb));
  NPU_TRY(check_memref(out, "out", 2, NPU_F32, &po));
  NPU_TRY(check_act(act));
  const int64_t M = A->sizes[0], K = A->sizes[1], N = B->sizes[1];
  if (B->sizes[0] != K)
    return fail(NPU_ERR_INVALID_ARG, "B: sizes[0] = %lld, expected K = %lld",
                (long long)B->sizes[0], (long long)K);
  if (out->sizes[0] != M || out->sizes[1] != N)
    return fail(NPU_ERR_INVALID_ARG, "out: [%lld,%lld], expected [%lld,%lld]",
                (long long)out->sizes[0], (long long)out->sizes[1], (long long)M, (long long)N);
  if (!absent(bias)) {
    NPU_TRY(check_memref(bias, "bias", 1, NPU_F32, &pbias));
    if (bias->sizes[0] != N)
      return fail(NPU_ERR_INVALID_ARG, "bias: size %lld, expected N = %lld",
                  (long long)bias->sizes[0], (long long)N);
  }
  if (!plan) return fail(NPU_ERR_INVALID_ARG, "plan is NULL");
  const npu_tile_plan &p = *plan;
  if (!npu::planned_matmul_tiles_ok(p.tm, p.tn, p.tk))
    return fail(NPU_ERR_UNSUPPORTED,
                "tile (%d, %d, %d): sizes must be positive with at most 64 16x16 output blocks",
                p.tm, p.tn, p.tk);
  if (p.lds_bytes <= 0 || p.lds_bytes > 163840 || p.lds_bytes % 4 != 0)
    return fail(NPU_ERR_INVALID_ARG, "lds_bytes = %d: must be in (0, 163840], a multiple of 4",
                p.lds_bytes);
  struct Buf {
    const char *name;
    int64_t off, bytes;
  };
  const int64_t t = 4;
  const Buf bufs[7] = {{"A", p.off_a, t * p.tm * p.tk},     {"A pong", p.off_a_pong, t * p.tm * p.tk},
                       {"B", p.off_b, t * p.tk * p.tn},     {"B pong", p.off_b_pong, t * p.tk * p.tn},
                       {"bias", p.off_bias, t * p.tn},       {"C", p.off_c, t * p.tm * p.tn},
                       {"Y", p.off_y, t * p.tm * p.tn}};
  // a plan without a bias buffer (off_bias < 0) is for a group without a bias
  const bool has_bias = p.off_bias >= 0;
  if (has_bias != (pbias != nullptr))
    return fail(NPU_ERR_INVALID_ARG, has_bias ? "plan has a bias buffer but bias is absent"
                                              : "bias given but the plan has no bias buffer");
  const int nbufs = 7;
  for (int i = 0; i < nbufs; ++i) {
    const Buf &b = bufs[i];
    if (i == 4 && !has_bias) continue;
    if (b.off < 0 || b.off % 4 != 0 || b.off + b.bytes > p.lds_bytes)
      return fail(NPU_ERR_INVALID_ARG,
                  "plan: %s at %lld (+%lld bytes) is not a 4-byte aligned offset inside the %d "
                  "bytes of SRAM", b.name, (long long)b.off, (long long)b.bytes, p.lds_bytes);
  }
  for (int i = 0; i < nbufs; ++i)
    for (int j = i + 1; j < nbufs; ++j)
      if ((has_bias || (i != 4 && j != 4)) && bufs[i].off < bufs[j].off + bufs[j].bytes && bufs[j].off < bufs[i].off + bufs[i].bytes)
        return fail(NPU_ERR_INVALID_ARG, "plan: %s and %s overlap", bufs[i].name, bufs[j].name);
  npu::PlannedMatmulArgs a{};
  a.A = static_cast<const float *>(pa);
  a.B = static_cast<const float *>(pb);
  a.bias = static_cast<const float *>(pbias);
  a.out = static_cast<float *>(const_cast<void *>(po));
  a.M = (int)M; a.N = (int)N; a.K = (int)K; a.act = act;
  a.tm = p.tm; a.tn = p.tn; a.tk = p.tk; a.lds_bytes = p.lds_bytes;
  a.off_a[0] = (int)p.off_a; a.off_a[1] = (int)p.off_a_pong;
  a.off_b[0] = (int)p.off_b; a.off_b[1] = (int)p.off_b_pong;
  a.off_bias = has_bias ? (int)p.off_bias : -1; a.off_c = (int)p.off_c; a.off_y = (int)p.off_y;
  a.lds_dump = lds_dump;
  return hip_status(npu::launch_planned_matmul(a, static_cast<hipStream_t>(stream)),
                    "npu_planned_matmul_bias_act launch");
}

npu_status npu_planned_conv2d_nchw_bias_act(const npu_memref *x, const npu_memref *w,
                                            const npu_memref *bias, const npu_memref *out,
                                            int32_t act, const npu_conv_tile_plan *plan,
                                            void *lds_dump, npu_stream stream) {
  npu::plans_reset();
  const void *px, *pw, *pbias = nullptr, *po;
  NPU_TRY(check_memref(x, "x", 4, NPU_F32, &px));
  NPU_TRY(check_memref(w, "w", 4, NPU_F32, &pw));
  NPU_TRY(check_memref(out, "out", 4, NPU_F32, &po));
  NPU_TRY(check_act(act));
  const int64_t N = x->sizes[0], C = x->sizes[1], Hp = x->sizes[2], Wp = x->sizes[3];
  const int64_t F = w->sizes[0], KH = w->sizes[2], KW = w->sizes[3];
  if (w->sizes[1] != C)
    return fail(NPU_ERR_INVALID_ARG, "w: sizes[1] = %lld, expected C = %lld",
                (long long)w->sizes[1], (long long)C);
  if (KH > Hp || KW > Wp)
    return fail(NPU_ERR_INVALID_ARG, "w: %lldx%lld filter larger than the %lldx%lld input",
                (long long)KH, (long long)KW, (long long)Hp, (long long)Wp);
  const int64_t Ho = Hp - KH + 1, Wo = Wp - KW + 1;
  if (out->sizes[0] != N || out->sizes[1] != F || out->sizes[2] != Ho || out->sizes[3] != Wo)
    return fail(NPU_ERR_INVALID_ARG, "out: [%lld,%lld,%lld,%lld], expected [%lld,%lld,%lld,%lld]",
                (long long)out->sizes[0], (long long)out->sizes[1], (long long)out->sizes[2],
                (long long)out->sizes[3], (long long)N, (long long)F, (long long)Ho, (long long)Wo);
  if (!absent(bias)) {
    NPU_TRY(check_memref(bias, "bias", 1, NPU_F32, &pbias));
    if (bias->sizes[0] != F)
      return fail(NPU_ERR_INVALID_ARG, "bias: size %lld, expected F = %lld",
                  (long long)bias->sizes[0], (long long)F);
  }
  if (!plan) return fail(NPU_ERR_INVALID_ARG, "plan is NULL");
  const npu_conv_tile_plan &p = *plan;
  if (p.tco < 1 || p.tco > F)
    return fail(NPU_ERR_INVALID_ARG, "plan: tco = %d, expected 1 .. F = %lld", p.tco, (long long)F);
  if (p.lds_bytes <= 0 || p.lds_bytes > 163840 || p.lds_bytes % 4 != 0)
    return fail(NPU_ERR_INVALID_ARG, "lds_bytes = %d: must be in (0, 163840], a multiple of 4",
                p.lds_bytes);
  struct Buf {
    const char *name;
    int64_t off, bytes;
  };
  const int64_t t = 4, in_b = t * C * KH * Wp, w_b = t * p.tco * C * KH * KW, row_b = t * p.tco * Wo;
  constexpr int kBufs = 11;
  const Buf bufs[kBufs] = {{"input rows", p.off_in, in_b}, {"input rows pong", p.off_in_pong, in_b},
                           {"input rows prefetch", p.off_in_prefetch, in_b},
                           {"filters", p.off_w, w_b}, {"filters pong", p.off_w_pong, w_b},
                           {"filters prefetch", p.off_w_prefetch, w_b},
                           {"bias", p.off_bias, t * p.tco}, {"bias pong", p.off_bias_pong, t * p.tco},
                           {"bias prefetch", p.off_bias_prefetch, t * p.tco},
                           {"C", p.off_c, row_b}, {"Y", p.off_y, row_b}};
  const bool has_bias = p.off_bias >= 0;
  if (has_bias != (pbias != nullptr))
    return fail(NPU_ERR_INVALID_ARG, has_bias ? "plan has a bias buffer but bias is absent"
                                              : "bias given but the plan has no bias buffer");
  // -1: the buffer is not in SRAM (a spilled input, no pong, no prefetch
  // region, no bias); C and Y must be in SRAM, and a buffer not in SRAM has
  // neither a pong nor a prefetch region
  if (p.off_c < 0 || p.off_y < 0) return fail(NPU_ERR_INVALID_ARG, "plan: C and Y must be in SRAM");
  if ((p.off_in < 0 && (p.off_in_pong >= 0 || p.off_in_prefetch >= 0)) ||
      (p.off_w < 0 && (p.off_w_pong >= 0 || p.off_w_prefetch >= 0)) ||
      (p.off_bias < 0 && (p.off_bias_pong >= 0 || p.off_bias_prefetch >= 0)))
    return fail(NPU_ERR_INVALID_ARG, "plan: a buffer outside SRAM with a pong or prefetch buffer");
  auto used = [&](int i) { return bufs[i].off >= 0; };
  for (int i = 0; i < kBufs; ++i) {
    if (!used(i)) continue;
    const Buf &b = bufs[i];
    if (b.off % 4 != 0 || b.off + b.bytes > p.lds_bytes)
      return fail(NPU_ERR_INVALID_ARG,
                  "plan: %s at %lld (+%lld bytes) is not a 4-byte aligned offset inside the %d "
                  "bytes of SRAM", b.name, (long long)b.off, (long long)b.bytes, p.lds_bytes);
  }
  for (int i = 0; i < kBufs; ++i)
    for (int j = i + 1; j < kBufs; ++j)
      if (used(i) && used(j) && bufs[i].off < bufs[j].off + bufs[j].bytes &&
          bufs[j].off < bufs[i].off + bufs[i].bytes)
        return fail(NPU_ERR_INVALID_ARG, "plan: %s and %s overlap", bufs[i].name, bufs[j].name);
  npu::PlannedConvArgs a{};
  a.x = static_cast<const float *>(px);
  a.w = static_cast<const float *>(pw);
  a.bias = static_cast<const float *>(pbias);
  a.out = static_cast<float *>(const_cast<void *>(po));
  a.N = (int)N; a.C = (int)C; a.Hp = (int)Hp; a.Wp = (int)Wp; a.F = (int)F;
  a.KH = (int)KH; a.KW = (int)KW; a.Ho = (int)Ho; a.Wo = (int)Wo; a.act = act;
  a.tco = p.tco; a.lds_bytes = p.lds_bytes;
  a.off_in[0] = (int)p.off_in; a.off_in[1] = (int)p.off_in_pong;
  a.off_w[0] = (int)p.off_w; a.off_w[1] = (int)p.off_w_pong;
  a.off_in_pre = (int)p.off_in_prefetch; a.off_w_pre = (int)p.off_w_prefetch;
  a.off_bias[0] = (int)p.off_bias; a.off_bias[1] = (int)p.off_bias_pong;
  a.off_bias_pre = (int)p.off_bias_prefetch;
  a.off_c = (int)p.off_c; a.off_y = (int)p.off_y;
  a.lds_dump = lds_dump;
  return hip_status(npu::launch_planned_conv(a, static_cast<hipStream_t>(stream)),
                    "npu_planned_conv2d_nchw_bias_act launch");
}

namespace {

// fused_conv2d_nhwc_bias_act and its residual variant: checks, then the LDS
// halo kernel for 3x3 / pad 1 rows of at most 64 pixels without a residual,
// the implicit-GEMM kernel otherwise.
npu_status conv_entry(const npu_memref *x, const npu_memref *w, const npu_memref *bias,
                      const npu_memref *res, const npu_memref *out, int32_t pad, int32_t act,
                      npu_stream stream, const char *name) {
  npu::plans_reset();
  if (!x) return fail(NPU_ERR_INVALID_ARG, "x: null descriptor");
  const int32_t dt = x->dtype;
  if (dt != NPU_F32 && dt != NPU_BF16)
    return fail(NPU_ERR_UNSUPPORTED, "x: dtype %s, expected f32 or bf16", dtype_name(dt));
  const void *px, *pw, *pbias = nullptr, *pres = nullptr, *po;
  NPU_TRY(check_memref(x, "x", 4, dt, &px));
  NPU_TRY(check_memref(w, "w", 4, dt, &pw));
  NPU_TRY(check_memref(out, "out", 4, dt, &po));
  NPU_TRY(check_act(act));
  const int64_t N = x->sizes[0], H = x->sizes[1], W = x->sizes[2], C = x->sizes[3];
  const int64_t F = w->sizes[0], KH = w->sizes[1], KW = w->sizes[2];
  if (w->sizes[3] != C)
    return fail(NPU_ERR_INVALID_ARG, "w: channels %lld, expected C = %lld",
                (long long)w->sizes[3], (long long)C);
  if (pad < 0) return fail(NPU_ERR_INVALID_ARG, "pad %d is negative", pad);
  const int64_t Ho = H + 2 * pad - KH + 1, Wo = W + 2 * pad - KW + 1;
  if (Ho <= 0 || Wo <= 0) return fail(NPU_ERR_INVALID_ARG, "empty output (%lld x %lld)",
                                      (long long)Ho, (long long)Wo);
  if (out->sizes[0] != N || out->sizes[1] != Ho || out->sizes[2] != Wo || out->sizes[3] != F)
    return fail(NPU_ERR_INVALID_ARG, "out: [%lld,%lld,%lld,%lld], expected [%lld,%lld,%lld,%lld]",
                (long long)out->sizes[0], (long long)out->sizes[1], (long long)out->sizes[2],
                (long long)out->sizes[3], (long long)N, (long long)Ho, (long long)Wo,
                (long long)F);
  if (!absent(bias)) {
    NPU_TRY(check_memref(bias, "bias", 1, NPU_F32, &pbias));
    if (bias->sizes[0] != F)
      return fail(NPU_ERR_INVALID_ARG, "bias: size %lld, expected F = %lld",
                  (long long)bias->sizes[0], (long long)F);
  }
  if (res) {
    NPU_TRY(check_memref(res, "res", 4, dt, &pres));
    for (int d = 0; d < 4; ++d)
      if (res->sizes[d] != out->sizes[d])
        return fail(NPU_ERR_INVALID_ARG, "res: [%lld,%lld,%lld,%lld], expected the output's shape",
                    (long long)res->sizes[0], (long long)res->sizes[1], (long long)res->sizes[2],
                    (long long)res->sizes[3]);
  }
  // a lane's operand is one 16-byte run of channels: 4 f32 or 8 bf16
  const int64_t cstep = dt == NPU_F32 ? 4 : 8;
  if (C % cstep != 0)
    return fail(NPU_ERR_UNSUPPORTED, "C = %lld must be a multiple of %lld for %s", (long long)C,
                (long long)cstep, dtype_name(dt));
  npu::ConvArgs a{px, pw, static_cast<const float *>(pbias), const_cast<void *>(po),
                  (int)N, (int)H, (int)W, (int)C, (int)F, (int)KH, (int)KW, pad,
                  (int)Ho, (int)Wo, act, pres};
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  if (!pres && npu::conv3x3_rows_supported(a, dt == NPU_F32 ? 4 : 2))
    e = dt == NPU_F32 ? npu::launch_conv3x3_f32(a, s) : npu::launch_conv3x3_bf16(a, s);
  else
    e = dt == NPU_F32 ? npu::launch_conv2d_nhwc_f32(a, s) : npu::launch_conv2d_nhwc_bf16(a, s);
  return hip_status(e, name);
}

}  // namespace

npu_status fused_conv2d_nhwc_bias_act(const npu_memref *x, const npu_memref *w,
                                      const npu_memref *bias, const npu_memref *out,
                                      int32_t pad, int32_t act, npu_stream stream) {
  return conv_entry(x, w, bias, nullptr, out, pad, act, stream,
                    "fused_conv2d_nhwc_bias_act launch");
}

npu_status fused_conv2d_nhwc_bias_res_act(const npu_memref *x, const npu_memref *w,
                                          const npu_memref *bias, const npu_memref *res,
                                          const npu_memref *out, int32_t pad, int32_t act,
                                          npu_stream stream) {
  if (!res) return fail(NPU_ERR_INVALID_ARG, "res: null descriptor");
  return conv_entry(x, w, bias, res, out, pad, act, stream,
                    "fused_conv2d_nhwc_bias_res_act launch");
}

namespace {

// fused_conv2d_nchw_bias_act and its residual variant.
npu_status conv_nchw_entry(const npu_memref *x, const npu_memref *w, const npu_memref *bias,
                           const npu_memref *res, const npu_memref *out, int32_t pad,
                           int32_t stride, int32_t act, npu_stream stream, const char *name) {
  npu::plans_reset();
  const void *px, *pw, *pbias = nullptr, *pres = nullptr, *po;
  NPU_TRY(check_memref(x, "x", 4, NPU_F32, &px));
  NPU_TRY(check_memref(w, "w", 4, NPU_F32, &pw));
  NPU_TRY(check_memref(out, "out", 4, NPU_F32, &po));
  NPU_TRY(check_act(act));
  const int64_t N = x->sizes[0], C = x->sizes[1], H = x->sizes[2], W = x->sizes[3];
  const int64_t F = w->sizes[0], KH = w->sizes[2], KW = w->sizes[3];
  if (w->sizes[1] != C)
    return fail(NPU_ERR_INVALID_ARG, "w: channels %lld, expected C = %lld",
                (long long)w->sizes[1], (long long)C);
  if (pad < 0) return fail(NPU_ERR_INVALID_ARG, "pad %d is negative", pad);
  if (stride < 1) return fail(NPU_ERR_INVALID_ARG, "stride %d must be positive", stride);
  if (H + 2 * pad < KH || W + 2 * pad < KW)
    return fail(NPU_ERR_INVALID_ARG, "filter %lldx%lld larger than the padded input",
                (long long)KH, (long long)KW);
  const int64_t Ho = (H + 2 * pad - KH) / stride + 1, Wo = (W + 2 * pad - KW) / stride + 1;
  if (out->sizes[0] != N || out->sizes[1] != F || out->sizes[2] != Ho || out->sizes[3] != Wo)
    return fail(NPU_ERR_INVALID_ARG, "out: [%lld,%lld,%lld,%lld], expected [%lld,%lld,%lld,%lld]",
                (long long)out->sizes[0], (long long)out->sizes[1], (long long)out->sizes[2],
                (long long)out->sizes[3], (long long)N, (long long)F, (long long)Ho,
                (long long)Wo);
  if (!absent(bias)) {
    NPU_TRY(check_memref(bias, "bias", 1, NPU_F32, &pbias));
    if (bias->sizes[0] != F)
      return fail(NPU_ERR_INVALID_ARG, "bias: size %lld, expected F = %lld",
                  (long long)bias->sizes[0], (long long)F);
  }
  if (res) {
    NPU_TRY(check_memref(res, "res", 4, NPU_F32, &pres));
    for (int d = 0; d < 4; ++d)
      if (res->sizes[d] != out->sizes[d])
        return fail(NPU_ERR_INVALID_ARG, "res: [%lld,%lld,%lld,%lld], expected the output's shape",
                    (long long)res->sizes[0], (long long)res->sizes[1], (long long)res->sizes[2],
                    (long long)res->sizes[3]);
  }
  npu::ConvArgs a{px, pw, static_cast<const float *>(pbias), const_cast<void *>(po),
                  (int)N, (int)H, (int)W, (int)C, (int)F, (int)KH, (int)KW, pad,
                  (int)Ho, (int)Wo, act, pres, stride};
  return hip_status(npu::launch_conv2d_nchw_f32(a, static_cast<hipStream_t>(stream)), name);
}

}  // namespace

npu_status fused_conv2d_nchw_bias_act(const npu_memref *x, const npu_memref *w,
                                      const npu_memref *bias, const npu_memref *out,
                                      int32_t pad, int32_t stride, int32_t act,
                                      npu_stream stream) {
  return conv_nchw_entry(x, w, bias, nullptr, out, pad, stride, act, stream,
                         "fused_conv2d_nchw_bias_act launch");
}

npu_status fused_conv2d_nchw_bias_res_act(const npu_memref *x, const npu_memref *w,
                                          const npu_memref *bias, const npu_memref *res,
                                          const npu_memref *out, int32_t pad, int32_t stride,
                                          int32_t act, npu_stream stream) {
  if (!res) return fail(NPU_ERR_INVALID_ARG, "res: null descriptor");
  return conv_nchw_entry(x, w, bias, res, out, pad, stride, act, stream,
                         "fused_conv2d_nchw_bias_res_act launch");
}

npu_status fused_qbottleneck_i8(const npu_memref *x, const npu_memref *w1,
                                const npu_memref *w2, const npu_memref *w3,
                                const npu_memref *m1, const npu_memref *s1,
                                const npu_memref *m2, const npu_memref *s2,
                                const npu_memref *m3, const npu_memref *s3,
                                const npu_memref *out, npu_stream stream) {
  npu::plans_reset();
  const void *px, *pw1, *pw2, *pw3, *pm1, *ps1, *pm2, *ps2, *pm3, *ps3, *po;
  NPU_TRY(check_memref(x, "x", 4, NPU_I8, &px));
  const int64_t N = x->sizes[0], H = x->sizes[1], W = x->sizes[2], C = x->sizes[3];
  NPU_TRY(check_memref(w1, "w1", 2, NPU_I8, &pw1));
  const int64_t M1 = w1->sizes[0];
  if (w1->sizes[1] != C)
    return fail(NPU_ERR_INVALID_ARG, "w1: [%lld,%lld], expected [M1,%lld]",
                (long long)w1->sizes[0], (long long)w1->sizes[1], (long long)C);
  NPU_TRY(check_memref(w2, "w2", 4, NPU_I8, &pw2));
  if (w2->sizes[0] != M1 || w2->sizes[1] != 3 || w2->sizes[2] != 3 || w2->sizes[3] != M1)
    return fail(NPU_ERR_INVALID_ARG, "w2: expected [%lld,3,3,%lld]", (long long)M1,
                (long long)M1);
  NPU_TRY(check_memref(w3, "w3", 2, NPU_I8, &pw3));
  if (w3->sizes[0] != C || w3->sizes[1] != M1)
    return fail(NPU_ERR_INVALID_ARG, "w3: expected [%lld,%lld]", (long long)C, (long long)M1);
  const npu_memref *qm[6] = {m1, s1, m2, s2, m3, s3};
  const char *qn[6] = {"m1", "s1", "m2", "s2", "m3", "s3"};
  const void **qp[6] = {&pm1, &ps1, &pm2, &ps2, &pm3, &ps3};
  for (int i = 0; i < 6; ++i) {
    NPU_TRY(check_memref(qm[i], qn[i], 1, NPU_I32, qp[i]));
    const int64_t want = i < 4 ? M1 : C;
    if (qm[i]->sizes[0] != want)
      return fail(NPU_ERR_INVALID_ARG, "%s: size %lld, expected %lld", qn[i],
                  (long long)qm[i]->sizes[0], (long long)want);
  }
  NPU_TRY(check_memref(out, "out", 4, NPU_I8, &po));
  for (int d = 0; d < 4; ++d)
    if (out->sizes[d] != x->sizes[d])
      return fail(NPU_ERR_INVALID_ARG, "out: size[%d] = %lld, expected %lld", d,
                  (long long)out->sizes[d], (long long)x->sizes[d]);
  if (!npu::qbottleneck_supported((int)C, (int)M1))
    return fail(NPU_ERR_UNSUPPORTED,
                "(C, M1) = (%lld, %lld): C must be a multiple of 64 up to 2048, M1 up to 512",
                (long long)C, (long long)M1);
  npu::QBottleneckArgs a{static_cast<const int8_t *>(px), static_cast<const int8_t *>(pw1),
                         static_cast<const int8_t *>(pw2), static_cast<const int8_t *>(pw3),
                         static_cast<const int32_t *>(pm1), static_cast<const int32_t *>(ps1),
                         static_cast<const int32_t *>(pm2), static_cast<const int32_t *>(ps2),
                         static_cast<const int32_t *>(pm3), static_cast<const int32_t *>(ps3),
                         const_cast<int8_t *>(static_cast<const int8_t *>(po)),
                         (int)N, (int)H, (int)W, (int)C, (int)M1};
  return hip_status(npu::launch_qbottleneck_i8(a, static_cast<hipStream_t>(stream)),
                    "fused_qbottleneck_i8 launch");
}

npu_status fused_irb_f32(const npu_memref *x, const npu_memref *we, const npu_memref *wdw,
                         const npu_memref *wp, const npu_memref *out, npu_stream stream) {
  npu::plans_reset();
  const void *px, *pwe, *pwdw, *pwp, *po;
  NPU_TRY(check_memref(x, "x", 4, NPU_F32, &px));
  const int64_t N = x->sizes[0], H = x->sizes[1], W = x->sizes[2], C = x->sizes[3];
  NPU_TRY(check_memref(we, "we", 2, NPU_F32, &pwe));
  const int64_t E = we->sizes[0];
  if (we->sizes[1] != C)
    return fail(NPU_ERR_INVALID_ARG, "we: [%lld,%lld], expected [E,%lld]",
                (long long)we->sizes[0], (long long)we->sizes[1], (long long)C);
  NPU_TRY(check_memref(wdw, "wdw", 3, NPU_F32, &pwdw));
  if (wdw->sizes[0] != 3 || wdw->sizes[1] != 3 || wdw->sizes[2] != E)
    return fail(NPU_ERR_INVALID_ARG, "wdw: expected [3,3,%lld]", (long long)E);
  NPU_TRY(check_memref(wp, "wp", 2, NPU_F32, &pwp));
  if (wp->sizes[0] != C || wp->sizes[1] != E)
    return fail(NPU_ERR_INVALID_ARG, "wp: expected [%lld,%lld]", (long long)C, (long long)E);
  NPU_TRY(check_memref(out, "out", 4, NPU_F32, &po));
  for (int d = 0; d < 4; ++d)
    if (out->sizes[d] != x->sizes[d])
      return fail(NPU_ERR_INVALID_ARG, "out: size[%d] = %lld, expected %lld", d,
                  (long long)out->sizes[d], (long long)x->sizes[d]);
  if (!npu::irb_supported((int)C, (int)E))
    return fail(NPU_ERR_UNSUPPORTED,
                "(C, E) = (%lld, %lld): C must be a multiple of 4 in [4, 320] and E of 16",
                (long long)C, (long long)E);
  npu::IrbArgs a{static_cast<const float *>(px), static_cast<const float *>(pwe),
                 static_cast<const float *>(pwdw), static_cast<const float *>(pwp),
                 const_cast<float *>(static_cast<const float *>(po)), (int)N, (int)H, (int)W,
                 (int)C, (int)E};
  return hip_status(npu::launch_irb_f32(a, static_cast<hipStream_t>(stream)),
                    "fused_irb_f32 launch");
}

}  // extern "C"

namespace {

// A 2-D operand of exactly [d0, d1].
npu_status check_2d(const npu_memref *m, const char *name, int32_t dtype, int64_t d0, int64_t d1,
                    const void **ptr) {
  NPU_TRY(check_memref(m, name, 2, dtype, ptr));
  if (m->sizes[0] != d0 || m->sizes[1] != d1)
    return fail(NPU_ERR_INVALID_ARG, "%s: [%lld,%lld], expected [%lld,%lld]", name,
                (long long)m->sizes[0], (long long)m->sizes[1], (long long)d0, (long long)d1);
  return NPU_OK;
}

npu_status check_1d(const npu_memref *m, const char *name, int32_t dtype, int64_t d0,
                    const void **ptr) {
  NPU_TRY(check_memref(m, name, 1, dtype, ptr));
  if (m->sizes[0] != d0)
    return fail(NPU_ERR_INVALID_ARG, "%s: size %lld, expected %lld", name,
                (long long)m->sizes[0], (long long)d0);
  return NPU_OK;
}

npu_status check_gemm_dims(int64_t S, int64_t K, int64_t N) {
  (void)S;  // any sequence length: rows past S are clamped on load and not stored
  if (K % 64 != 0) return fail(NPU_ERR_UNSUPPORTED, "K = %lld must be a multiple of 64", (long long)K);
  if (N % 64 != 0) return fail(NPU_ERR_UNSUPPORTED, "N = %lld must be a multiple of 64", (long long)N);
  return NPU_OK;
}

npu_status check_eps(float eps) {
  if (!(eps >= 0.0f)) return fail(NPU_ERR_INVALID_ARG, "eps must be >= 0");
  return NPU_OK;
}

const uint16_t *u16(const void *p) { return static_cast<const uint16_t *>(p); }
uint16_t *u16w(const void *p) { return const_cast<uint16_t *>(static_cast<const uint16_t *>(p)); }

}  // namespace

extern "C" {

npu_status fused_llama_qkv_rope(const npu_memref *x, const npu_memref *g1, const npu_memref *wq,
                                const npu_memref *wk, const npu_memref *wv,
                                const npu_memref *cos_t, const npu_memref *sin_t,
                                const npu_memref *Q, const npu_memref *K, const npu_memref *V,
                                float eps, npu_stream stream) {
  npu::plans_reset();
  const void *px, *pg, *pq, *pk, *pv, *pc, *ps, *oq, *ok, *ov;
  NPU_TRY(check_memref(x, "x", 2, NPU_BF16, &px));
  const int64_t S = x->sizes[0], D = x->sizes[1];
  if (D % 64 != 0) return fail(NPU_ERR_UNSUPPORTED, "D = %lld must be a multiple of 64", (long long)D);
  NPU_TRY(check_1d(g1, "g1", NPU_F32, D, &pg));
  NPU_TRY(check_2d(wq, "wq", NPU_BF16, D, D, &pq));
  NPU_TRY(check_2d(wk, "wk", NPU_BF16, D, D, &pk));
  NPU_TRY(check_2d(wv, "wv", NPU_BF16, D, D, &pv));
  // the head dim is twice the RoPE tables' width: 64 or 128
  NPU_TRY(check_memref(cos_t, "cos_t", 2, NPU_F32, &pc));
  const int64_t half = cos_t->sizes[1];
  if (half != 32 && half != 64)
    return fail(NPU_ERR_UNSUPPORTED, "cos_t: %lld columns, expected 32 or 64 (head dim 64 or 128)",
                (long long)half);
  if (D % (2 * half) != 0)
    return fail(NPU_ERR_INVALID_ARG, "D = %lld is not a multiple of the head dim %lld",
                (long long)D, (long long)(2 * half));
  NPU_TRY(check_2d(cos_t, "cos_t", NPU_F32, S, half, &pc));
  NPU_TRY(check_2d(sin_t, "sin_t", NPU_F32, S, half, &ps));
  NPU_TRY(check_2d(Q, "Q", NPU_BF16, S, D, &oq));
  NPU_TRY(check_2d(K, "K", NPU_BF16, S, D, &ok));
  NPU_TRY(check_2d(V, "V", NPU_BF16, S, D, &ov));
  NPU_TRY(check_gemm_dims(S, D, D));
  NPU_TRY(check_eps(eps));
  npu::LlamaGemmArgs a{};
  a.A = u16(px);
  a.gamma = static_cast<const float *>(pg);
  a.eps = eps;
  a.B[0] = u16(pq); a.B[1] = u16(pk); a.B[2] = u16(pv);
  a.nparts = 3;
  a.M = (int)S; a.K = (int)D; a.Npart = (int)D; a.Dh = (int)(2 * half);
  a.cos_t = static_cast<const float *>(pc);
  a.sin_t = static_cast<const float *>(ps);
  a.out[0] = u16w(oq); a.out[1] = u16w(ok); a.out[2] = u16w(ov);
  return hip_status(npu::launch_llama_gemm(a, npu::kProRmsnorm, npu::kEpiQkvRope,
                                           static_cast<hipStream_t>(stream)),
                    "fused_llama_qkv_rope launch");
}

npu_status fused_llama_attention(const npu_memref *Q, const npu_memref *K, const npu_memref *V,
                                 const npu_memref *A, int32_t n_heads, float scale,
                                 npu_stream stream) {
  npu::plans_reset();
  const void *pq, *pk, *pv, *pa;
  NPU_TRY(check_memref(Q, "Q", 2, NPU_BF16, &pq));
  const int64_t S = Q->sizes[0], D = Q->sizes[1];
  if (n_heads <= 0 || D % n_heads != 0 || (D / n_heads != 64 && D / n_heads != 128))
    return fail(NPU_ERR_UNSUPPORTED, "D = %lld must be n_heads * 64 or n_heads * 128 (n_heads = %d)",
                (long long)D, n_heads);
  const int dh = (int)(D / n_heads);
  NPU_TRY(check_2d(K, "K", NPU_BF16, S, D, &pk));
  NPU_TRY(check_2d(V, "V", NPU_BF16, S, D, &pv));
  NPU_TRY(check_2d(A, "A", NPU_BF16, S, D, &pa));
  if (!(scale > 0.0f)) return fail(NPU_ERR_INVALID_ARG, "scale must be positive");
  return hip_status(npu::launch_llama_attention(u16(pq), u16(pk), u16(pv), u16w(pa), (int)S,
                                                n_heads, dh, scale, static_cast<hipStream_t>(stream)),
                    "fused_llama_attention launch");
}

npu_status fused_llama_matmul_residual(const npu_memref *am, const npu_memref *w,
                                       const npu_memref *res, const npu_memref *out,
                                       npu_stream stream) {
  npu::plans_reset();
  const void *pa, *pw, *pr, *po;
  NPU_TRY(check_memref(am, "a", 2, NPU_BF16, &pa));
  const int64_t S = am->sizes[0], Kd = am->sizes[1];
  NPU_TRY(check_memref(w, "w", 2, NPU_BF16, &pw));
  const int64_t N = w->sizes[1];
  if (w->sizes[0] != Kd)
    return fail(NPU_ERR_INVALID_ARG, "w: sizes[0] = %lld, expected K = %lld",
                (long long)w->sizes[0], (long long)Kd);
  NPU_TRY(check_2d(res, "res", NPU_BF16, S, N, &pr));
  NPU_TRY(check_2d(out, "out", NPU_BF16, S, N, &po));
  NPU_TRY(check_gemm_dims(S, Kd, N));
  npu::LlamaGemmArgs a{};
  a.A = u16(pa);
  a.B[0] = a.B[1] = a.B[2] = u16(pw);
  a.nparts = 1;
  a.M = (int)S; a.K = (int)Kd; a.Npart = (int)N; a.Dh = 64;
  a.res = u16(pr);
  a.out[0] = a.out[1] = a.out[2] = u16w(po);
  return hip_status(npu::launch_llama_gemm(a, npu::kProPlain, npu::kEpiResidual,
                                           static_cast<hipStream_t>(stream)),
                    "fused_llama_matmul_residual launch");
}

npu_status fused_llama_rmsnorm_swiglu(const npu_memref *h, const npu_memref *g2,
                                      const npu_memref *wg, const npu_memref *wu,
                                      const npu_memref *act, float eps, npu_stream stream) {
  npu::plans_reset();
  const void *ph, *pg, *pwg, *pwu, *po;
  NPU_TRY(check_memref(h, "h", 2, NPU_BF16, &ph));
  const int64_t S = h->sizes[0], D = h->sizes[1];
  NPU_TRY(check_1d(g2, "g2", NPU_F32, D, &pg));
  NPU_TRY(check_memref(wg, "wg", 2, NPU_BF16, &pwg));
  const int64_t F = wg->sizes[1];
  if (wg->sizes[0] != D)
    return fail(NPU_ERR_INVALID_ARG, "wg: sizes[0] = %lld, expected D = %lld",
                (long long)wg->sizes[0], (long long)D);
  NPU_TRY(check_2d(wu, "wu", NPU_BF16, D, F, &pwu));
  NPU_TRY(check_2d(act, "act", NPU_BF16, S, F, &po));
  NPU_TRY(check_gemm_dims(S, D, F));
  if (D % 8 != 0) return fail(NPU_ERR_UNSUPPORTED, "D must be a multiple of 8");
  NPU_TRY(check_eps(eps));
  npu::LlamaGemmArgs a{};
  a.A = u16(ph);
  a.gamma = static_cast<const float *>(pg);
  a.eps = eps;
  a.B[0] = u16(pwg); a.B[1] = u16(pwu); a.B[2] = u16(pwu);
  a.nparts = 2;
  a.M = (int)S; a.K = (int)D; a.Npart = (int)F; a.Dh = 64;
  a.out[0] = a.out[1] = a.out[2] = u16w(po);
  return hip_status(npu::launch_llama_gemm(a, npu::kProRmsnorm, npu::kEpiSwiglu,
                                           static_cast<hipStream_t>(stream)),
                    "fused_llama_rmsnorm_swiglu launch");
}

}  // extern "C"
