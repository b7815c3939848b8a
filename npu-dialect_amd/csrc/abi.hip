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

namespace {

thread_local std::string g_last_error;

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

int32_t npu_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return -1;
  return n;
}

npu_status fused_matmul_bias_act(const npu_memref *A, const npu_memref *B,
                                 const npu_memref *bias, const npu_memref *out, int32_t act,
                                 npu_stream stream) {
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

npu_status fused_conv2d_nhwc_bias_act(const npu_memref *x, const npu_memref *w,
                                      const npu_memref *bias, const npu_memref *out,
                                      int32_t pad, int32_t act, npu_stream stream) {
  if (!x) return fail(NPU_ERR_INVALID_ARG, "x: null descriptor");
  const int32_t dt = x->dtype;
  if (dt != NPU_F32 && dt != NPU_BF16)
    return fail(NPU_ERR_UNSUPPORTED, "x: dtype %s, expected f32 or bf16", dtype_name(dt));
  const void *px, *pw, *pbias = nullptr, *po;
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
  const int64_t cstep = dt == NPU_F32 ? 16 : 32;
  if (C % cstep != 0)
    return fail(NPU_ERR_UNSUPPORTED, "C = %lld must be a multiple of %lld for %s", (long long)C,
                (long long)cstep, dtype_name(dt));
  if (F % 16 != 0)
    return fail(NPU_ERR_UNSUPPORTED, "F = %lld must be a multiple of 16", (long long)F);
  npu::ConvArgs a{px, pw, static_cast<const float *>(pbias), const_cast<void *>(po),
                  (int)N, (int)H, (int)W, (int)C, (int)F, (int)KH, (int)KW, pad,
                  (int)Ho, (int)Wo, act};
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e = dt == NPU_F32 ? npu::launch_conv2d_nhwc_f32(a, s)
                               : npu::launch_conv2d_nhwc_bf16(a, s);
  return hip_status(e, "fused_conv2d_nhwc_bias_act launch");
}

}  // extern "C"
