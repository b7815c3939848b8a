/*
 * npu_oracle.c -- TEST INFRASTRUCTURE: the checker, never the product.
 *
 * CPU restatement of the reference's "lower linalg to loops, run on the
 * CPU" execution (tools/harness/e2e_verify.py:232-251).  Single-threaded
 * (libnpu_oracle.so), built with -O2 -ffp-contract=off and without fast-math
 * so every
 * arith.mulf / arith.addf is its own IEEE-754 binary32 operation, as the
 * scalar code that convert-linalg-to-loops + convert-arith-to-llvm produce.
 * The `omp parallel for` pragmas split only the outer parallel loops of a
 * nest: each output element is still computed by one thread in the same
 * order, so the OpenMP build (libnpu_oracle_omp.so, the all-cores CPU
 * baseline) returns the same bits as the single-threaded one.
 * See npu_oracle.h for the op forms and the parity status of each function.
 */
#include "npu_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* bf16 <-> f32 (arith.truncf rounds to nearest even; extf is exact)         */
/* ------------------------------------------------------------------------ */
static inline float bf2f(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static inline uint16_t f2bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu))
    return (uint16_t)((u >> 16) | 0x0040u); /* quiet NaN */
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

void orc_trunc_f32_bf16(const float *in, uint16_t *out, int64_t n) {
  #pragma omp parallel for
  for (int64_t i = 0; i < n; ++i) out[i] = f2bf(in[i]);
}
void orc_ext_bf16_f32(const uint16_t *in, float *out, int64_t n) {
  #pragma omp parallel for
  for (int64_t i = 0; i < n; ++i) out[i] = bf2f(in[i]);
}

/* arith.maximumf / arith.minimumf propagate NaN. */
static inline float maximumf(float a, float b) {
  if (a != a || b != b) return NAN;
  return a > b ? a : b;
}
static inline float minimumf(float a, float b) {
  if (a != a || b != b) return NAN;
  return a < b ? a : b;
}

/* ------------------------------------------------------------------------ */
/* elementary ops                                                            */
/* ------------------------------------------------------------------------ */
void orc_fill_f32(float *out, int64_t n, float v) {
  #pragma omp parallel for
  for (int64_t i = 0; i < n; ++i) out[i] = v;
}

void orc_matmul_f32(const float *A, int64_t lda, const float *B, int64_t ldb,
                    float *C, int64_t ldc, int64_t M, int64_t N, int64_t K) {
  #pragma omp parallel for
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n)
      for (int64_t k = 0; k < K; ++k) {
        float p = A[m * lda + k] * B[k * ldb + n];
        C[m * ldc + n] = C[m * ldc + n] + p;
      }
}

void orc_matmul_bf16_f32(const uint16_t *A, int64_t lda, const uint16_t *B,
                         int64_t ldb, float *C, int64_t ldc, int64_t M,
                         int64_t N, int64_t K) {
  #pragma omp parallel for
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n)
      for (int64_t k = 0; k < K; ++k) {
        float p = bf2f(A[m * lda + k]) * bf2f(B[k * ldb + n]);
        C[m * ldc + n] = C[m * ldc + n] + p;
      }
}

void orc_matmul_tiled_m_f32(const float *A, const float *B, float *C,
                            int64_t M, int64_t N, int64_t K, int64_t tile_m) {
  for (int64_t i = 0; i < M; i += tile_m) {
    int64_t tm = (M - i) < tile_m ? (M - i) : tile_m;
    orc_matmul_f32(A + i * K, K, B, N, C + i * N, N, tm, N, K);
  }
}

void orc_batch_matmul_f32(const float *A, const float *B, float *C,
                          int64_t Bt, int64_t M, int64_t N, int64_t K) {
  #pragma omp parallel for collapse(2)
  for (int64_t b = 0; b < Bt; ++b)
    for (int64_t m = 0; m < M; ++m)
      for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k) {
          float p = A[(b * M + m) * K + k] * B[(b * K + k) * N + n];
          C[(b * M + m) * N + n] = C[(b * M + m) * N + n] + p;
        }
}

void orc_relu_f32(const float *in, float *out, int64_t n) {
  #pragma omp parallel for
  for (int64_t i = 0; i < n; ++i) out[i] = maximumf(in[i], 0.0f);
}
void orc_relu6_f32(const float *in, float *out, int64_t n) {
  #pragma omp parallel for
  for (int64_t i = 0; i < n; ++i) out[i] = minimumf(maximumf(in[i], 0.0f), 6.0f);
}
void orc_add_f32(const float *a, const float *b, float *out, int64_t n) {
  #pragma omp parallel for
  for (int64_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
}
void orc_bias_add_f32(const float *in, const float *bias, float *out,
                      int64_t rows, int64_t cols) {
  #pragma omp parallel for
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < cols; ++c)
      out[r * cols + c] = in[r * cols + c] + bias[c];
}
void orc_silu_mul_f32(const float *g, const float *u, float *out, int64_t n) {
  #pragma omp parallel for
  for (int64_t i = 0; i < n; ++i) {
    float e = expf(-g[i]);
    float den = 1.0f + e;
    float s = g[i] / den;
    out[i] = s * u[i];
  }
}

/* tensor.pad, constant value v. */
void orc_pad_nchw_f32(const float *in, float *out, int64_t N, int64_t C,
                      int64_t H, int64_t W, int64_t pt, int64_t pb,
                      int64_t pl, int64_t pr, float v) {
  int64_t Hp = H + pt + pb, Wp = W + pl + pr;
  #pragma omp parallel for collapse(2)
  for (int64_t n = 0; n < N; ++n)
    for (int64_t c = 0; c < C; ++c)
      for (int64_t h = 0; h < Hp; ++h)
        for (int64_t w = 0; w < Wp; ++w) {
          int64_t ih = h - pt, iw = w - pl;
          out[((n * C + c) * Hp + h) * Wp + w] =
              (ih >= 0 && ih < H && iw >= 0 && iw < W)
                  ? in[((n * C + c) * H + ih) * W + iw]
                  : v;
        }
}

#define PAD_NHWC_BODY(T, ZERO)                                               \
  int64_t Hp = H + pt + pb, Wp = W + pl + pr;                                \
  _Pragma("omp parallel for collapse(2)")                                    \
  for (int64_t n = 0; n < N; ++n)                                            \
    for (int64_t h = 0; h < Hp; ++h)                                         \
      for (int64_t w = 0; w < Wp; ++w)                                       \
        for (int64_t c = 0; c < C; ++c) {                                    \
          int64_t ih = h - pt, iw = w - pl;                                  \
          out[((n * Hp + h) * Wp + w) * C + c] =                             \
              (ih >= 0 && ih < H && iw >= 0 && iw < W)                       \
                  ? in[((n * H + ih) * W + iw) * C + c]                      \
                  : (T)(ZERO);                                               \
        }

void orc_pad_nhwc_f32(const float *in, float *out, int64_t N, int64_t H,
                      int64_t W, int64_t C, int64_t pt, int64_t pb,
                      int64_t pl, int64_t pr, float v) {
  PAD_NHWC_BODY(float, v)
}
void orc_pad_nhwc_u16(const uint16_t *in, uint16_t *out, int64_t N, int64_t H,
                      int64_t W, int64_t C, int64_t pt, int64_t pb,
                      int64_t pl, int64_t pr) {
  PAD_NHWC_BODY(uint16_t, 0)
}
void orc_pad_nhwc_i8(const int8_t *in, int8_t *out, int64_t N, int64_t H,
                     int64_t W, int64_t C, int64_t pt, int64_t pb, int64_t pl,
                     int64_t pr) {
  PAD_NHWC_BODY(int8_t, 0)
}

void orc_conv2d_nchw_fchw_f32(const float *in, const float *w, float *out,
                              int64_t N, int64_t C, int64_t Hp, int64_t Wp,
                              int64_t F, int64_t KH, int64_t KW, int64_t SH,
                              int64_t SW) {
  int64_t Ho = (Hp - KH) / SH + 1, Wo = (Wp - KW) / SW + 1;
  #pragma omp parallel for collapse(2)
  for (int64_t n = 0; n < N; ++n)
    for (int64_t f = 0; f < F; ++f)
      for (int64_t oh = 0; oh < Ho; ++oh)
        for (int64_t ow = 0; ow < Wo; ++ow)
          for (int64_t c = 0; c < C; ++c)
            for (int64_t kh = 0; kh < KH; ++kh)
              for (int64_t kw = 0; kw < KW; ++kw) {
                float a = in[((n * C + c) * Hp + oh * SH + kh) * Wp + ow * SW + kw];
                float b = w[((f * C + c) * KH + kh) * KW + kw];
                float p = a * b;
                int64_t o = ((n * F + f) * Ho + oh) * Wo + ow;
                out[o] = out[o] + p;
              }
}

void orc_conv2d_nhwc_fhwc_f32(const float *in, const float *w, float *out,
                              int64_t N, int64_t Hp, int64_t Wp, int64_t C,
                              int64_t F, int64_t KH, int64_t KW, int64_t SH,
                              int64_t SW) {
  int64_t Ho = (Hp - KH) / SH + 1, Wo = (Wp - KW) / SW + 1;
  #pragma omp parallel for collapse(2)
  for (int64_t n = 0; n < N; ++n)
    for (int64_t oh = 0; oh < Ho; ++oh)
      for (int64_t ow = 0; ow < Wo; ++ow)
        for (int64_t f = 0; f < F; ++f) {
          int64_t o = ((n * Ho + oh) * Wo + ow) * F + f;
          for (int64_t kh = 0; kh < KH; ++kh)
            for (int64_t kw = 0; kw < KW; ++kw)
              for (int64_t c = 0; c < C; ++c) {
                float a = in[((n * Hp + oh * SH + kh) * Wp + ow * SW + kw) * C + c];
                float b = w[((f * KH + kh) * KW + kw) * C + c];
                float p = a * b;
                out[o] = out[o] + p;
              }
        }
}

void orc_conv2d_nhwc_fhwc_bf16_f32(const uint16_t *in, const uint16_t *w,
                                   float *out, int64_t N, int64_t Hp,
                                   int64_t Wp, int64_t C, int64_t F,
                                   int64_t KH, int64_t KW, int64_t SH,
                                   int64_t SW) {
  int64_t Ho = (Hp - KH) / SH + 1, Wo = (Wp - KW) / SW + 1;
  #pragma omp parallel for collapse(2)
  for (int64_t n = 0; n < N; ++n)
    for (int64_t oh = 0; oh < Ho; ++oh)
      for (int64_t ow = 0; ow < Wo; ++ow)
        for (int64_t f = 0; f < F; ++f) {
          int64_t o = ((n * Ho + oh) * Wo + ow) * F + f;
          for (int64_t kh = 0; kh < KH; ++kh)
            for (int64_t kw = 0; kw < KW; ++kw)
              for (int64_t c = 0; c < C; ++c) {
                float a = bf2f(in[((n * Hp + oh * SH + kh) * Wp + ow * SW + kw) * C + c]);
                float b = bf2f(w[((f * KH + kh) * KW + kw) * C + c]);
                float p = a * b;
                out[o] = out[o] + p;
              }
        }
}

void orc_conv2d_nhwc_fhwc_i8_i32(const int8_t *in, const int8_t *w,
                                 int32_t *out, int64_t N, int64_t Hp,
                                 int64_t Wp, int64_t C, int64_t F, int64_t KH,
                                 int64_t KW, int64_t SH, int64_t SW) {
  int64_t Ho = (Hp - KH) / SH + 1, Wo = (Wp - KW) / SW + 1;
  #pragma omp parallel for collapse(2)
  for (int64_t n = 0; n < N; ++n)
    for (int64_t oh = 0; oh < Ho; ++oh)
      for (int64_t ow = 0; ow < Wo; ++ow)
        for (int64_t f = 0; f < F; ++f) {
          int64_t o = ((n * Ho + oh) * Wo + ow) * F + f;
          int32_t acc = out[o];
          for (int64_t kh = 0; kh < KH; ++kh)
            for (int64_t kw = 0; kw < KW; ++kw)
              for (int64_t c = 0; c < C; ++c) {
                int32_t a = in[((n * Hp + oh * SH + kh) * Wp + ow * SW + kw) * C + c];
                int32_t b = w[((f * KH + kh) * KW + kw) * C + c];
                acc += a * b;
              }
          out[o] = acc;
        }
}

void orc_depthwise_conv2d_nhwc_hwc_f32(const float *in, const float *w,
                                       float *out, int64_t N, int64_t Hp,
                                       int64_t Wp, int64_t C, int64_t KH,
                                       int64_t KW, int64_t SH, int64_t SW) {
  int64_t Ho = (Hp - KH) / SH + 1, Wo = (Wp - KW) / SW + 1;
  #pragma omp parallel for collapse(2)
  for (int64_t n = 0; n < N; ++n)
    for (int64_t oh = 0; oh < Ho; ++oh)
      for (int64_t ow = 0; ow < Wo; ++ow)
        for (int64_t c = 0; c < C; ++c) {
          int64_t o = ((n * Ho + oh) * Wo + ow) * C + c;
          for (int64_t kh = 0; kh < KH; ++kh)
            for (int64_t kw = 0; kw < KW; ++kw) {
              float a = in[((n * Hp + oh * SH + kh) * Wp + ow * SW + kw) * C + c];
              float b = w[(kh * KW + kw) * C + c];
              float p = a * b;
              out[o] = out[o] + p;
            }
        }
}

void orc_apply_scale_i32(const int32_t *acc, const int32_t *mult,
                         const int32_t *shift, int32_t *out, int64_t rows,
                         int64_t cols) {
  #pragma omp parallel for
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < cols; ++c) {
      int64_t v = (int64_t)acc[r * cols + c] * (int64_t)mult[c];
      v += (int64_t)1 << (shift[c] - 1);
      v >>= shift[c]; /* arithmetic shift: gcc sign-extends on signed types */
      out[r * cols + c] = (int32_t)v;
    }
}
void orc_add_i32(const int32_t *a, const int32_t *b, int32_t *out, int64_t n) {
  #pragma omp parallel for
  for (int64_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
}
void orc_add_i32_i8(const int32_t *a, const int8_t *b, int32_t *out, int64_t n) {
  #pragma omp parallel for
  for (int64_t i = 0; i < n; ++i) out[i] = a[i] + (int32_t)b[i];
}
void orc_clamp_i32_i8(const int32_t *in, int8_t *out, int64_t n, int32_t lo,
                      int32_t hi) {
  #pragma omp parallel for
  for (int64_t i = 0; i < n; ++i) {
    int32_t v = in[i] < lo ? lo : in[i];
    v = v > hi ? hi : v;
    out[i] = (int8_t)v;
  }
}

void orc_rmsnorm_f32(const float *x, const float *g, float *out, int64_t rows,
                     int64_t d, float eps) {
  #pragma omp parallel for
  for (int64_t r = 0; r < rows; ++r) {
    const float *xr = x + r * d;
    float s = 0.0f;
    for (int64_t j = 0; j < d; ++j) {
      float sq = xr[j] * xr[j];
      s = s + sq;
    }
    float ms = s / (float)d;
    float inv = 1.0f / sqrtf(ms + eps);
    for (int64_t j = 0; j < d; ++j) {
      float t = xr[j] * inv;
      out[r * d + j] = t * g[j];
    }
  }
}

void orc_rope_f32(const float *x, const float *cos_t, const float *sin_t,
                  float *out, int64_t S, int64_t H, int64_t Dh) {
  int64_t half = Dh / 2, D = H * Dh;
  #pragma omp parallel for collapse(2)
  for (int64_t s = 0; s < S; ++s)
    for (int64_t h = 0; h < H; ++h)
      for (int64_t i = 0; i < half; ++i) {
        float c = cos_t[s * half + i], sn = sin_t[s * half + i];
        float x0 = x[s * D + h * Dh + 2 * i], x1 = x[s * D + h * Dh + 2 * i + 1];
        float a = x0 * c, b = x1 * sn, e = x0 * sn, f = x1 * c;
        out[s * D + h * Dh + 2 * i] = a - b;
        out[s * D + h * Dh + 2 * i + 1] = e + f;
      }
}

void orc_causal_softmax_f32(float *s, int64_t rows, int64_t cols) {
  int64_t off = cols - rows;
  #pragma omp parallel for
  for (int64_t i = 0; i < rows; ++i) {
    float *r = s + i * cols;
    int64_t last = i + off; /* keys 0..last are visible */
    float m = -INFINITY;
    for (int64_t j = 0; j <= last; ++j) m = maximumf(m, r[j]);
    float sum = 0.0f;
    for (int64_t j = 0; j <= last; ++j) {
      float d = r[j] - m;
      r[j] = expf(d);
      sum = sum + r[j];
    }
    for (int64_t j = 0; j < cols; ++j) r[j] = (j <= last) ? r[j] / sum : 0.0f;
  }
}

/* ------------------------------------------------------------------------ */
/* composite blocks                                                          */
/* ------------------------------------------------------------------------ */
static void *xmalloc(size_t n) {
  void *p = malloc(n ? n : 1);
  if (!p) abort();
  return p;
}

static void apply_act_f32(float *buf, int64_t n, int act) {
  if (act == 1) orc_relu_f32(buf, buf, n);
  else if (act == 2) orc_relu6_f32(buf, buf, n);
}

void orc_block_matmul_bias_act_f32(const float *A, const float *B,
                                   const float *bias, float *out, int64_t M,
                                   int64_t N, int64_t K, int act) {
  float *acc = (float *)xmalloc(sizeof(float) * M * N);
  orc_fill_f32(acc, M * N, 0.0f);
  orc_matmul_f32(A, K, B, N, acc, N, M, N, K);
  if (bias) orc_bias_add_f32(acc, bias, out, M, N);
  else memcpy(out, acc, sizeof(float) * M * N);
  apply_act_f32(out, M * N, act);
  free(acc);
}

void orc_block_conv_bias_act_f32(const float *x, const float *w,
                                 const float *bias, float *out, int64_t N,
                                 int64_t H, int64_t W, int64_t C, int64_t F,
                                 int64_t KH, int64_t KW, int64_t pad, int act) {
  int64_t Hp = H + 2 * pad, Wp = W + 2 * pad;
  int64_t Ho = Hp - KH + 1, Wo = Wp - KW + 1;
  float *xp = (float *)xmalloc(sizeof(float) * N * Hp * Wp * C);
  float *acc = (float *)xmalloc(sizeof(float) * N * Ho * Wo * F);
  orc_pad_nhwc_f32(x, xp, N, H, W, C, pad, pad, pad, pad, 0.0f);
  orc_fill_f32(acc, N * Ho * Wo * F, 0.0f);
  orc_conv2d_nhwc_fhwc_f32(xp, w, acc, N, Hp, Wp, C, F, KH, KW, 1, 1);
  if (bias) orc_bias_add_f32(acc, bias, out, N * Ho * Wo, F);
  else memcpy(out, acc, sizeof(float) * N * Ho * Wo * F);
  apply_act_f32(out, N * Ho * Wo * F, act);
  free(xp);
  free(acc);
}

void orc_block_conv_bias_act_bf16(const uint16_t *x, const uint16_t *w,
                                  const float *bias, uint16_t *out, int64_t N,
                                  int64_t H, int64_t W, int64_t C, int64_t F,
                                  int64_t KH, int64_t KW, int64_t pad, int act) {
  int64_t Hp = H + 2 * pad, Wp = W + 2 * pad;
  int64_t Ho = Hp - KH + 1, Wo = Wp - KW + 1, no = N * Ho * Wo * F;
  uint16_t *xp = (uint16_t *)xmalloc(sizeof(uint16_t) * N * Hp * Wp * C);
  float *acc = (float *)xmalloc(sizeof(float) * no);
  orc_pad_nhwc_u16(x, xp, N, H, W, C, pad, pad, pad, pad);
  orc_fill_f32(acc, no, 0.0f);
  orc_conv2d_nhwc_fhwc_bf16_f32(xp, w, acc, N, Hp, Wp, C, F, KH, KW, 1, 1);
  if (bias) orc_bias_add_f32(acc, bias, acc, N * Ho * Wo, F);
  apply_act_f32(acc, no, act);
  orc_trunc_f32_bf16(acc, out, no);
  free(xp);
  free(acc);
}

void orc_block_irb_f32(const float *x, const float *we, const float *wdw,
                       const float *wp, float *out, int64_t N, int64_t H,
                       int64_t W, int64_t C, int64_t E) {
  int64_t P = N * H * W;
  float *e = (float *)xmalloc(sizeof(float) * P * E);
  float *ep = (float *)xmalloc(sizeof(float) * N * (H + 2) * (W + 2) * E);
  float *d = (float *)xmalloc(sizeof(float) * P * E);
  float *p = (float *)xmalloc(sizeof(float) * P * C);
  /* 1x1 expand: conv_2d_nhwc_fhwc with a [E,1,1,C] filter */
  orc_fill_f32(e, P * E, 0.0f);
  orc_conv2d_nhwc_fhwc_f32(x, we, e, N, H, W, C, E, 1, 1, 1, 1);
  orc_relu6_f32(e, e, P * E);
  orc_pad_nhwc_f32(e, ep, N, H, W, E, 1, 1, 1, 1, 0.0f);
  orc_fill_f32(d, P * E, 0.0f);
  orc_depthwise_conv2d_nhwc_hwc_f32(ep, wdw, d, N, H + 2, W + 2, E, 3, 3, 1, 1);
  orc_relu6_f32(d, d, P * E);
  /* 1x1 project: [C,1,1,E] filter */
  orc_fill_f32(p, P * C, 0.0f);
  orc_conv2d_nhwc_fhwc_f32(d, wp, p, N, H, W, E, C, 1, 1, 1, 1);
  orc_add_f32(p, x, out, P * C);
  free(e);
  free(ep);
  free(d);
  free(p);
}

void orc_block_qbottleneck_i8(const int8_t *x, const int8_t *w1,
                              const int8_t *w2, const int8_t *w3,
                              const int32_t *m1, const int32_t *s1,
                              const int32_t *m2, const int32_t *s2,
                              const int32_t *m3, const int32_t *s3,
                              int8_t *out, int64_t N, int64_t H, int64_t W,
                              int64_t C, int64_t M1) {
  int64_t P = N * H * W;
  int32_t *acc1 = (int32_t *)calloc((size_t)(P * M1), sizeof(int32_t));
  int8_t *y1 = (int8_t *)xmalloc((size_t)(P * M1));
  int8_t *y1p = (int8_t *)xmalloc((size_t)(N * (H + 2) * (W + 2) * M1));
  int32_t *acc2 = (int32_t *)calloc((size_t)(P * M1), sizeof(int32_t));
  int8_t *y2 = (int8_t *)xmalloc((size_t)(P * M1));
  int32_t *acc3 = (int32_t *)calloc((size_t)(P * C), sizeof(int32_t));
  if (!acc1 || !acc2 || !acc3) abort();
  orc_conv2d_nhwc_fhwc_i8_i32(x, w1, acc1, N, H, W, C, M1, 1, 1, 1, 1);
  orc_apply_scale_i32(acc1, m1, s1, acc1, P, M1);
  orc_clamp_i32_i8(acc1, y1, P * M1, 0, 127);
  orc_pad_nhwc_i8(y1, y1p, N, H, W, M1, 1, 1, 1, 1);
  orc_conv2d_nhwc_fhwc_i8_i32(y1p, w2, acc2, N, H + 2, W + 2, M1, M1, 3, 3, 1, 1);
  orc_apply_scale_i32(acc2, m2, s2, acc2, P, M1);
  orc_clamp_i32_i8(acc2, y2, P * M1, 0, 127);
  orc_conv2d_nhwc_fhwc_i8_i32(y2, w3, acc3, N, H, W, M1, C, 1, 1, 1, 1);
  orc_apply_scale_i32(acc3, m3, s3, acc3, P, C);
  orc_add_i32_i8(acc3, x, acc3, P * C);
  orc_clamp_i32_i8(acc3, out, P * C, 0, 127);
  free(acc1);
  free(y1);
  free(y1p);
  free(acc2);
  free(y2);
  free(acc3);
}

/* ---- Llama decoder layer sub-groups ---------------------------------- */
static void ext_all(const uint16_t *in, float *out, int64_t n) {
  orc_ext_bf16_f32(in, out, n);
}

void orc_llama_qkv_bf16(const uint16_t *x, const float *g1, const uint16_t *wq,
                        const uint16_t *wk, const uint16_t *wv,
                        const float *cos_t, const float *sin_t, uint16_t *Q,
                        uint16_t *K, uint16_t *V, int64_t S, int64_t D,
                        int64_t H, float eps) {
  int64_t Dh = D / H;
  float *xf = (float *)xmalloc(sizeof(float) * S * D);
  float *xnf = (float *)xmalloc(sizeof(float) * S * D);
  uint16_t *xn = (uint16_t *)xmalloc(sizeof(uint16_t) * S * D);
  float *acc = (float *)xmalloc(sizeof(float) * S * D);
  float *rot = (float *)xmalloc(sizeof(float) * S * D);
  ext_all(x, xf, S * D);
  orc_rmsnorm_f32(xf, g1, xnf, S, D, eps);
  orc_trunc_f32_bf16(xnf, xn, S * D);
  /* Q */
  orc_fill_f32(acc, S * D, 0.0f);
  orc_matmul_bf16_f32(xn, D, wq, D, acc, D, S, D, D);
  orc_rope_f32(acc, cos_t, sin_t, rot, S, H, Dh);
  orc_trunc_f32_bf16(rot, Q, S * D);
  /* K */
  orc_fill_f32(acc, S * D, 0.0f);
  orc_matmul_bf16_f32(xn, D, wk, D, acc, D, S, D, D);
  orc_rope_f32(acc, cos_t, sin_t, rot, S, H, Dh);
  orc_trunc_f32_bf16(rot, K, S * D);
  /* V */
  orc_fill_f32(acc, S * D, 0.0f);
  orc_matmul_bf16_f32(xn, D, wv, D, acc, D, S, D, D);
  orc_trunc_f32_bf16(acc, V, S * D);
  free(xf);
  free(xnf);
  free(xn);
  free(acc);
  free(rot);
}

void orc_llama_attention_bf16(const uint16_t *Q, const uint16_t *K,
                              const uint16_t *V, uint16_t *A, int64_t S,
                              int64_t H, int64_t Dh, float scale) {
  int64_t D = H * Dh;
  float *qh = (float *)xmalloc(sizeof(float) * S * Dh);
  float *kt = (float *)xmalloc(sizeof(float) * Dh * S);
  float *vh = (float *)xmalloc(sizeof(float) * S * Dh);
  float *s = (float *)xmalloc(sizeof(float) * S * S);
  float *o = (float *)xmalloc(sizeof(float) * S * Dh);
  for (int64_t h = 0; h < H; ++h) {
    for (int64_t i = 0; i < S; ++i)
      for (int64_t d = 0; d < Dh; ++d) {
        qh[i * Dh + d] = bf2f(Q[i * D + h * Dh + d]);
        kt[d * S + i] = bf2f(K[i * D + h * Dh + d]); /* linalg.transpose */
        vh[i * Dh + d] = bf2f(V[i * D + h * Dh + d]);
      }
    orc_fill_f32(s, S * S, 0.0f);
    orc_matmul_f32(qh, Dh, kt, S, s, S, S, S, Dh);
    #pragma omp parallel for
    for (int64_t i = 0; i < S * S; ++i) s[i] = s[i] * scale;
    orc_causal_softmax_f32(s, S, S);
    orc_fill_f32(o, S * Dh, 0.0f);
    orc_matmul_f32(s, S, vh, Dh, o, Dh, S, Dh, S);
    for (int64_t i = 0; i < S; ++i)
      for (int64_t d = 0; d < Dh; ++d)
        A[i * D + h * Dh + d] = f2bf(o[i * Dh + d]);
  }
  free(qh);
  free(kt);
  free(vh);
  free(s);
  free(o);
}

void orc_llama_matmul_residual_bf16(const uint16_t *a, const uint16_t *w,
                                    const uint16_t *res, uint16_t *out,
                                    int64_t S, int64_t N, int64_t Kd) {
  float *acc = (float *)xmalloc(sizeof(float) * S * N);
  float *rf = (float *)xmalloc(sizeof(float) * S * N);
  orc_fill_f32(acc, S * N, 0.0f);
  orc_matmul_bf16_f32(a, Kd, w, N, acc, N, S, N, Kd);
  ext_all(res, rf, S * N);
  orc_add_f32(rf, acc, acc, S * N);
  orc_trunc_f32_bf16(acc, out, S * N);
  free(acc);
  free(rf);
}

void orc_llama_swiglu_bf16(const uint16_t *h, const float *g2,
                           const uint16_t *wg, const uint16_t *wu,
                           uint16_t *act, int64_t S, int64_t D, int64_t F,
                           float eps) {
  float *hf = (float *)xmalloc(sizeof(float) * S * D);
  uint16_t *hn = (uint16_t *)xmalloc(sizeof(uint16_t) * S * D);
  float *gacc = (float *)xmalloc(sizeof(float) * S * F);
  float *uacc = (float *)xmalloc(sizeof(float) * S * F);
  ext_all(h, hf, S * D);
  orc_rmsnorm_f32(hf, g2, hf, S, D, eps);
  orc_trunc_f32_bf16(hf, hn, S * D);
  orc_fill_f32(gacc, S * F, 0.0f);
  orc_matmul_bf16_f32(hn, D, wg, F, gacc, F, S, F, D);
  orc_fill_f32(uacc, S * F, 0.0f);
  orc_matmul_bf16_f32(hn, D, wu, F, uacc, F, S, F, D);
  orc_silu_mul_f32(gacc, uacc, gacc, S * F);
  orc_trunc_f32_bf16(gacc, act, S * F);
  free(hf);
  free(hn);
  free(gacc);
  free(uacc);
}

void orc_block_llama_layer_bf16(const uint16_t *x, const float *g1,
                                const float *g2, const uint16_t *wq,
                                const uint16_t *wk, const uint16_t *wv,
                                const uint16_t *wo, const uint16_t *wg,
                                const uint16_t *wu, const uint16_t *wd,
                                const float *cos_t, const float *sin_t,
                                uint16_t *h, uint16_t *out, int64_t S,
                                int64_t D, int64_t H, int64_t F, float eps) {
  int64_t Dh = D / H;
  uint16_t *Q = (uint16_t *)xmalloc(sizeof(uint16_t) * S * D);
  uint16_t *K = (uint16_t *)xmalloc(sizeof(uint16_t) * S * D);
  uint16_t *V = (uint16_t *)xmalloc(sizeof(uint16_t) * S * D);
  uint16_t *A = (uint16_t *)xmalloc(sizeof(uint16_t) * S * D);
  uint16_t *act = (uint16_t *)xmalloc(sizeof(uint16_t) * S * F);
  orc_llama_qkv_bf16(x, g1, wq, wk, wv, cos_t, sin_t, Q, K, V, S, D, H, eps);
  orc_llama_attention_bf16(Q, K, V, A, S, H, Dh, 1.0f / sqrtf((float)Dh));
  orc_llama_matmul_residual_bf16(A, wo, x, h, S, D, D);
  orc_llama_swiglu_bf16(h, g2, wg, wu, act, S, D, F, eps);
  orc_llama_matmul_residual_bf16(act, wd, h, out, S, D, F);
  free(Q);
  free(K);
  free(V);
  free(A);
  free(act);
}
