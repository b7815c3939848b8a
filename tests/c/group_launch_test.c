/* A compiled C caller of the outlined-group boundary (include/npu_amd.h,
 * npu_group_launch), the way a host module built from the reference's
 * pipeline output would call a group: by the outliner's name, with MLIR
 * memref descriptors in the outlined function's argument order
 * (lib/Transforms/OutlineFusedGroupsPass.cpp:218-263, 306-316) and the
 * harness's argument fills 0.01 * (i + 1) (tools/harness/e2e_verify.py:186-203).
 *
 *   group_launch_test validate   rejections before any launch (no GPU used)
 *   group_launch_test gpu        launches on device 0, checked against the
 *                                reference's closed forms and the oracle
 * Exit status 0 when every check passes. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "../../include/npu_amd.h"
#include "../../oracle/npu_oracle.h"

static int failures = 0;

#define CHECK(cond, ...)                         \
  do {                                           \
    if (!(cond)) {                               \
      fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
      fprintf(stderr, __VA_ARGS__);              \
      fprintf(stderr, "\n");                     \
      ++failures;                                \
    }                                            \
  } while (0)

static npu_arg scalar(double v) {
  npu_arg a;
  memset(&a, 0, sizeof a);
  a.kind = NPU_ARG_SCALAR;
  a.dtype = NPU_F32;
  a.scalar = v;
  return a;
}

static npu_arg mem2(npu_strided_memref_2d *d, void *data, int64_t r, int64_t c) {
  npu_arg a;
  memset(&a, 0, sizeof a);
  d->allocated = d->aligned = data;
  d->offset = 0;
  d->sizes[0] = r;
  d->sizes[1] = c;
  d->strides[0] = c;
  d->strides[1] = 1;
  a.rank = 2;
  a.descriptor = d;
  a.dtype = NPU_F32;
  a.kind = NPU_ARG_MEMREF;
  return a;
}

static npu_arg mem4(npu_strided_memref_4d *d, void *data, int64_t n, int64_t h, int64_t w,
                    int64_t c) {
  npu_arg a;
  memset(&a, 0, sizeof a);
  d->allocated = d->aligned = data;
  d->offset = 0;
  d->sizes[0] = n;
  d->sizes[1] = h;
  d->sizes[2] = w;
  d->sizes[3] = c;
  d->strides[3] = 1;
  d->strides[2] = c;
  d->strides[1] = w * c;
  d->strides[0] = h * w * c;
  a.rank = 4;
  a.descriptor = d;
  a.dtype = NPU_F32;
  a.kind = NPU_ARG_MEMREF;
  return a;
}

static npu_arg mem1(npu_strided_memref_1d *d, void *data, int64_t n) {
  npu_arg a;
  memset(&a, 0, sizeof a);
  d->allocated = d->aligned = data;
  d->offset = 0;
  d->sizes[0] = n;
  d->strides[0] = 1;
  a.rank = 1;
  a.descriptor = d;
  a.dtype = NPU_F32;
  a.kind = NPU_ARG_MEMREF;
  return a;
}

static npu_group_attrs relu_attrs(void) {
  npu_group_attrs at;
  memset(&at, 0, sizeof at);
  for (int i = 0; i < NPU_GROUP_MAX_CHAINS; ++i) at.act[i] = NPU_ACT_RELU;
  return at;
}

/* --- rejections: every call below fails validation before a launch ---- */
static void validate(void) {
  /* fake device addresses: never dereferenced, the calls are rejected */
  void *A = (void *)0x100000, *B = (void *)0x200000, *O = (void *)0x300000;
  npu_strided_memref_2d dA, dB, dI, dE, dO, dBad;
  npu_strided_memref_1d db;
  npu_group_attrs at = relu_attrs();
  npu_arg in[6], out[1];
  in[0] = scalar(0.0);
  in[1] = mem2(&dI, NULL, 128, 512);
  in[2] = mem2(&dA, A, 128, 256);
  in[3] = mem2(&dB, B, 256, 512);
  in[4] = mem2(&dE, NULL, 128, 512);
  out[0] = mem2(&dO, O, 128, 512);

  npu_status s = npu_group_launch("fused_fill_batch_matmul_generic_0", &at, in, 5, out, 1, NULL);
  CHECK(s == NPU_ERR_UNSUPPORTED, "unknown chain: status %d", s);
  CHECK(strstr(npu_last_error(), "fill_batch_matmul_generic") != NULL, "message: %s",
        npu_last_error());
  /* the reference's NCHW conv group takes rank-4 operands */
  s = npu_group_launch("fused_fill_conv2d_generic_0", &at, in, 5, out, 1, NULL);
  CHECK(s == NPU_ERR_INVALID_ARG && strstr(npu_last_error(), "rank-4"),
        "NCHW group with matrices: status %d (%s)", s, npu_last_error());

  s = npu_group_launch("fused_fill_matmul_generic_0", &at, in, 4, out, 1, NULL);
  CHECK(s == NPU_ERR_INVALID_ARG, "missing destination: status %d", s);

  in[0] = scalar(1.0);
  s = npu_group_launch("fused_fill_matmul_generic_3", &at, in, 5, out, 1, NULL);
  CHECK(s == NPU_ERR_UNSUPPORTED && strstr(npu_last_error(), "fill value"),
        "fill of 1.0: status %d (%s)", s, npu_last_error());
  in[0] = scalar(0.0);

  in[3] = mem2(&dBad, B, 255, 512);
  s = npu_group_launch("fused_fill_matmul_generic_0", &at, in, 5, out, 1, NULL);
  CHECK(s == NPU_ERR_INVALID_ARG && strstr(npu_last_error(), "K differs"),
        "B rows != K: status %d (%s)", s, npu_last_error());
  in[3] = mem2(&dB, B, 256, 512);

  in[4] = mem2(&dE, NULL, 128, 511);
  s = npu_group_launch("fused_fill_matmul_generic_0", &at, in, 5, out, 1, NULL);
  CHECK(s == NPU_ERR_INVALID_ARG, "destination shape: status %d", s);
  in[4] = mem2(&dE, NULL, 128, 512);

  /* a bias of the wrong length */
  npu_arg inb[6] = {in[0], in[1], in[2], in[3], mem1(&db, O, 511), in[4]};
  s = npu_group_launch("fused_fill_matmul_generic_0", &at, inb, 6, out, 1, NULL);
  CHECK(s == NPU_ERR_INVALID_ARG && strstr(npu_last_error(), "bias"),
        "bias length: status %d (%s)", s, npu_last_error());

  s = npu_group_launch(NULL, &at, in, 5, out, 1, NULL);
  CHECK(s == NPU_ERR_INVALID_ARG, "null name: status %d", s);
  s = npu_group_launch("fused_fill_matmul_generic_0", &at, in, 5, out, 2, NULL);
  CHECK(s == NPU_ERR_UNSUPPORTED, "two results: status %d", s);
  in[2].rank = 7;
  s = npu_group_launch("fused_fill_matmul_generic_0", &at, in, 5, out, 1, NULL);
  CHECK(s == NPU_ERR_UNSUPPORTED, "rank 7: status %d", s);
  in[2].rank = 2;
  /* two matmul chains need a destination to hold the first result */
  npu_strided_memref_2d dI2, dW2, dE2, dO2;
  npu_arg in2[8] = {in[0], in[1], in[2], in[3], mem2(&dE, NULL, 128, 512),
                    mem2(&dI2, NULL, 128, 256), mem2(&dW2, B, 512, 256),
                    mem2(&dE2, NULL, 128, 256)};
  npu_arg out2[1] = {mem2(&dO2, O, 128, 256)};
  s = npu_group_launch("fused_fill_matmul_generic_fill_matmul_generic_0", &at, in2, 8, out2, 1,
                       NULL);
  CHECK(s == NPU_ERR_INVALID_ARG && strstr(npu_last_error(), "intermediate"),
        "mlp without storage: status %d (%s)", s, npu_last_error());
  /* every chain is checked before the first launches: a second chain whose
   * weight does not match the first chain's result is rejected as such (on a
   * machine without a GPU a launch of the first chain would fail instead) */
  npu_strided_memref_2d dW2b;
  in2[4] = mem2(&dE, A, 128, 512);
  in2[6] = mem2(&dW2b, B, 500, 256);
  s = npu_group_launch("fused_fill_matmul_generic_fill_matmul_generic_0", &at, in2, 8, out2, 1,
                       NULL);
  CHECK(s == NPU_ERR_INVALID_ARG && strstr(npu_last_error(), "K differs"),
        "mlp, second weight: status %d (%s)", s, npu_last_error());
  in2[6] = mem2(&dW2, B, 512, 256);
  npu_strided_memref_2d dO3;
  npu_arg out3[1] = {mem2(&dO3, O, 128, 255)};
  s = npu_group_launch("fused_fill_matmul_generic_fill_matmul_generic_0", &at, in2, 8, out3, 1,
                       NULL);
  CHECK(s == NPU_ERR_INVALID_ARG && strstr(npu_last_error(), "result"),
        "mlp, result shape: status %d (%s)", s, npu_last_error());
  /* a conv group's residual named by index must be a rank-4 operand before
   * the last destination */
  {
    npu_strided_memref_4d dI4, dX4, dW4, dR4, dE41, dE42, dO4;
    void *X = (void *)0x400000, *W = (void *)0x500000, *R = (void *)0x600000;
    npu_arg ic[7] = {scalar(0.0), mem4(&dI4, NULL, 2, 8, 8, 16), mem4(&dX4, X, 2, 8, 8, 16),
                     mem4(&dW4, W, 16, 3, 3, 16), mem4(&dR4, R, 2, 8, 8, 16),
                     mem4(&dE41, O, 2, 8, 8, 16), mem4(&dE42, O, 2, 8, 8, 16)};
    npu_arg oc[1] = {mem4(&dO4, O, 2, 8, 8, 16)};
    npu_group_attrs ac = relu_attrs();
    ac.pad = 1;
    ac.res_arg = 6;
    s = npu_group_launch("fused_fill_linalg_conv_2d_nhwc_fhwc_generic_generic_0", &ac, ic, 7, oc, 1,
                         NULL);
    CHECK(s == NPU_ERR_INVALID_ARG && strstr(npu_last_error(), "res_arg"),
          "res_arg at the last destination: status %d (%s)", s, npu_last_error());
    /* without res_arg, destinations with data leave the residual ambiguous */
    ac.res_arg = 0;
    s = npu_group_launch("fused_fill_linalg_conv_2d_nhwc_fhwc_generic_generic_0", &ac, ic, 7, oc, 1,
                         NULL);
    CHECK(s == NPU_ERR_INVALID_ARG && strstr(npu_last_error(), "residual"),
          "ambiguous residual: status %d (%s)", s, npu_last_error());
  }
}

/* --- launches ------------------------------------------------------------ */
static float *dev_filled(int64_t n, float v) {
  float *h = (float *)malloc(n * sizeof(float)), *d = NULL;
  for (int64_t i = 0; i < n; ++i) h[i] = v;
  if (hipMalloc((void **)&d, n * sizeof(float)) != hipSuccess) abort();
  if (hipMemcpy(d, h, n * sizeof(float), hipMemcpyHostToDevice) != hipSuccess) abort();
  free(h);
  return d;
}

static float *dev_from(const float *h, int64_t n) {
  float *d = NULL;
  if (hipMalloc((void **)&d, n * sizeof(float)) != hipSuccess) abort();
  if (hipMemcpy(d, h, n * sizeof(float), hipMemcpyHostToDevice) != hipSuccess) abort();
  return d;
}

static float *host_of(const float *d, int64_t n) {
  float *h = (float *)malloc(n * sizeof(float));
  if (hipDeviceSynchronize() != hipSuccess) abort();
  if (hipMemcpy(h, d, n * sizeof(float), hipMemcpyDeviceToHost) != hipSuccess) abort();
  return h;
}

/* uniform in [-1, 1) from a 64-bit LCG (test inputs only) */
static float urand(uint64_t *s) {
  *s = *s * 6364136223846793005ull + 1442695040888963407ull;
  return (float)((double)(*s >> 11) / 9007199254740992.0 * 2.0 - 1.0);
}

static void gpu(void) {
  npu_group_attrs at = relu_attrs();
  /* test/matmul_relu.mlir under the harness: A = 0.01, B = 0.02, K = 256,
   * so every output is relu(256 * 2e-4) = 0.0512 (e2e_verify.py:288-309). */
  {
    const int64_t M = 128, K = 256, N = 512;
    float *A = dev_filled(M * K, 0.01f), *B = dev_filled(K * N, 0.02f), *O = dev_filled(M * N, -1);
    npu_strided_memref_2d dI, dA, dB, dE, dO;
    npu_arg in[5] = {scalar(0.0), mem2(&dI, NULL, M, N), mem2(&dA, A, M, K), mem2(&dB, B, K, N),
                     mem2(&dE, NULL, M, N)};
    npu_arg out[1] = {mem2(&dO, O, M, N)};
    npu_status s = npu_group_launch("fused_fill_matmul_generic_0", &at, in, 5, out, 1, NULL);
    CHECK(s == NPU_OK, "matmul_relu: %s", npu_last_error());
    float *h = host_of(O, M * N);
    double worst = 0;
    for (int64_t i = 0; i < M * N; ++i) worst = fmax(worst, fabs(h[i] - 0.0512));
    CHECK(worst <= 1e-4 * 0.0512 + 1e-7, "matmul_relu: max |out - 0.0512| = %g", worst);
    printf("matmul_relu KAT: max |out - 0.0512| = %.3g\n", worst);
    free(h);
    hipFree(A); hipFree(B); hipFree(O);
  }
  /* test/mlp.mlir: input 0.01, w1 0.02, w2 0.03: relu1 = 0.0512 everywhere,
   * out = 512 * 0.0512 * 0.03 = 0.786432. */
  {
    const int64_t M = 128, K = 256, H = 512, N = 256;
    float *X = dev_filled(M * K, 0.01f), *W1 = dev_filled(K * H, 0.02f);
    float *W2 = dev_filled(H * N, 0.03f), *R1 = dev_filled(M * H, 0), *O = dev_filled(M * N, -1);
    npu_strided_memref_2d dI1, dX, dW1, dE1, dI2, dW2, dE2, dO;
    npu_arg in[8] = {scalar(0.0), mem2(&dI1, NULL, M, H), mem2(&dX, X, M, K),
                     mem2(&dW1, W1, K, H), mem2(&dE1, R1, M, H), mem2(&dI2, NULL, M, N),
                     mem2(&dW2, W2, H, N), mem2(&dE2, NULL, M, N)};
    npu_arg out[1] = {mem2(&dO, O, M, N)};
    npu_status s = npu_group_launch("fused_fill_matmul_generic_fill_matmul_generic_0", &at, in,
                                    8, out, 1, NULL);
    CHECK(s == NPU_OK, "mlp: %s", npu_last_error());
    float *h = host_of(O, M * N);
    double worst = 0;
    for (int64_t i = 0; i < M * N; ++i) worst = fmax(worst, fabs(h[i] - 0.786432));
    CHECK(worst <= 1e-5 * 0.786432 * 2, "mlp: max |out - 0.786432| = %g", worst);
    printf("mlp KAT: max |out - 0.786432| = %.3g\n", worst);
    free(h);
    hipFree(X); hipFree(W1); hipFree(W2); hipFree(R1); hipFree(O);
  }
  /* the C1 group with a bias on seeded inputs, against the oracle's unfused
   * loops: |gpu - oracle| <= 1e-5 * sum_k |a b| + |bias| */
  {
    const int64_t M = 256, K = 512, N = 256;
    float *hA = malloc(M * K * 4), *hB = malloc(K * N * 4), *hb = malloc(N * 4);
    float *ref = malloc(M * N * 4);
    uint64_t seed = 0x4e505501;
    for (int64_t i = 0; i < M * K; ++i) hA[i] = urand(&seed);
    for (int64_t i = 0; i < K * N; ++i) hB[i] = urand(&seed);
    for (int64_t i = 0; i < N; ++i) hb[i] = urand(&seed);
    orc_block_matmul_bias_act_f32(hA, hB, hb, ref, M, N, K, 1);
    float *A = dev_from(hA, M * K), *B = dev_from(hB, K * N), *b = dev_from(hb, N);
    float *O = dev_filled(M * N, -1);
    npu_strided_memref_2d dI, dA, dB, dE, dO;
    npu_strided_memref_1d db;
    npu_arg in[6] = {scalar(0.0), mem2(&dI, NULL, M, N), mem2(&dA, A, M, K), mem2(&dB, B, K, N),
                     mem1(&db, b, N), mem2(&dE, NULL, M, N)};
    npu_arg out[1] = {mem2(&dO, O, M, N)};
    npu_status s = npu_group_launch("fused_fill_matmul_generic_7", &at, in, 6, out, 1, NULL);
    CHECK(s == NPU_OK, "matmul+bias+relu: %s", npu_last_error());
    float *h = host_of(O, M * N);
    int bad = 0;
    double worst = 0;
    for (int64_t m = 0; m < M; ++m)
      for (int64_t n = 0; n < N; ++n) {
        double mag = fabs(hb[n]);
        for (int64_t k = 0; k < K; ++k) mag += fabs((double)hA[m * K + k] * hB[k * N + n]);
        const double err = fabs((double)h[m * N + n] - ref[m * N + n]);
        worst = fmax(worst, err / mag);
        bad += err > 1e-5 * mag;
      }
    CHECK(bad == 0, "matmul+bias+relu: %d outputs outside 1e-5 * mag (worst %.3g)", bad, worst);
    printf("matmul+bias+relu vs oracle: worst |err|/mag = %.3g\n", worst);
    npu_launch_plan p[4];
    CHECK(npu_last_launch_plans(p, 4) == 1, "one launch plan recorded");
    free(h); free(hA); free(hB); free(hb); free(ref);
    hipFree(A); hipFree(B); hipFree(b); hipFree(O);
  }
  /* a ResNet-style conv group (add of the block input, then ReLU, in two
   * generics) called the way a bufferized host module calls it: every
   * destination allocated, the residual named by attrs.res_arg */
  {
    const int64_t N = 2, H = 8, W = 8, C = 16, F = 16;
    const int64_t nx = N * H * W * C, nw = F * 9 * C, no = N * H * W * F;
    float *hx = malloc(nx * 4), *hw = malloc(nw * 4), *hr = malloc(no * 4);
    float *conv = malloc(no * 4);
    uint64_t seed = 0x4e505502;
    for (int64_t i = 0; i < nx; ++i) hx[i] = urand(&seed);
    for (int64_t i = 0; i < nw; ++i) hw[i] = urand(&seed) * 0.1f;
    for (int64_t i = 0; i < no; ++i) hr[i] = urand(&seed);
    orc_block_conv_bias_act_f32(hx, hw, NULL, conv, N, H, W, C, F, 3, 3, 1, 0);
    float *X = dev_from(hx, nx), *Wt = dev_from(hw, nw), *R = dev_from(hr, no);
    float *D1 = dev_filled(no, 7), *D2 = dev_filled(no, 7), *I = dev_filled(no, 7);
    float *O = dev_filled(no, -1);
    npu_strided_memref_4d dI, dX, dW, dR, dD1, dD2, dO;
    npu_arg in[7] = {scalar(0.0), mem4(&dI, I, N, H, W, F), mem4(&dX, X, N, H, W, C),
                     mem4(&dW, Wt, F, 3, 3, C), mem4(&dR, R, N, H, W, F),
                     mem4(&dD1, D1, N, H, W, F), mem4(&dD2, D2, N, H, W, F)};
    npu_arg out[1] = {mem4(&dO, O, N, H, W, F)};
    npu_group_attrs ac = relu_attrs();
    ac.pad = 1;
    ac.res_arg = 4;
    npu_status s = npu_group_launch("fused_fill_linalg_conv_2d_nhwc_fhwc_generic_generic_3", &ac,
                                    in, 7, out, 1, NULL);
    CHECK(s == NPU_OK, "conv + residual + relu: %s", npu_last_error());
    float *h = host_of(O, no);
    int bad = 0;
    double worst = 0;
    for (int64_t n = 0; n < N; ++n)
      for (int64_t y = 0; y < H; ++y)
        for (int64_t x = 0; x < W; ++x)
          for (int64_t f = 0; f < F; ++f) {
            const int64_t o = ((n * H + y) * W + x) * F + f;
            double mag = fabs(hr[o]);
            for (int64_t ky = 0; ky < 3; ++ky)
              for (int64_t kx = 0; kx < 3; ++kx) {
                const int64_t iy = y + ky - 1, ix = x + kx - 1;
                if (iy < 0 || iy >= H || ix < 0 || ix >= W) continue;
                for (int64_t c = 0; c < C; ++c)
                  mag += fabs((double)hx[((n * H + iy) * W + ix) * C + c] * hw[((f * 3 + ky) * 3 + kx) * C + c]);
              }
            float ref = conv[o] + hr[o];
            ref = ref > 0.0f ? ref : 0.0f;
            const double err = fabs((double)h[o] - ref);
            worst = fmax(worst, err / mag);
            bad += err > 1e-5 * mag;
          }
    CHECK(bad == 0, "conv + residual + relu: %d outputs outside 1e-5 * mag (worst %.3g)", bad, worst);
    printf("conv + residual + relu (res_arg) vs oracle: worst |err|/mag = %.3g\n", worst);
    free(h); free(hx); free(hw); free(hr); free(conv);
    hipFree(X); hipFree(Wt); hipFree(R); hipFree(D1); hipFree(D2); hipFree(I); hipFree(O);
  }
}

int main(int argc, char **argv) {
  if (argc != 2 || (strcmp(argv[1], "validate") && strcmp(argv[1], "gpu"))) {
    fprintf(stderr, "usage: %s validate|gpu\n", argv[0]);
    return 2;
  }
  if (!strcmp(argv[1], "validate"))
    validate();
  else
    gpu();
  printf("%s: %d failure(s)\n", argv[1], failures);
  return failures ? 1 : 0;
}
