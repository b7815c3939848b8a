/* The compiled host side of test/matmul_relu.mlir after
 * `npu-opt --npu-fusion --npu-outline-fused-groups`, written in C the way
 * MLIR lowers that module's parent function: the tile-and-fuse loop over
 * 16-row tiles (FusionPass.cpp:306-359), each trip taking memref.subview
 * descriptors of A, the fill's destination and the output, and calling the
 * outlined kernel through its C interface,
 *   _mlir_ciface_fused_fill_matmul_generic_0(&result, fill, init, A, B, out)
 * (the function npu_amd.ciface generates for the module and this program
 * links as libciface_shim.so; tools/harness/e2e_verify.py:221 for the
 * llvm.emit_c_interface convention).
 *
 *   ciface_test validate   a bad descriptor is refused before any launch
 *                          and reported through npu_ciface_status (no GPU)
 *   ciface_test gpu        the eight tile calls on device 0: the harness's
 *                          fills give 0.0512 everywhere (e2e_verify.py:
 *                          288-309); seeded inputs match the oracle's loops
 * Exit status 0 when every check passes. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "../../include/npu_amd.h"
#include "../../oracle/npu_oracle.h"

/* the generated shim */
void _mlir_ciface_fused_fill_matmul_generic_0(npu_strided_memref_2d *result, float a0,
                                              npu_strided_memref_2d *a1,
                                              npu_strided_memref_2d *a2,
                                              npu_strided_memref_2d *a3,
                                              npu_strided_memref_2d *a4);
void npu_ciface_set_stream(npu_stream s);
npu_status npu_ciface_status(void);
const char *npu_ciface_error(void);
void npu_ciface_clear(void);

enum { M = 128, K = 256, N = 512, TM = 16 };

static int failures = 0;

#define CHECK(cond, ...)                                   \
  do {                                                     \
    if (!(cond)) {                                         \
      fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
      fprintf(stderr, __VA_ARGS__);                        \
      fprintf(stderr, "\n");                               \
      ++failures;                                          \
    }                                                      \
  } while (0)

/* memref.subview %base[off, 0] [rows, cols] [1, 1] of a row-major [.., ld] buffer */
static npu_strided_memref_2d subview(float *base, int64_t row0, int64_t rows, int64_t cols,
                                     int64_t ld) {
  npu_strided_memref_2d d;
  d.allocated = d.aligned = base;
  d.offset = row0 * ld;
  d.sizes[0] = rows;
  d.sizes[1] = cols;
  d.strides[0] = ld;
  d.strides[1] = 1;
  return d;
}

/* the parent function's loop: scf.for %i = 0 to 128 step 16 */
static void host_module(float *A, float *B, float *init, float *out) {
  npu_strided_memref_2d b = subview(B, 0, K, N, N);
  for (int64_t i = 0; i < M; i += TM) {
    npu_strided_memref_2d a = subview(A, i, TM, K, K);
    npu_strided_memref_2d c = subview(init, i, TM, N, N);
    npu_strided_memref_2d o = subview(out, i, TM, N, N);
    npu_strided_memref_2d r;
    _mlir_ciface_fused_fill_matmul_generic_0(&r, 0.0f, &c, &a, &b, &o);
    CHECK(r.aligned == out && r.offset == i * N && r.sizes[0] == TM && r.sizes[1] == N,
          "tile %ld: result descriptor is not the output slice", (long)i);
  }
}

static void validate(void) {
  float *A = (float *)0x100000, *B = (float *)0x200000, *I = (float *)0x300000;
  float *O = (float *)0x400000;  /* never dereferenced: the call is refused */
  npu_strided_memref_2d a = subview(A, 0, TM, K - 4, K - 4);  /* K mismatch */
  npu_strided_memref_2d b = subview(B, 0, K, N, N);
  npu_strided_memref_2d c = subview(I, 0, TM, N, N);
  npu_strided_memref_2d o = subview(O, 0, TM, N, N), r;
  npu_ciface_clear();
  _mlir_ciface_fused_fill_matmul_generic_0(&r, 0.0f, &c, &a, &b, &o);
  CHECK(npu_ciface_status() == NPU_ERR_INVALID_ARG, "K mismatch: status %d (%s)",
        npu_ciface_status(), npu_ciface_error());
  CHECK(strstr(npu_ciface_error(), "fused_fill_matmul_generic_0") != NULL, "message: %s",
        npu_ciface_error());
  /* a nonzero fill is refused at the launch, as the kernel's value */
  a = subview(A, 0, TM, K, K);
  npu_ciface_clear();
  _mlir_ciface_fused_fill_matmul_generic_0(&r, 1.0f, &c, &a, &b, &o);
  CHECK(npu_ciface_status() == NPU_ERR_UNSUPPORTED, "fill 1.0: status %d (%s)",
        npu_ciface_status(), npu_ciface_error());
  npu_ciface_clear();
}

static uint64_t lcg = 0x4E505500u;
static float uniform(void) {
  lcg = lcg * 6364136223846793005ull + 1442695040888963407ull;
  return (float)((lcg >> 40) * (1.0 / 16777216.0)) * 2.0f - 1.0f;
}

static void gpu(void) {
  float *hA = malloc(sizeof(float) * M * K), *hB = malloc(sizeof(float) * K * N);
  float *hO = malloc(sizeof(float) * M * N), *ref = malloc(sizeof(float) * M * N);
  float *A, *B, *I, *O;
  hipMalloc((void **)&A, sizeof(float) * M * K);
  hipMalloc((void **)&B, sizeof(float) * K * N);
  hipMalloc((void **)&I, sizeof(float) * M * N);
  hipMalloc((void **)&O, sizeof(float) * M * N);
  hipStream_t s;
  hipStreamCreate(&s);
  npu_ciface_set_stream(s);
  for (int pass = 0; pass < 2; ++pass) {
    for (int64_t j = 0; j < M * K; ++j) hA[j] = pass ? uniform() : 0.01f;
    for (int64_t j = 0; j < K * N; ++j) hB[j] = pass ? uniform() : 0.02f;
    hipMemcpy(A, hA, sizeof(float) * M * K, hipMemcpyHostToDevice);
    hipMemcpy(B, hB, sizeof(float) * K * N, hipMemcpyHostToDevice);
    hipMemset(O, 0xff, sizeof(float) * M * N);  /* NaN: every element must be written */
    npu_ciface_clear();
    host_module(A, B, I, O);
    hipStreamSynchronize(s);
    CHECK(npu_ciface_status() == NPU_OK, "launch failed: %s", npu_ciface_error());
    hipMemcpy(hO, O, sizeof(float) * M * N, hipMemcpyDeviceToHost);
    orc_fill_f32(ref, M * N, 0.0f);
    orc_matmul_f32(hA, K, hB, N, ref, N, M, N, K);
    int bad = 0;
    for (int64_t j = 0; j < M * N; ++j) {
      const double r = ref[j] > 0 ? ref[j] : 0.0;  /* the generic's ReLU */
      double mag = 0;
      for (int64_t k = 0; k < K; ++k)
        mag += fabs((double)hA[(j / N) * K + k] * hB[k * N + j % N]);
      if (!(fabs(hO[j] - r) <= 1e-5 * mag + 1e-30)) ++bad;
      if (pass == 0 && !(fabs(hO[j] - 0.0512) <= 1e-4 * 0.0512)) ++bad;
    }
    CHECK(bad == 0, "%s inputs: %d of %d outputs outside the bound", pass ? "seeded" : "harness",
          bad, M * N);
  }
  hipStreamDestroy(s);
  hipFree(A);
  hipFree(B);
  hipFree(I);
  hipFree(O);
  free(hA);
  free(hB);
  free(hO);
  free(ref);
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
