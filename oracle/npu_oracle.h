/*
 * npu_oracle.h -- CPU restatement of the reference's only execution path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP
 * product path.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  Nothing in the shipped library links it.
 *
 * What it restates.  The reference runs a fused group on the CPU by lowering
 * linalg with `mlir-opt --convert-linalg-to-loops --convert-scf-to-cf ...
 * --convert-func-to-llvm` and JIT-running it with `mlir-runner`
 * (tools/harness/e2e_verify.py:232-251).  convert-linalg-to-loops emits one
 * scalar loop nest per linalg op, loops in iteration-domain order, the
 * reduction loops innermost and sequential, and the body's arith ops one at a
 * time (no fused multiply-add: built with -ffp-contract=off, no fast-math).
 * Each function below is one such loop nest, and cites the op form it
 * follows.  Every op is unfused: each writes its whole output before the
 * next op runs, exactly as the lowered, bufferized function does.
 *
 * Element types.  The reference's tests are f16 text that the harness
 * rewrites to f32 before running (e2e_verify.py:164), so f32 is the native
 * form.  bf16 values are carried as uint16_t bit patterns; a linalg named op
 * with bf16 inputs and an f32 init extends each input (arith.extf, exact) and
 * accumulates in f32.  int8 convolutions extend to i32 (arith.extsi).
 *
 * Parity status of each function is recorded next to it: "pinned" means a
 * known-answer test from the reference or a mathematical check covers it in
 * tests/test_oracle.py.
 */
#ifndef NPU_ORACLE_H
#define NPU_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- elementary linalg ops -------------------------------------------- */

/* linalg.fill (test/matmul_relu.mlir:9).  pinned (KAT fills). */
void orc_fill_f32(float *out, int64_t n, float v);

/* linalg.matmul (test/matmul_relu.mlir:10-11): C[m,n] += A[m,k]*B[k,n],
 * loops m,n,k.  Leading dimensions allow memref.subview operands as used by
 * the tiled KAT (tools/harness/numerical_verify.py:160-190).  pinned. */
void orc_matmul_f32(const float *A, int64_t lda, const float *B, int64_t ldb,
                    float *C, int64_t ldc, int64_t M, int64_t N, int64_t K);

/* linalg.matmul with bf16 ins and an f32 init (extf then mulf/addf). pinned. */
void orc_matmul_bf16_f32(const uint16_t *A, int64_t lda, const uint16_t *B,
                         int64_t ldb, float *C, int64_t ldc, int64_t M,
                         int64_t N, int64_t K);

/* M-tiled matmul: scf.for over M with subviews of A and C
 * (numerical_verify.py:160-190).  pinned (must equal untiled bit for bit). */
void orc_matmul_tiled_m_f32(const float *A, const float *B, float *C,
                            int64_t M, int64_t N, int64_t K, int64_t tile_m);

/* linalg.batch_matmul (test/lit/batch_matmul_tiling.mlir:10-11):
 * C[b,m,n] += A[b,m,k]*B[b,k,n].  pinned. */
void orc_batch_matmul_f32(const float *A, const float *B, float *C,
                          int64_t Bt, int64_t M, int64_t N, int64_t K);

/* linalg.generic elementwise bodies (test/matmul_relu.mlir:15-25,
 * test/mobilenet_block.mlir:81-91).  pinned. */
void orc_relu_f32(const float *in, float *out, int64_t n);   /* maximumf(x,0) */
void orc_relu6_f32(const float *in, float *out, int64_t n);  /* minimumf(maximumf(x,0),6) */
void orc_add_f32(const float *a, const float *b, float *out, int64_t n);
/* broadcast add, indexing map (d0,d1)->(d1): out[r,c] = in[r,c] + v[c]. */
void orc_bias_add_f32(const float *in, const float *bias, float *out,
                      int64_t rows, int64_t cols);
/* silu(g)*u = g / (1 + exp(-g)) * u. */
void orc_silu_mul_f32(const float *g, const float *u, float *out, int64_t n);

/* tensor.pad with a constant (test/conv2d_relu.mlir:13-16 uses NCHW
 * low[0,0,1,1] high[0,0,1,1]).  pinned. */
void orc_pad_nchw_f32(const float *in, float *out, int64_t N, int64_t C,
                      int64_t H, int64_t W, int64_t pt, int64_t pb,
                      int64_t pl, int64_t pr, float v);
void orc_pad_nhwc_f32(const float *in, float *out, int64_t N, int64_t H,
                      int64_t W, int64_t C, int64_t pt, int64_t pb,
                      int64_t pl, int64_t pr, float v);
void orc_pad_nhwc_u16(const uint16_t *in, uint16_t *out, int64_t N, int64_t H,
                      int64_t W, int64_t C, int64_t pt, int64_t pb,
                      int64_t pl, int64_t pr);
void orc_pad_nhwc_i8(const int8_t *in, int8_t *out, int64_t N, int64_t H,
                     int64_t W, int64_t C, int64_t pt, int64_t pb, int64_t pl,
                     int64_t pr);

/* linalg.conv_2d_nchw_fchw (test/conv2d_relu.mlir:21-25) on a pre-padded
 * input, loops n,f,oh,ow,c,kh,kw.  pinned (KAT). */
void orc_conv2d_nchw_fchw_f32(const float *in, const float *w, float *out,
                              int64_t N, int64_t C, int64_t Hp, int64_t Wp,
                              int64_t F, int64_t KH, int64_t KW, int64_t SH,
                              int64_t SW);

/* linalg.conv_2d_nhwc_fhwc on a pre-padded input, loops n,oh,ow,f,kh,kw,c:
 * O[n,oh,ow,f] += I[n,oh*SH+kh,ow*SW+kw,c] * W[f,kh,kw,c].  Not in the
 * reference (NCHW only); pinned against the NCHW op by transposition. */
void orc_conv2d_nhwc_fhwc_f32(const float *in, const float *w, float *out,
                              int64_t N, int64_t Hp, int64_t Wp, int64_t C,
                              int64_t F, int64_t KH, int64_t KW, int64_t SH,
                              int64_t SW);
void orc_conv2d_nhwc_fhwc_bf16_f32(const uint16_t *in, const uint16_t *w,
                                   float *out, int64_t N, int64_t Hp,
                                   int64_t Wp, int64_t C, int64_t F,
                                   int64_t KH, int64_t KW, int64_t SH,
                                   int64_t SW);
void orc_conv2d_nhwc_fhwc_i8_i32(const int8_t *in, const int8_t *w,
                                 int32_t *out, int64_t N, int64_t Hp,
                                 int64_t Wp, int64_t C, int64_t F, int64_t KH,
                                 int64_t KW, int64_t SH, int64_t SW);

/* linalg.depthwise_conv_2d_nhwc_hwc, loops n,oh,ow,c,kh,kw:
 * O[n,oh,ow,c] += I[n,oh*SH+kh,ow*SW+kw,c] * W[kh,kw,c].  Not in the
 * reference (it models depthwise as a full conv, test/mobilenet_block.mlir:45-53);
 * pinned against a full conv with a block-diagonal filter. */
void orc_depthwise_conv2d_nhwc_hwc_f32(const float *in, const float *w,
                                       float *out, int64_t N, int64_t Hp,
                                       int64_t Wp, int64_t C, int64_t KH,
                                       int64_t KW, int64_t SH, int64_t SW);

/* arith.truncf f32->bf16 (round to nearest even) and arith.extf. pinned. */
void orc_trunc_f32_bf16(const float *in, uint16_t *out, int64_t n);
void orc_ext_bf16_f32(const uint16_t *in, float *out, int64_t n);

/* Fixed-point requantisation, TOSA apply_scale_32 with double_round=false:
 * r = (int64(acc)*mult[c] + (1 << (shift[c]-1))) >> shift[c] (arithmetic
 * shift), per channel c = index % cols.  pinned (big-integer closed form). */
void orc_apply_scale_i32(const int32_t *acc, const int32_t *mult,
                         const int32_t *shift, int32_t *out, int64_t rows,
                         int64_t cols);
void orc_add_i32(const int32_t *a, const int32_t *b, int32_t *out, int64_t n);
void orc_add_i32_i8(const int32_t *a, const int8_t *b, int32_t *out, int64_t n);
/* clamp to [lo,hi] then trunci to i8 (ReLU folds into lo = 0). */
void orc_clamp_i32_i8(const int32_t *in, int8_t *out, int64_t n, int32_t lo,
                      int32_t hi);

/* RMSNorm (Zhang & Sennrich 2019): ms = sum_j x_j*x_j / d (sequential f32),
 * inv = 1/sqrtf(ms + eps), y_j = (x_j * inv) * g_j.  Not in the reference;
 * pinned against the defining formula in float64. */
void orc_rmsnorm_f32(const float *x, const float *g, float *out, int64_t rows,
                     int64_t d, float eps);

/* Rotary embedding (Su et al. 2021), interleaved pairs (2i, 2i+1) of each
 * head, rotated by a position/frequency table:  x [S][H*Dh],
 * cos/sin [S][Dh/2].  y0 = x0*c - x1*s ; y1 = x0*s + x1*c.  pinned
 * (position 0 is the identity, rotation preserves pair norms). */
void orc_rope_f32(const float *x, const float *cos_t, const float *sin_t,
                  float *out, int64_t S, int64_t H, int64_t Dh);

/* Causal row softmax over scores [rows][cols] (in place), query row i
 * attends to keys j <= i + (cols - rows): m = max, e = expf(s - m),
 * p = e / sum(e); masked entries become 0. pinned (rows sum to 1, matches
 * float64 softmax). */
void orc_causal_softmax_f32(float *s, int64_t rows, int64_t cols);

/* ---- composite blocks: the authored linalg chain of each fused group ----
 * Each is the unfused sequence of the ops above, with intermediates in
 * host memory, i.e. what the lowered function does before any fusion. */

/* C1: fill(0) -> matmul -> bias add -> relu.  A[M,K], B[K,N], bias[N]. */
void orc_block_matmul_bias_act_f32(const float *A, const float *B,
                                   const float *bias, float *out, int64_t M,
                                   int64_t N, int64_t K, int act);

/* C2: pad NHWC -> fill(0) -> conv_2d_nhwc_fhwc -> bias add -> act.
 * act: 0 none, 1 relu, 2 relu6.  x[N,H,W,C], w[F,KH,KW,C], stride 1. */
void orc_block_conv_bias_act_f32(const float *x, const float *w,
                                 const float *bias, float *out, int64_t N,
                                 int64_t H, int64_t W, int64_t C, int64_t F,
                                 int64_t KH, int64_t KW, int64_t pad, int act);
/* same with bf16 x, w (fp32 accumulate), fp32 bias, bf16 out (truncf). */
void orc_block_conv_bias_act_bf16(const uint16_t *x, const uint16_t *w,
                                  const float *bias, uint16_t *out, int64_t N,
                                  int64_t H, int64_t W, int64_t C, int64_t F,
                                  int64_t KH, int64_t KW, int64_t pad, int act);

/* C3: MobileNetV2 inverted residual, fp32, NHWC:
 * e = relu6(conv1x1(x, we));  d = relu6(dw3x3(pad(e), wdw));
 * out = conv1x1(d, wp) + x.   x[N,H,W,C], we[E,C], wdw[3,3,E], wp[C,E]. */
void orc_block_irb_f32(const float *x, const float *we, const float *wdw,
                       const float *wp, float *out, int64_t N, int64_t H,
                       int64_t W, int64_t C, int64_t E);

/* C4: int8 bottleneck, NHWC, zero points 0:
 * y1 = clamp(apply_scale(conv1x1(x, w1), m1, s1), 0, 127)
 * y2 = clamp(apply_scale(conv3x3(pad(y1), w2), m2, s2), 0, 127)
 * out = clamp(apply_scale(conv1x1(y2, w3), m3, s3) + x, 0, 127)
 * x[N,H,W,C], w1[M1,C], w2[M1,3,3,M1], w3[C,M1]. */
void orc_block_qbottleneck_i8(const int8_t *x, const int8_t *w1,
                              const int8_t *w2, const int8_t *w3,
                              const int32_t *m1, const int32_t *s1,
                              const int32_t *m2, const int32_t *s2,
                              const int32_t *m3, const int32_t *s3,
                              int8_t *out, int64_t N, int64_t H, int64_t W,
                              int64_t C, int64_t M1);

/* C5 sub-groups of one Llama decoder layer (bf16 storage, f32 compute).
 * x[S,D]; wq/wk/wv/wo[D,D]; wg/wu[D,F]; wd[F,D]; gamma f32[D];
 * cos/sin f32[S,Dh/2].  Rounding to bf16 happens only at sub-group
 * outputs and at matmul inputs (the normalised activations). */
/* K5a: xn = bf16(rmsnorm(x, g1)); Q = bf16(rope(xn@wq)); K = bf16(rope(xn@wk));
 * V = bf16(xn@wv).  Q/K/V are [S, H*Dh] row-major. */
void orc_llama_qkv_bf16(const uint16_t *x, const float *g1, const uint16_t *wq,
                        const uint16_t *wk, const uint16_t *wv,
                        const float *cos_t, const float *sin_t, uint16_t *Q,
                        uint16_t *K, uint16_t *V, int64_t S, int64_t D,
                        int64_t H, float eps);
/* K5b: per head h: s = (Q_h @ K_h^T) * scale, causal softmax (f32),
 * A_h = bf16(p @ V_h).  A is [S, H*Dh]. */
void orc_llama_attention_bf16(const uint16_t *Q, const uint16_t *K,
                              const uint16_t *V, uint16_t *A, int64_t S,
                              int64_t H, int64_t Dh, float scale);
/* K5c / K5e: out = bf16(res + a @ w), a[S,Kd] bf16, w[Kd,N] bf16, res[S,N] bf16. */
void orc_llama_matmul_residual_bf16(const uint16_t *a, const uint16_t *w,
                                    const uint16_t *res, uint16_t *out,
                                    int64_t S, int64_t N, int64_t Kd);
/* K5d: hn = bf16(rmsnorm(h, g2)); act = bf16(silu(hn@wg) * (hn@wu)). */
void orc_llama_swiglu_bf16(const uint16_t *h, const float *g2,
                           const uint16_t *wg, const uint16_t *wu,
                           uint16_t *act, int64_t S, int64_t D, int64_t F,
                           float eps);
/* Whole layer: K5a -> K5b -> K5c -> K5d -> K5e.  h (bf16 [S,D]) receives
 * the post-attention residual stream, out the layer output. */
void orc_block_llama_layer_bf16(const uint16_t *x, const float *g1,
                                const float *g2, const uint16_t *wq,
                                const uint16_t *wk, const uint16_t *wv,
                                const uint16_t *wo, const uint16_t *wg,
                                const uint16_t *wu, const uint16_t *wd,
                                const float *cos_t, const float *sin_t,
                                uint16_t *h, uint16_t *out, int64_t S,
                                int64_t D, int64_t H, int64_t F, float eps);

#ifdef __cplusplus
}
#endif
#endif
