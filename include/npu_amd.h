/*
 * npu_amd.h -- C-ABI of the MI355X (gfx950) execution backend for the fused
 * tile groups produced by NPU-Dialect's npu-fusion / npu-outline-fused-groups
 * / npu-spatial-tiling / npu-temporal-tiling / npu-bufferize pipeline.
 *
 * The unit of execution is one outlined group, i.e. one
 *   func.func private @fused_<ops>_<idx>(ext inputs...) -> (ext outputs...)
 *       attributes {npu.fused_kernel}
 * (lib/Transforms/OutlineFusedGroupsPass.cpp:259-283) together with the
 * spatial / temporal tile loops wrapped around its func.call
 * (lib/Transforms/FusionPass.cpp:330-357, SpatialTilingPass.cpp:146-166,
 * OutlineFusedGroupsPass.cpp:306-316).  One call here replaces the whole
 * tile-loop nest: the loop bounds become the launch grid.
 *
 * Conventions (all entry points):
 *  - Buffers are device pointers in HBM, owned by the caller
 *    (destination-passing style, as linalg's `outs`, test/matmul_relu.mlir:10-11;
 *    the caller allocates, tools/harness/e2e_verify.py:195-203).  The library
 *    never frees caller memory.
 *  - Every call is asynchronous on the caller's HIP stream (`npu_stream` is a
 *    hipStream_t; NULL = the null stream).  Launches on distinct streams may
 *    run concurrently; the library keeps no per-call device state.
 *  - Errors are returned as npu_status; nothing throws across the ABI.  Shape,
 *    dtype and layout mismatches are rejected before any launch, and
 *    npu_last_error() (thread-local) says why.  Every dimension must be
 *    positive: a memref with a zero-sized dimension is rejected with
 *    NPU_ERR_INVALID_ARG (the reference's groups have static, nonzero
 *    shapes; nothing is launched for such a call).
 *  - No entry point allocates device memory.
 */
#ifndef NPU_AMD_H
#define NPU_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------------- */
/* Status codes.  Replace the reference's diagnostics / exit codes
 * (lib/Transforms/BufferizePass.cpp:63-65, tools/npu-opt/npu-opt.cpp:65-66). */
typedef int32_t npu_status;
#define NPU_OK 0
#define NPU_ERR_INVALID_ARG 1  /* null pointer, bad rank/shape/dtype       */
#define NPU_ERR_UNSUPPORTED 2  /* valid linalg, not handled by a kernel     */
#define NPU_ERR_HIP 3          /* a HIP runtime call failed                 */
#define NPU_ERR_OOM 4          /* reserved: no entry point allocates        */

typedef void *npu_stream; /* hipStream_t */

/* Element types of memref descriptors. */
#define NPU_F32 0
#define NPU_BF16 1
#define NPU_I8 2
#define NPU_I32 3

#define NPU_MAX_RANK 4

/* Strided memref descriptor: the field order of MLIR's ranked memref C
 * interface ({allocated, aligned, offset, sizes[R], strides[R]}, which the
 * reference harness relies on through llvm.emit_c_interface,
 * tools/harness/e2e_verify.py:221), at a fixed maximum rank, followed by the
 * rank and element type.  Offsets and strides are in elements.  Kernels
 * require the row-major contiguous layout of their operand; other layouts are
 * rejected with NPU_ERR_UNSUPPORTED. */
typedef struct npu_memref {
  void *allocated;
  void *aligned;
  int64_t offset;
  int64_t sizes[NPU_MAX_RANK];
  int64_t strides[NPU_MAX_RANK];
  int32_t rank;
  int32_t dtype;
} npu_memref;

/* Epilogue activation of a `linalg.generic` consumer. */
#define NPU_ACT_NONE 0
#define NPU_ACT_RELU 1  /* arith.maximumf(x, 0), test/matmul_relu.mlir:15-25 */
#define NPU_ACT_RELU6 2 /* minimumf(maximumf(x, 0), 6)                        */

/* ---------------------------------------------------------------------- */
/* Library information and errors. */
const char *npu_version(void);
const char *npu_last_error(void);
const char *npu_status_string(npu_status s);
/* Number of visible HIP devices (0 when none), or -1 when the runtime fails. */
int32_t npu_device_count(void);

/* ---------------------------------------------------------------------- */
/* Fused-group entry points.  Each names the op chain of the outlined group it
 * replaces; the outliner's own symbol is `fused_` + the short op names +
 * `_<idx>` (OutlineFusedGroupsPass.cpp:69-82, 259-263).  The mapping from
 * outlined chains to these entry points is the group classifier of the
 * host lowering. */

/* Group `fill -> matmul -> generic(bias add, act)`
 * (test/matmul_relu.mlir:6-28 plus a broadcast bias; outlined as
 * @fused_fill_matmul_generic_<idx> after elementwise fusion,
 * FusionPass.cpp:458-499).
 *   A    f32 [M,K]      B f32 [K,N]      bias f32 [N] (aligned may be NULL: no bias)
 *   out  f32 [M,N] = act(A @ B + bias)
 * Requires K % 4 == 0. */
npu_status fused_matmul_bias_act(const npu_memref *A, const npu_memref *B,
                                 const npu_memref *bias, const npu_memref *out,
                                 int32_t act, npu_stream stream);

/* Group `pad -> fill -> conv_2d_nhwc_fhwc -> generic(bias add, act)`
 * (NHWC restatement of test/conv2d_relu.mlir:7-42; the zero pad is folded
 * into predicated halo loads instead of a materialised tensor.pad).
 *   x    [N,H,W,C]  f32 or bf16      w [F,KH,KW,C] same dtype
 *   bias f32 [F] (aligned may be NULL)
 *   out  [N,Ho,Wo,F] same dtype as x (bf16: fp32 accumulate, one rounding)
 * Stride 1, symmetric zero padding `pad`; Ho = H + 2*pad - KH + 1.
 * Requires C % 4 == 0 (f32) / C % 8 == 0 (bf16).
 * f32 results are within f32 accuracy of the sequential f32 sum (the
 * parity bound 1e-5 * sum |x w|), with +-Inf and NaN where the f32 loops give
 * them.  3x3 / pad-1 launches with 32 or 64 channels, F % 64 == 0 and at
 * least 48 row pairs (N * ceil(H/2) >= 48) compute the products on the bf16
 * matrix pipe from exact three-part bf16 splits of every value.  The split
 * is exact for zero and magnitudes in [2^-55, 2^55); a launch in which an
 * input or filter value lies outside that (Inf, NaN, |v| >= 2^55,
 * 0 < |v| < 2^-55) or a bias is an f32 subnormal recomputes the rows that
 * value's workgroup owns on a scalar path bit-identical to the sequential
 * f32 loops -- correct, but about two orders of magnitude slower for those
 * rows. */
npu_status fused_conv2d_nhwc_bias_act(const npu_memref *x, const npu_memref *w,
                                      const npu_memref *bias,
                                      const npu_memref *out, int32_t pad,
                                      int32_t act, npu_stream stream);

/* The same group with a residual term in its generic:
 * `fill -> conv_2d -> generic(conv + bias + res, act)`, the residual add of a
 * ResNet block and of the projection conv of an inverted residual block
 * (test/resnet_block.mlir, test/models/mobilenetv2.mlir:211-226, where the
 * generic adds the block's input to the last convolution).
 *   res  [N,Ho,Wo,F] same dtype as out
 *   out  = act(conv(x, w) + bias + res), f32 sums, bf16: one rounding
 * Same limits as fused_conv2d_nhwc_bias_act. */
npu_status fused_conv2d_nhwc_bias_res_act(const npu_memref *x, const npu_memref *w,
                                          const npu_memref *bias, const npu_memref *res,
                                          const npu_memref *out, int32_t pad, int32_t act,
                                          npu_stream stream);

/* The reference's own layout: group `pad -> fill -> conv_2d_nchw_fchw ->
 * generic...` (test/conv2d_relu.mlir:7-42, test/resnet_block.mlir,
 * test/resnet50_block.mlir, test/mobilenet_block.mlir, and every network of
 * test/models/, e.g. resnet18.mlir; outlined as
 * @fused_fill_conv2d[_generic...]_<idx>, OutlineFusedGroupsPass.cpp:69-82),
 * with the zero pad folded into the launch.  f32 (f16 text runs as f32,
 * tools/harness/e2e_verify.py:163-164).
 *   x    f32 [N,C,H,W]       w f32 [F,C,KH,KW], any KH, KW
 *   bias f32 [F] (aligned may be NULL)
 *   out  f32 [N,F,Ho,Wo] = act(conv(pad(x), w, stride) + bias),
 *        Ho = (H + 2*pad - KH) / stride + 1 (the `strides` attribute, the
 *        same in both dimensions)
 * 1x1 and 3x3 filters at stride 1 or 2 stage their halo in LDS; other shapes
 * read their operands directly.  Computed on the f32 matrix pipe: within f32
 * accuracy of the sequential f32 sum, +-Inf and NaN as there. */
npu_status fused_conv2d_nchw_bias_act(const npu_memref *x, const npu_memref *w,
                                      const npu_memref *bias, const npu_memref *out,
                                      int32_t pad, int32_t stride, int32_t act,
                                      npu_stream stream);

/* The same with the residual term of a ResNet block's add generic
 * (test/resnet_block.mlir:55-67, test/resnet50_block.mlir:77-102):
 *   res  f32 [N,F,Ho,Wo]     out = act(conv(pad(x), w, stride) + bias + res) */
npu_status fused_conv2d_nchw_bias_res_act(const npu_memref *x, const npu_memref *w,
                                          const npu_memref *bias, const npu_memref *res,
                                          const npu_memref *out, int32_t pad, int32_t stride,
                                          int32_t act, npu_stream stream);

/* Group chain of the int8 ResNet-50 bottleneck (int8 restatement of
 * test/resnet50_block.mlir:5-105, NHWC, zero points 0), fused across both
 * tensor.pads into one launch:
 *   y1  = clamp(apply_scale(conv1x1(x, w1), m1, s1), 0, 127)
 *   y2  = clamp(apply_scale(conv3x3(pad1(y1), w2), m2, s2), 0, 127)
 *   out = clamp(apply_scale(conv1x1(y2, w3), m3, s3) + x, 0, 127)
 * apply_scale is TOSA apply_scale_32 with single rounding:
 *   (int64(acc) * m + (1 << (s - 1))) >> s, per output channel.
 *   x i8 [N,H,W,C]; w1 i8 [M1,C]; w2 i8 [M1,3,3,M1]; w3 i8 [C,M1];
 *   m1,s1,m2,s2 i32 [M1]; m3,s3 i32 [C]; out i8 [N,H,W,C].
 * (C, M1) = (256,64), (128,64), (64,64) run on kernels tuned for them; any
 * other C and M1 that are multiples of 64 with C <= 2048 and M1 <= 512 on a
 * kernel that reads its filter blocks from L2 where they are used; other
 * counts return NPU_ERR_UNSUPPORTED.  Precondition (TOSA): every shift is in
 * [2, 62]. */
npu_status fused_qbottleneck_i8(const npu_memref *x, const npu_memref *w1,
                                const npu_memref *w2, const npu_memref *w3,
                                const npu_memref *m1, const npu_memref *s1,
                                const npu_memref *m2, const npu_memref *s2,
                                const npu_memref *m3, const npu_memref *s3,
                                const npu_memref *out, npu_stream stream);

/* Group chain of the MobileNetV2 inverted residual block (NHWC restatement
 * of test/mobilenet_block.mlir:8-94 with a true depthwise stage), fused
 * across the tensor.pad into one launch, f32:
 *   e   = relu6(conv1x1(x, we))
 *   d   = relu6(depthwise_conv_2d_nhwc_hwc(pad1(e), wdw))
 *   out = conv1x1(d, wp) + x
 *   x f32 [N,H,W,C]; we f32 [E,C]; wdw f32 [3,3,E]; wp f32 [C,E];
 *   out f32 [N,H,W,C].
 * (C, E) = (24,144), (16,96), (32,192) run on kernels tuned for them; any
 * other C % 4 == 0, 4 <= C <= 320 with E % 16 == 0 on a kernel that streams
 * the expanded channels in chunks of 16 (filters read from L2 per chunk);
 * other channel counts return NPU_ERR_UNSUPPORTED. */
npu_status fused_irb_f32(const npu_memref *x, const npu_memref *we,
                         const npu_memref *wdw, const npu_memref *wp,
                         const npu_memref *out, npu_stream stream);

/* Groups of one Llama decoder layer (bf16 storage, f32 accumulation and
 * elementwise math; bf16 rounding at each group output and at the
 * normalised matmul inputs).  The reference's llama_attention.mlir:5-67
 * replaces softmax by ReLU and has no RMSNorm, RoPE or gating; these groups
 * implement the real layer.  Row-major [S, D] activations, D = H * Dh with
 * head dim Dh = 64 or 128, weights [K, N] as linalg.matmul takes them.  Any
 * sequence length S; the matmul groups require K % 64 == 0 and N % 64 == 0.
 *
 * QKV: xn = bf16(rmsnorm(x) * g1) with inv = 1/sqrt(mean(x^2) + eps);
 *      Q = bf16(rope(xn @ wq)), K = bf16(rope(xn @ wk)), V = bf16(xn @ wv).
 *      RoPE rotates interleaved pairs (2t, 2t+1) of each Dh-wide head by the
 *      tables cos_t / sin_t f32 [S, Dh / 2] (their width gives Dh). */
npu_status fused_llama_qkv_rope(const npu_memref *x, const npu_memref *g1,
                                const npu_memref *wq, const npu_memref *wk,
                                const npu_memref *wv, const npu_memref *cos_t,
                                const npu_memref *sin_t, const npu_memref *Q,
                                const npu_memref *K, const npu_memref *V,
                                float eps, npu_stream stream);
/* Causal attention per head (head dim Dh = D / n_heads, 64 or 128):
 * A = bf16(softmax(Q K^T * scale with keys j <= i) @ V).  Q, K, V, A bf16
 * [S, D]. */
npu_status fused_llama_attention(const npu_memref *Q, const npu_memref *K,
                                 const npu_memref *V, const npu_memref *A,
                                 int32_t n_heads, float scale,
                                 npu_stream stream);
/* out = bf16(res + a @ w); a [S, K], w [K, N], res and out [S, N]. */
npu_status fused_llama_matmul_residual(const npu_memref *a, const npu_memref *w,
                                       const npu_memref *res,
                                       const npu_memref *out, npu_stream stream);
/* hn = bf16(rmsnorm(h) * g2); act = bf16(silu(hn @ wg) * (hn @ wu));
 * h [S, D], wg / wu [D, F], act [S, F]. */
npu_status fused_llama_rmsnorm_swiglu(const npu_memref *h, const npu_memref *g2,
                                      const npu_memref *wg, const npu_memref *wu,
                                      const npu_memref *act, float eps,
                                      npu_stream stream);

/* ---- the reference's SRAM plan as the LDS layout --------------------------
 * The group `fill -> matmul -> generic(bias add, act)` run as the tile loop
 * that npu-temporal-tiling and npu-bufferize make of it (per output tile of
 * tm x tn, a K loop of tk steps, each step a DMA of the A and B slices into
 * SRAM and a matmul into the SRAM accumulator; then the generic into the
 * output slice and its DMA back; BufferizePass.cpp:97-222), with every
 * buffer at the byte offset NPUSRAMAllocationPass's dual-end plan gives it
 * (SRAMAllocationPass.cpp:172-342: sram_offset, sram_offset_pong) in one
 * workgroup's LDS, in the slice's own row-major f32 layout.  Each K step is
 * one npu-barrier-alloc subgraph (DMASchedulingPass.cpp:92-147) and one
 * s_barrier; the step uses the ping buffers when even, the pong ones when
 * odd.  The plan is checked before the launch: every buffer inside
 * [0, lds_bytes), lds_bytes <= 163840 (the reference simulator's bound,
 * tools/harness/sram_simulator.py:243-256), no two buffers overlapping.
 * This path keeps the reference's layout and schedule; fused_matmul_bias_act
 * is the fast kernel for the same group. */
typedef struct npu_tile_plan {
  int32_t tm, tn, tk;      /* output tile rows, columns; K step            */
  int32_t lds_bytes;       /* SRAM (LDS) size the plan was made for         */
  int64_t off_a, off_a_pong; /* A slice [tm][tk]                            */
  int64_t off_b, off_b_pong; /* B slice [tk][tn]                            */
  int64_t off_bias;        /* bias slice [tn]; -1: the group has no bias    */
  int64_t off_c;           /* accumulator tile [tm][tn]                     */
  int64_t off_y;           /* output tile [tm][tn]                          */
} npu_tile_plan;
/* A f32 [M,K], B f32 [K,N], bias f32 [N] (aligned may be NULL), out f32
 * [M,N] = act(A @ B + bias).  Any tile sizes with at most 64 16x16 output
 * blocks per tile (ceil(tm/16) * ceil(tn/16) <= 64).  lds_dump (device memory of lds_bytes, may be
 * NULL) receives output tile (0, 0)'s whole LDS at the end: the layout the
 * launch used. */
npu_status npu_planned_matmul_bias_act(const npu_memref *A, const npu_memref *B,
                                       const npu_memref *bias, const npu_memref *out,
                                       int32_t act, const npu_tile_plan *plan,
                                       void *lds_dump, npu_stream stream);

/* The group `fill -> conv_2d_nchw_fchw -> generic(bias add, act)` as the
 * reference's temporal tile loop over output-channel tiles, every SRAM
 * buffer where the reference's SRAM plan puts it in one workgroup's LDS
 * (SRAMAllocationPass.cpp:172-363: sram_offset, sram_offset_pong,
 * double_buffered, prefetch_addr, spills).  A workgroup is one core's
 * share: one output row (n, ho).  Per tile i (output channels i*tco ..
 * +tco): the input rows [C][KH][Wp], the filter slice [tco][C][KH][KW]
 * and the bias slice [tco] in their ping (i even) or pong (i odd)
 * buffers, the tile's MACs into the accumulator row [tco][Wo], the
 * generic (bias slice, activation) into the output row, DMA'd back.  A
 * buffer with a prefetch region (prefetch_addr) has tile i+2's copy
 * fetched from HBM into it after tile i, and tile i+1's copy made
 * SRAM-to-SRAM from it (the reference's "next tile iteration's data in
 * free SRAM"); a buffer without a pong reuses its ping; spilled input rows
 * or filters (offset -1) are read from HBM where they lie; a bias, when
 * the group has one, is in SRAM.  Stride 1, no dilation; x is the padded
 * input [N][C][Hp][Wp].  The plan is checked before the launch: every
 * buffer 4-byte aligned inside [0, lds_bytes), lds_bytes <= 163840, no two
 * buffers overlapping, no pong or prefetch region for a buffer outside
 * SRAM. */
typedef struct npu_conv_tile_plan {
  int32_t tco;             /* output channels per temporal tile             */
  int32_t lds_bytes;       /* SRAM (LDS) size the plan was made for         */
  int64_t off_in, off_in_pong, off_in_prefetch;        /* rows [C][KH][Wp]  */
  int64_t off_w, off_w_pong, off_w_prefetch;     /* filters [tco][C][KH][KW] */
  int64_t off_bias, off_bias_pong, off_bias_prefetch;  /* bias [tco]; off_bias
                              -1: the group has no bias                    */
  int64_t off_c;           /* accumulator row [tco][Wo]                     */
  int64_t off_y;           /* output row [tco][Wo]                          */
} npu_conv_tile_plan;
/* x f32 [N,C,Hp,Wp] (padded), w f32 [F,C,KH,KW], bias f32 [F] (aligned may
 * be NULL), out f32 [N,F,Ho,Wo] = act(conv + bias), Ho = Hp-KH+1,
 * Wo = Wp-KW+1.  lds_dump (device memory of lds_bytes, may be NULL)
 * receives workgroup 0's (image 0, output row 0) whole LDS at the end. */
npu_status npu_planned_conv2d_nchw_bias_act(const npu_memref *x, const npu_memref *w,
                                            const npu_memref *bias, const npu_memref *out,
                                            int32_t act, const npu_conv_tile_plan *plan,
                                            void *lds_dump, npu_stream stream);

/* ---- the outlined-group boundary -----------------------------------------
 * A host module produced by the reference's pipeline calls each fused group
 * as `func.call @fused_<ops>_<idx>(external inputs...)` with the group's
 * external inputs in first-use order and its results after them
 * (OutlineFusedGroupsPass.cpp:218-257, 306-316); after bufferization the
 * shaped arguments are memrefs, passed through MLIR's memref C interface
 * (tools/harness/e2e_verify.py:221).  npu_group_launch is that call: it is
 * keyed by the outlined name and takes the arguments in that order.
 *
 * Descriptors: a ranked memref of rank R has MLIR's StridedMemRefType<T, R>
 * layout, declared below for R = 1..4 (the element type is not part of the
 * descriptor, as in MLIR); an argument is MLIR's UnrankedMemRefType
 * ({rank, descriptor}) followed by what the function type says of it: its
 * element type, and for a scalar argument (the `arith.constant` a
 * linalg.fill writes, which the outliner passes as an argument) its value. */
#define NPU_STRIDED_MEMREF(R)  \
  struct {                     \
    void *allocated;           \
    void *aligned;             \
    int64_t offset;            \
    int64_t sizes[R];          \
    int64_t strides[R];        \
  }
typedef NPU_STRIDED_MEMREF(1) npu_strided_memref_1d;
typedef NPU_STRIDED_MEMREF(2) npu_strided_memref_2d;
typedef NPU_STRIDED_MEMREF(3) npu_strided_memref_3d;
typedef NPU_STRIDED_MEMREF(4) npu_strided_memref_4d;

#define NPU_ARG_MEMREF 0
#define NPU_ARG_SCALAR 1
typedef struct npu_arg {
  int64_t rank;      /* UnrankedMemRefType::rank (0 for a scalar)               */
  void *descriptor;  /* UnrankedMemRefType::descriptor: a StridedMemRefType
                        layout of `rank` (NULL for a scalar)                    */
  int32_t dtype;     /* element type from the function type: NPU_F32 ...        */
  int32_t kind;      /* NPU_ARG_MEMREF or NPU_ARG_SCALAR                        */
  double scalar;     /* the value of a scalar argument                          */
} npu_arg;

/* What the outlined body computes beyond its signature: constants inside the
 * generic regions and the folding of a feeding tensor.pad. */
#define NPU_GROUP_MAX_CHAINS 16
typedef struct npu_group_attrs {
  int32_t act[NPU_GROUP_MAX_CHAINS]; /* NPU_ACT_* of each matmul/conv chain of
                                        the group, in order                    */
  int32_t pad;     /* > 0: the convolution's padded-input argument is given
                      unpadded and this zero padding is folded into the launch
                      (the host lowering removed the tensor.pad); 0: the
                      argument is the padded tensor itself                      */
  int32_t n_heads; /* attention: heads of 64                                   */
  float eps;       /* RMSNorm epsilon                                          */
  float scale;     /* attention score scale                                    */
  int32_t res_arg; /* conv groups: index in `in` of the residual operand a
                      generic adds, 0 when none is named (in[0] is always the
                      fill constant, never a residual)                        */
  int32_t stride;  /* NCHW conv groups: the conv's `strides` (0 or 1: 1)      */
} npu_group_attrs;

/* Runs one outlined group, or a chain of outlined groups that the host
 * lowering fuses across a tensor.pad, as one launch sequence on `stream`.
 *
 * outlined_name: the outliner's symbol, `fused_` + the short op names +
 *   `_<idx>` (OutlineFusedGroupsPass.cpp:69-82, 259-263); the index is
 *   ignored.  A chain of groups is their names joined by '+', in order.
 * in: the external inputs in first-use order over the group's ops (for a
 *   chain: over all its ops, values produced inside the chain left out);
 *   out: the results.  Arguments that come from tensor.empty (a fill's or a
 *   generic's destination) carry their shape; their data are never read and
 *   may be NULL, except where the group keeps an intermediate result there,
 *   as the bufferized function writes its destinations (the first matmul's
 *   ReLU destination of a two-layer chain).  The fill value must be 0.0.
 *
 * Groups (chain key = the names with `fused_` and the index removed):
 *   fill_matmul_generic                   -> fused_matmul_bias_act
 *     (cst, init[M,N], A[M,K], B[K,N], [bias[N]], dest[M,N]) -> (out[M,N])
 *   fill_matmul[_generic] repeated k <= 16 times (test/mlp.mlir: one group
 *     of two matmul -> ReLU chains; test/models/autoencoder.mlir: eight, the
 *     last without a generic)             -> k fused_matmul_bias_act calls
 *     (cst, init1, x, w1, [b1], dest1, init2, w2, [b2], dest2, ...) -> (out);
 *     a chain without a generic has no dest, its result is its init
 *   fill_linalg_conv_2d_nhwc_fhwc_generic[_generic...] (the epilogue in one
 *     or several generics: an add of the block input, then a ReLU)
 *                                         -> fused_conv2d_nhwc_bias_act, or
 *     with a residual term fused_conv2d_nhwc_bias_res_act
 *     (cst, init, x, w, then each generic's operands -- [bias f32 [F]],
 *      [res [N,Ho,Wo,F]] -- and its destination) -> (out); with several
 *     generics, attrs->res_arg names the residual's index in `in` (when it
 *     is 0, the destinations before the last must be passed without data,
 *     NULL, which tells them from the residual)
 *   fill_conv2d[_generic...] (the reference's linalg.conv_2d_nchw_fchw,
 *     test/conv2d_relu.mlir, test/resnet_block.mlir, test/resnet50_block.mlir,
 *     test/mobilenet_block.mlir, the networks of test/models/)
 *                                         -> fused_conv2d_nchw_bias_act, or
 *     with a residual term fused_conv2d_nchw_bias_res_act; the same argument
 *     order as the NHWC group, every tensor NCHW / FCHW, attrs->stride the
 *     conv's stride; without a generic (a classifier conv) the group is
 *     (cst, init, x, w) -> (out)
 *   fill_linalg_conv_2d_nhwc_fhwc_generic + the depthwise / project group(s)
 *     of an inverted residual block after its tensor.pad -> fused_irb_f32
 *     (cst, init_e, x, we[E,1,1,C], dest_e, init_d, wdw[3,3,E], dest_d,
 *      init_p, wp[C,1,1,E], dest) -> (out)
 *   the three conv -> requantizing generic groups of the int8 bottleneck,
 *     across the pad before the 3x3 conv   -> fused_qbottleneck_i8
 *     (cst, init1, x, w1[M1,1,1,C], m1, s1, dest1, init2, w2[M1,3,3,M1], m2,
 *      s2, dest2, init3, w3[C,1,1,M1], m3, s3, dest) -> (out)
 * Shapes, element types and counts are checked against the group before any
 * launch (NPU_ERR_INVALID_ARG); an unknown chain is NPU_ERR_UNSUPPORTED.
 * Launch plans of every launch of the sequence are recorded. */
npu_status npu_group_launch(const char *outlined_name, const npu_group_attrs *attrs,
                            const npu_arg *in, int32_t n_in, const npu_arg *out,
                            int32_t n_out, npu_stream stream);

/* ---- launch plans ------------------------------------------------------
 * What each kernel launch of the calling thread's most recent entry-point
 * call does per work tile: the input of the MI355X launch model in
 * npu_cost.h (npu_cm_predict_launch).  This is the GPU counterpart of the
 * per-tile DMA and compute figures the reference's cost model derives from
 * a tile configuration (evaluateConv2dTile / evaluateMatmulTile,
 * lib/Analysis/CostModel.cpp:232-324): a work tile is what one workgroup
 * computes between two loads of fresh input; a persistent workgroup walks
 * several.  Filled by every fused_* entry point; the most recent call's
 * plans replace the previous ones.  Byte and operation counts are of the
 * work as issued (padding, halo re-reads and recompute included). */
typedef struct npu_launch_plan {
  char kernel[48];          /* kernel family                                   */
  int32_t grid;             /* workgroups launched (256 lanes each)            */
  int32_t wg_per_cu;        /* resident workgroups per CU (runtime occupancy)  */
  int32_t tiles;            /* work tiles of the launch                        */
  int32_t load_phases;      /* dependent global-load round trips per tile that
                               no prefetch hides                               */
  int32_t mfma_bits;        /* MFMA operand width: 32 (f32), 16 (bf16), 8 (i8) */
  int32_t unit_waves;       /* waves of one grid unit (0: four); tile_valu and
                               wg_setup_valu are summed over a unit's waves    */
  double tile_macs;         /* MFMA multiply-adds per tile                     */
  double tile_valu;         /* vector-ALU instructions per tile besides the
                               MFMAs, summed over the workgroup's waves
                               (index arithmetic, epilogues, depthwise taps,
                               norms, softmax, requant): the kernel's loop
                               bodies, per iteration as compiled, times the
                               trip counts the launch's shape gives            */
  double tile_lds_bytes;    /* LDS bytes read and written per tile             */
  double tile_load_bytes;   /* global bytes loaded per tile                    */
  double tile_store_bytes;  /* global bytes stored per tile                    */
  double wg_setup_bytes;    /* global bytes a persistent workgroup loads once  */
  double hbm_bytes;         /* compulsory HBM bytes of the launch              */
  double wg_setup_valu;     /* vector-ALU instructions a persistent workgroup
                               runs once before its first tile (filter splits,
                               tables), summed over its waves                  */
} npu_launch_plan;

/* Copies up to max_plans plans of the calling thread's most recent fused_*
 * call and returns how many that call recorded. */
int32_t npu_last_launch_plans(npu_launch_plan *plans, int32_t max_plans);

#ifdef __cplusplus
}
#endif
#endif /* NPU_AMD_H */
