/* MI355X (gfx950) kernel library and model runtime of the ml-graph-compiler `hip` backend.
 *
 * This header is the C ABI between the code the hip emitter generates for one model and the
 * prebuilt library libmgc_hip.so. Every kernel entry point takes plain pointers and sizes; device
 * pointers point into the single HBM allocation that holds the planner's arena, the weights blob
 * and the input/output staging buffers of a model.
 *
 * Reference counterparts (paths relative to the reference repository):
 *   mgc_hip_gemm            <- mgc_gemm + mgc_gemm_args/mgc_operand/mgc_epilogue
 *                              (src/ml_graph_compiler/codegen/runtime/mgc_runtime.h:120-161,
 *                               mgc_kernels.c:328-396)
 *   mgc_hip_depthwise       <- mgc_depthwise_nhwc / mgc_depthwise_nchw (mgc_runtime.h:175-182)
 *   mgc_hip_pool            <- mgc_pool_nhwc / mgc_pool_nchw (mgc_runtime.h:185-190)
 *   mgc_hip_reduce_mid      <- mgc_reduce_mid (mgc_runtime.h:193)
 *   mgc_hip_gather_layer_norm <- op_Gather (codegen/c.py:662-688), the Add after it (c.py:360-529)
 *                              and mgc_layer_norm (mgc_runtime.h:199-200), fused
 *   mgc_hip_pool_fc         <- mgc_reduce_mid (global average pooling, codegen/c.py:1255-1270) then
 *                              mgc_gemm for the FusedGemm that reads it (c.py:974-1003), fused
 *   mgc_hip_softmax         <- mgc_softmax (mgc_runtime.h:196)
 *   mgc_hip_layer_norm      <- mgc_layer_norm (mgc_runtime.h:199-200)
 *   mgc_hip_gemm_layer_norm <- mgc_gemm then mgc_layer_norm, fused (mgc_runtime.h:120-161, 199-200)
 *   mgc_hip_elementwise     <- the loop nests CEmitter.elementwise/loops emit (codegen/c.py:360-529)
 *   mgc_hip_space_to_depth  <- no counterpart (feeds the stem convolution's stride-1 form)
 *   mgc_hip_conv_stem       <- mgc_gemm over the stem's MGC_OP_CONV_NCHW operand (codegen/c.py:1099-1226,
 *                              mgc_kernels.c:86-133, 370-396), reading the NCHW image in place
 *   mgc_hip_copy            <- the identity-body loop nests of op_Transpose/Expand/Tile/Slice/
 *                              Concat/Split/Pad (codegen/c.py:558-660) and output copies (c.py:1283)
 *   mgc_hip_fill            <- constant loops of _write_constant/op_ConstantOfShape (c.py:690-722)
 *   mgc_hip_gather          <- op_Gather (codegen/c.py:662-688), error code 1 on a bad index
 *   mgc_hip_range           <- op_Range (codegen/c.py:724-734)
 *   mgc_hip_attention       <- no single counterpart: replaces the MatMul -> Mul -> Softmax ->
 *                              MatMul chain and its head Transposes (samples.py:178-245) when
 *                              the hip emitter recognizes it
 *   mgc_hip_reduce          <- CEmitter._reduce generic loop (codegen/c.py:736-799)
 *   mgc_hip_argmax          <- op_ArgMax (codegen/c.py:801-821)
 *   mgc_hip_model_*         <- what mgc_run and CompiledModel do around the generated function
 *                              (codegen/c.py:1276-1326, codegen/runtime_lib.py:44-156)
 */
#ifndef MGC_HIP_H
#define MGC_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------------------------------- */
/* shared enums                                                                             */
/* ---------------------------------------------------------------------------------------- */

/* Activations fused into GEMM / convolution / depthwise epilogues (same set and order as the
 * reference's MGC_ACT_*, mgc_runtime.h:93-101). */
enum {
    MGC_ACT_NONE = 0,
    MGC_ACT_RELU = 1,
    MGC_ACT_CLIP = 2,
    MGC_ACT_GELU = 3,
    MGC_ACT_GELU_TANH = 4,
    MGC_ACT_TANH = 5,
    MGC_ACT_SIGMOID = 6
};

/* Element types understood by the elementwise, copy, fill, reduce and gather kernels. */
enum {
    MGC_F32 = 0,
    MGC_F64 = 1,
    MGC_I64 = 2,
    MGC_I32 = 3,
    MGC_I8 = 4,
    MGC_U8 = 5,
    MGC_BOOL = 6
};

/* Status codes returned by the model runtime and by mgc_run. */
enum {
    MGC_OK = 0,
    MGC_ERR_GATHER_INDEX = 1, /* a Gather index was out of range (reference: mgc_run returns 1) */
    MGC_ERR_HIP = 2,          /* a HIP runtime call failed; see mgc_hip_last_error() */
    MGC_ERR_ARGS = 3          /* the library was called with arguments it does not accept */
};

/* Opaque execution context: stream, error flag and profiling state of one model. */
typedef struct mgc_hip_exec mgc_hip_exec;

/* An execution context for calling the kernel entry points below directly, without a compiled
 * model (tests, custom launchers): their kernels go to `stream` (a hipStream_t; NULL = the null
 * stream). Allocates the context and its device error flag; NULL on failure (see
 * mgc_hip_last_error). No counterpart in the reference: its C kernels take no context. */
mgc_hip_exec *mgc_hip_exec_create(void *stream);
/* Status of the calls made with x since the last check, then cleared: MGC_OK, MGC_ERR_ARGS (a
 * launcher refused its operands), MGC_ERR_HIP (a launch failed) or MGC_ERR_GATHER_INDEX (after
 * synchronizing the stream: a Gather index was out of range). */
int mgc_hip_exec_status(mgc_hip_exec *x);
void mgc_hip_exec_destroy(mgc_hip_exec *x);

/* ---------------------------------------------------------------------------------------- */
/* GEMM and implicit-GEMM convolution on fp32 MFMA                                            */
/* ---------------------------------------------------------------------------------------- */

/* How an operand matrix is read.
 *   MGC_OP_STRIDED:   element (r, c) = p[r * rs + c * cs]
 *   MGC_OP_CONV_NHWC: A only. Implicit im2col of an NHWC image batch: row m is output pixel
 *                     (n, oh, ow) with m = (n * OH + oh) * OW + ow, column k is
 *                     (kh * KW + kw) * cg + c; p already includes the group channel offset.
 *   MGC_OP_CONV_NCHW: B only. Implicit im2col of one NCHW image: row k = (c * KH + kh) * KW + kw,
 *                     column = output pixel oh * OW + ow.                                      */
enum { MGC_OP_STRIDED = 0, MGC_OP_CONV_NHWC = 1, MGC_OP_CONV_NCHW = 2 };

typedef struct {
    int kind;
    const float *p;
    long rs, cs;
    int H, W, C, KH, KW, SH, SW, DH, DW, PT, PL, OH, OW, cg;
} mgc_hip_operand;

/* C[z] = act(alpha * A[z] B[z] + bias + beta * R[z]) for every batch index z.
 * bias_mode 1 adds bias[n] per column, 2 adds bias[m] per row. The batch index z runs over
 * batch_dims[0..batch_rank) (row-major) and moves each pointer by sum_d idx_d * x_bs[d]
 * elements. split_k > 1 splits K over that many partial products in `workspace`
 * (split_k * M * N floats per batch element, with batch_count <= 1); 0 lets the library choose
 * and then requires workspace_floats to say how much workspace is available. */
typedef struct {
    int M, N, K;
    mgc_hip_operand a, b;
    float *c;
    long ldc;
    float alpha, beta;
    const float *bias;
    int bias_mode;
    const float *res;
    long ldr;
    int act;
    float lo, hi;
    int batch_rank;
    int batch_dims[4];
    long a_bs[4], b_bs[4], c_bs[4], r_bs[4];
    float *workspace;
    long workspace_floats;
    int split_k;
    /* A concatenated-K GEMM when k1 > 0: columns k >= k1 of A are columns k - k1 of a2, an
     * NHWC image read as a 1 x 1 convolution (kind MGC_OP_CONV_NHWC, KH = KW = 1, no padding,
     * strides SH / SW, output OH x OW, cg = C), so one launch computes act([A | A2] B + bias)
     * with B the (K1 + K2) x N stack of both weight matrices: a residual block's last 1 x 1
     * convolution together with its projection shortcut. Needs a strided A with unit column
     * stride (row stride, a2's C and both pointers multiples of 4 floats / 16 bytes), a2's
     * C = K - k1, k1 a multiple of 32, B packed as [N][K] (rs 1, cs a multiple of 4) and
     * batch_rank 0; sets the launch error otherwise. k1 = 0 is an ordinary GEMM. */
    mgc_hip_operand a2;
    int k1;
    /* Kernel family (MGC_GEMM_*): MGC_GEMM_AUTO (0, what the emitter uses) lets the library
     * choose family and K split from the shape; any other value runs that family with split_k
     * as its K split (0 or 1: none) and sets the launch error when the operands, split or
     * workspace are outside what the family accepts. Counterpart of the reference's
     * mgc_set_blocking (src/ml_graph_compiler/codegen/runtime/mgc_kernels.c:34-70), which its
     * tests use to force the C kernels' edge paths (tests/test_codegen.py:444-455); here it
     * lets a test run every family on shapes the library would send elsewhere. */
    int kernel;
} mgc_hip_gemm_args;

/* GEMM kernel families for mgc_hip_gemm_args.kernel. */
enum {
    MGC_GEMM_AUTO = 0,     /* the library's choice */
    MGC_GEMM_TILED = 1,    /* 64 x 64 tiles through an LDS DMA ring (gemm_dma_kernel) */
    MGC_GEMM_QUARTER = 2,  /* the same, the second half of the tiles as 32 x 32 quarter tiles
                              (gemm_dma_tail_kernel); batch 1, no K split */
    MGC_GEMM_NARROW = 3,   /* 128 x 32 tiles (four waves along M) */
    MGC_GEMM_WSPLIT = 4,   /* 32 x 32 tiles, K stages dealt to four waves */
    MGC_GEMM_WSPLIT16 = 5, /* 16 x 16 tiles, K stages dealt to four or eight waves */
    MGC_GEMM_STREAM = 6,   /* short-K streaming kernel: row-major A with K <= 32, or an NHWC image
                              of one channel group with K <= 48; batch 1, no K split, a column
                              bias (or none), activation none / relu / clip */
    MGC_GEMM_REGISTER = 7  /* register-staged operands: every operand form (gemm_mfma_kernel) */
};

void mgc_hip_gemm(mgc_hip_exec *x, const mgc_hip_gemm_args *g);

/* Workspace floats mgc_hip_gemm wants for a GEMM of this shape (0 = none). The emitter asks
 * at compile time and reserves it through the memory planner's workspace hook. */
long mgc_hip_gemm_workspace(int M, int N, int K, int batch);

/* Floats of device scratch the library holds per GPU for mgc_hip_gemm_noalloc (32 MiB). */
#define MGC_HIP_NOALLOC_SCRATCH_FLOATS (1L << 23)

/* mgc_hip_gemm for callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc). No counterpart in the reference: its C
 * backend allocates nothing to begin with. Computes exactly what mgc_hip_gemm computes with a
 * workspace of MGC_HIP_NOALLOC_SCRATCH_FLOATS floats, which it keeps in the library's own
 * per-GPU device array: g->workspace and g->workspace_floats are ignored, and the call
 * allocates nothing. A K split the library chooses (split_k 0) whose partials would not fit
 * is dropped, as mgc_hip_gemm drops it for a small workspace; an explicit split_k that does
 * not fit is refused. `stream` is a hipStream_t (NULL = the null stream); the call only
 * enqueues work. Returns MGC_OK, MGC_ERR_ARGS (no arguments, an explicit split_k whose
 * partials need more than MGC_HIP_NOALLOC_SCRATCH_FLOATS floats, or operands outside a
 * kernel's limits; see mgc_hip_last_error) or MGC_ERR_HIP (launch or runtime failure). An
 * error left pending on the calling thread before the call is cleared, not reported. Every
 * call on one GPU shares that GPU's array: calls that overlap on one GPU (different streams
 * without ordering) race on it. */
int mgc_hip_gemm_noalloc(void *stream, const mgc_hip_gemm_args *g);

/* A GEMM (batch_rank 0) whose output rows then go through a LayerNorm: out = LayerNorm(C) with
 * C = act(alpha A B + bias + beta R) as mgc_hip_gemm computes it. K is always split (at least
 * in two) and the split-K reduction applies the epilogue, stores C when g->c is not NULL and
 * normalizes each row from registers (two-pass float mean and variance, then * ln_scale +
 * ln_bias; either may be NULL), so C is not read back and the LayerNorm has no launch of its
 * own. Needs N % 4 == 0, N <= 1024, M < 2^25, 16-byte aligned pointers and row strides, and
 * g->workspace of mgc_hip_gemm_layer_norm_workspace(M, N, K) floats; sets the launch error
 * otherwise. Replaces mgc_gemm followed by mgc_layer_norm
 * (src/ml_graph_compiler/codegen/runtime/mgc_kernels.c:328-396, 657-679) for a FusedGemm the
 * schedule puts right before the LayerNormalization of its output. */
void mgc_hip_gemm_layer_norm(mgc_hip_exec *x, const mgc_hip_gemm_args *g, const float *ln_scale,
                             const float *ln_bias, float eps, float *ln_out);

/* Workspace floats mgc_hip_gemm_layer_norm needs (0 when the shape is outside its limits). */
long mgc_hip_gemm_layer_norm_workspace(int M, int N, int K);

/* 1 when mgc_hip_gemm_layer_norm takes an M x N output. */
int mgc_hip_gemm_layer_norm_supported(int M, int N);

/* A depthwise 3 x 3 convolution and the 1 x 1 convolution that reads its output, as one
 * launch: the GEMM of g (C = act(alpha A B + bias + beta R), batch_rank 0, B packed [N][K])
 * whose A operand is computed on the fly as the depthwise output
 *   A[m][k] = act_d(bias_d[k] + sum_{i,j < 3} x[n][oh SH - PT + i][ow SW - PL + j][k] w[(3 i + j) C + k])
 * for output pixel m = (n OH + oh) OW + ow of the NHWC batch x [n][H][W][C] (taps outside the
 * image are zero), so the depthwise output is never stored; g->a is not read and g->K = C.
 * Replaces mgc_depthwise_nhwc followed by mgc_gemm of the pointwise convolution
 * (src/ml_graph_compiler/codegen/runtime/mgc_kernels.c:455-473 and :370-396, which the
 * reference's C backend emits as two calls, codegen/c.py:1126-1135 and :1140-1167). Needs
 * SH = SW in {1, 2}, C % 4 == 0, 16-byte aligned x, w, bias and B, B's column stride a multiple
 * of 4, bias_mode 1 (or no bias), M a whole number of OH x OW images and x below 2 GiB; sets the
 * launch error otherwise. */
typedef struct {
    const float *x;     /* NHWC input [N][H][W][C] */
    const float *w;     /* [3][3][C], channel fastest */
    const float *bias;  /* [C] or NULL */
    int H, W, C, SH, SW, PT, PL, OH, OW;
    int act;            /* MGC_ACT_* applied to the depthwise output */
    float lo, hi;
} mgc_hip_dw_args;

void mgc_hip_gemm_dw(mgc_hip_exec *x, const mgc_hip_gemm_args *g, const mgc_hip_dw_args *dw);

/* A whole inverted-residual block (the MobileNetV2 pattern with expansion > 1) as one launch:
 * the projection GEMM of g (C = act(alpha A B + bias + beta R), batch_rank 0, B packed [N][K],
 * K = Cexp) whose A operand is computed on the fly as
 *   A[m][k] = act_d(bd[k] + sum_{i,j < 3} E[n][oh SH - PT + i][ow SW - PL + j][k] wd[(3 i + j) Cexp + k])
 *   E[n][y][z][k] = act_e(be[k] + sum_c x[n][y][z][c] we[k Cin + c])  (zero outside the image)
 * for output pixel m = (n OH + oh) OW + ow of the NHWC batch x [n][H][W][Cin]: the expanded
 * tensor and the depthwise output never go to memory; g->a is not read. Replaces mgc_gemm,
 * mgc_depthwise_nhwc and mgc_gemm of the block's three convolutions
 * (src/ml_graph_compiler/codegen/runtime/mgc_kernels.c:370-396, 455-473, which the reference's
 * C backend emits as three calls, codegen/c.py:1102-1226). Needs the shapes
 * mgc_hip_mbconv_supported accepts (Cin 16, 24 or 32; Cexp % 4 == 0 and Cexp <= 256; N <= 32;
 * SH = SW in {1, 2}), act_e and act_d relu or clip, 16-byte aligned x, we, be, wd, bd and B, B's
 * column stride a multiple of 4,
 * bias_mode 1 (or no bias), M a whole number of OH x OW images and x below 2 GiB; sets the
 * launch error otherwise. */
typedef struct {
    const float *x;     /* block input NHWC [N][H][W][Cin] */
    const float *we;    /* expansion weights packed [Cexp][Cin] */
    const float *be;    /* expansion bias [Cexp] or NULL */
    const float *wd;    /* depthwise weights [3][3][Cexp], channel fastest */
    const float *bd;    /* depthwise bias [Cexp] or NULL */
    int H, W, Cin, Cexp, SH, SW, PT, PL, OH, OW;
    int act_e, act_d;   /* MGC_ACT_* after the expansion and after the depthwise convolution */
    float lo_e, hi_e, lo_d, hi_d;
} mgc_hip_mbconv_args;

int mgc_hip_mbconv_supported(int Cin, int Cexp, int Cout, int stride);
void mgc_hip_mbconv(mgc_hip_exec *x, const mgc_hip_gemm_args *g, const mgc_hip_mbconv_args *mb);

/* The same launch when the block input is itself a convolution's output that never goes to
 * memory: MobileNetV2's stem (a 3 x 3 convolution of the 3-channel image with its activation)
 * ahead of the first block (3 x 3 depthwise with its activation, 1 x 1 projection). E above is
 * then the stem's output,
 *   E[n][y][z][k] = act_e(be[k] + sum_{i,j < 3, c < 3} img(n, c, y SH - PT + i, z SW - PL + j) we[k 32 + (3 i + j) 3 + c])
 * with img(n, c, r, s) = st->img[n sn + c sc + r sh + s sw] (zero outside the H x W image), and
 * zero for (y, z) outside the mb->H x mb->W stem output: an NCHW graph input is read in place,
 * with no NHWC copy. mb->x is not read; mb->Cin is 32 (the 27 window values, padded), mb->we
 * [Cexp][32] with columns 27..31 zero, mb->H x mb->W the stem's output size. Replaces the
 * stem's mgc_gemm over its im2col operand and the block's mgc_depthwise_nhwc and mgc_gemm
 * (src/ml_graph_compiler/codegen/runtime/mgc_kernels.c:86-133, 370-396, 455-473; three calls
 * in the reference's C backend, codegen/c.py:1102-1226). Needs the shapes
 * mgc_hip_mbconv_stem_supported accepts (C = 3, KH = KW = 3; the mbconv limits for Cexp, N and
 * the depthwise stride), stem strides SH, SW of 1 or 2, non-negative padding and image strides, img 4-byte aligned and the image
 * below 2 GiB, and otherwise what mgc_hip_mbconv needs; sets the launch error otherwise. */
typedef struct {
    const float *img;       /* the stem convolution's input image */
    int C, H, W;            /* its channels and size */
    long sn, sc, sh, sw;    /* element strides of image, channel, row and column (NCHW: C H W, H W, W, 1) */
    int KH, KW, SH, SW, PT, PL; /* the stem's window (3 x 3), strides (1 or 2) and top / left padding */
} mgc_hip_stem_args;

int mgc_hip_mbconv_stem_supported(int C, int KH, int KW, int Cexp, int Cout, int stride);
void mgc_hip_mbconv_stem(mgc_hip_exec *x, const mgc_hip_gemm_args *g, const mgc_hip_mbconv_args *mb,
                         const mgc_hip_stem_args *st);

/* The ResNet stem convolution as one launch that reads the image in place (an NCHW graph input
 * needs no NHWC or space-to-depth copy):
 *   out[n][oh][ow][k] = act(bias[k] + sum_{c < 3, i, j < 7} img(n, c, oh SH - PT + i, ow SW - PL + j) W[k][c][i][j])
 * with img(n, c, r, s) = st->img[n sn + c sc + r sh + s sw] (zero outside the st->H x st->W
 * image) and out NHWC with a->ldc floats per pixel. st->C = 3, KH = KW = 7, SH = SW = 2 and 64
 * output channels (mgc_hip_conv_stem_supported); st->img and a->out 4-byte aligned, the image
 * below 2 GiB, a->w 16-byte aligned, a->ldc >= 64. a->w holds
 * mgc_hip_conv_stem_weight_floats() floats packed as
 *   a->w[((e 32 + l) 2 + h) 2 + b] = W[32 b + l][c][i][2 q + h]  (zero for 2 q + h >= 7)
 * for step e = (c 7 + i) 4 + q. The output is cut into tiles of 8 x 16 pixels that persistent
 * workgroups take in turn; a->workgroups caps their number (0: the library's choice, one round
 * over the CUs). Sets the launch error outside these limits. Replaces the stem's mgc_gemm over
 * its MGC_OP_CONV_NCHW operand in the reference's C backend
 * (src/ml_graph_compiler/codegen/c.py:1099-1226; runtime/mgc_kernels.c:86-133 packs the im2col
 * panels, :370-396 multiplies). */
typedef struct {
    const float *w;     /* packed weights, mgc_hip_conv_stem_weight_floats() floats */
    const float *bias;  /* [64] or NULL */
    float *out;         /* NHWC [N][OH][OW] pixels of ldc floats (channels 0..63 written) */
    long ldc;
    int N, OH, OW;
    int act;            /* MGC_ACT_* */
    float lo, hi;
    int workgroups;     /* 0 (library's choice) or at most this many persistent workgroups */
} mgc_hip_conv_stem_args;

int mgc_hip_conv_stem_supported(int C, int KH, int KW, int SH, int SW, int Cout);
long mgc_hip_conv_stem_weight_floats(void);
void mgc_hip_conv_stem(mgc_hip_exec *x, const mgc_hip_stem_args *st, const mgc_hip_conv_stem_args *a);

/* The expansion and depthwise convolutions of an inverted-residual block as one launch, with
 * the expanded tensor never in memory:
 *   out[n][oh][ow][k] = act_d(bd[k] + sum_{i,j < 3} E[n][oh SH - PT + i][ow SW - PL + j][k] wd[(3 i + j) Cexp + k])
 *   E[n][y][z][k] = act_e(be[k] + sum_c x[n][y][z][c] we[k Cin + c])  (zero outside the image)
 * for the NHWC batch x [N][H][W][Cin] and out [N][OH][OW][Cexp]. Replaces mgc_gemm and
 * mgc_depthwise_nhwc of the block's first two convolutions
 * (src/ml_graph_compiler/codegen/runtime/mgc_kernels.c:370-396, 455-473, which the reference's
 * C backend emits as two calls, codegen/c.py:1102-1226). One workgroup per image and 32
 * expanded channels, so it suits small images at large batch (MobileNetV2's 14 x 14 and 7 x 7
 * blocks at batch 32). Needs the shapes mgc_hip_expand_dw_supported accepts (Cin 64 or 96 with
 * H W <= 256, or 160 with H W <= 64; Cexp % 32 == 0; SH = SW in {1, 2}; the depthwise window
 * ((OH - 1) SH + 3) x ((OW - 1) SW + 3) at most 256 pixels, 128 for Cin 160), PT and PL in
 * 0..2, act_e and act_d relu or clip, 16-byte aligned x, we, be, wd, bd and out, and x below
 * 2 GiB; sets the launch error otherwise. */
typedef struct {
    const float *x;     /* block input NHWC [N][H][W][Cin] */
    const float *we;    /* expansion weights packed [Cexp][Cin] */
    const float *be;    /* expansion bias [Cexp] or NULL */
    const float *wd;    /* depthwise weights [3][3][Cexp], channel fastest */
    const float *bd;    /* depthwise bias [Cexp] or NULL */
    float *out;         /* depthwise output NHWC [N][OH][OW][Cexp] */
    int N, H, W, Cin, Cexp, SH, SW, PT, PL, OH, OW;
    int act_e, act_d;   /* MGC_ACT_* after the expansion and after the depthwise convolution */
    float lo_e, hi_e, lo_d, hi_d;
} mgc_hip_expand_dw_args;

int mgc_hip_expand_dw_supported(int H, int W, int Cin, int Cexp, int stride, int OH, int OW);
void mgc_hip_expand_dw(mgc_hip_exec *x, const mgc_hip_expand_dw_args *a);

/* ---------------------------------------------------------------------------------------- */
/* memory-bound kernels                                                                      */
/* ---------------------------------------------------------------------------------------- */

/* Depthwise convolution (one input channel per group) with bias, residual and activation.
 * NHWC with HWC-ordered weights (w[(kh * KW + kw) * C + c]) or NCHW with CHW weights. */
void mgc_hip_depthwise(mgc_hip_exec *x, int nhwc, int N, int H, int W, int C, int KH, int KW,
                       int SH, int SW, int DH, int DW, int PT, int PL, int OH, int OW,
                       const float *in, const float *w, const float *bias, const float *res,
                       int act, float lo, float hi, float *out);

/* Max or average pooling; pads are (top, left, bottom, right). */
void mgc_hip_pool(mgc_hip_exec *x, int nhwc, int is_max, int N, int H, int W, int C, int KH,
                  int KW, int SH, int SW, int DH, int DW, int PT, int PL, int PB, int PR, int OH,
                  int OW, int count_include_pad, const float *in, float *out);

/* Mean or max over the middle axis of an [outer, n, inner] float tensor. */
void mgc_hip_reduce_mid(mgc_hip_exec *x, int is_max, long outer, long n, long inner,
                        const float *in, float *out);

/* Global average pooling of an NHWC activation followed by a fully connected layer, as one
 * launch (for a few images: every workgroup pools its whole image):
 *   out[i * ldo + f] = act(bias[f] + sum_c w[f * C + c] * (1 / P) sum_p x[(i * P + p) * C + c])
 * for i < N, f < F. Replaces mgc_reduce_mid's mean (mgc_kernels.c:593-612) feeding mgc_gemm
 * (mgc_kernels.c:370). x and w 16-byte aligned, C % 4 == 0 and C <= 4096
 * (mgc_hip_pool_fc_supported), ldo >= F; anything else sets MGC_ERR_ARGS. N <= 0 or F <= 0:
 * nothing to do. */
typedef struct mgc_hip_pool_fc_args {
    const float *x;     /* N images of P pixels x C channels (NHWC) */
    const float *w;     /* F x C: row f holds output f's weights (a Gemm's B with transB = 1) */
    const float *bias;  /* F floats, or NULL */
    float *out;         /* row i at out + i * ldo */
    long ldo;
    int N, P, C, F;
    int act;            /* MGC_ACT_* */
    float lo, hi;       /* clip bounds for MGC_ACT_CLIP */
} mgc_hip_pool_fc_args;

int mgc_hip_pool_fc_supported(int N, int P, int C, int F);
void mgc_hip_pool_fc(mgc_hip_exec *x, const mgc_hip_pool_fc_args *a);

/* Embedding lookup, addend and LayerNorm as one launch (a transformer encoder's input):
 *   y = table[idx[r]] + addend[r % add_rows];  out[r] = (y - mean(y)) / sqrt(var(y) + eps) * scale + bias
 * for each of the rows rows of cols floats, y itself also stored to sum when that is not NULL.
 * Replaces op_Gather (codegen/c.py:662-688), the Add that reads it (c.py:360-529) and
 * mgc_layer_norm (mgc_runtime.h:199-200); rounds as the Add and mgc_hip_layer_norm do apart.
 * cols % 4 == 0 and cols <= 1024; table, addend, scale, bias, out and sum 16-byte aligned
 * (anything else sets MGC_ERR_ARGS); an index outside [-dim, dim) sets MGC_ERR_GATHER_INDEX and
 * leaves its row unwritten, as mgc_hip_gather does. */
typedef struct mgc_hip_gather_ln_args {
    const float *table;  /* dim rows of cols floats */
    long dim;
    const void *idx;     /* rows indices */
    int idx_dtype;       /* MGC_I64 or MGC_I32 */
    const float *addend; /* add_rows rows of cols floats, row r % add_rows added to row r; or NULL */
    long add_rows;
    const float *scale;  /* cols floats, or NULL */
    const float *bias;   /* cols floats, or NULL */
    float eps;
    float *out;          /* rows rows of cols floats */
    long rows;
    int cols;
    float *sum;          /* rows rows of cols floats: the sum before the LayerNorm, or NULL */
} mgc_hip_gather_ln_args;

void mgc_hip_gather_layer_norm(mgc_hip_exec *x, const mgc_hip_gather_ln_args *a);

/* Generic reduction over the middle axis of [outer, n, inner]: kind 0 sum, 1 mean, 2 max,
 * 3 min, 4 prod; float sums/means/products accumulate in double like the reference. */
void mgc_hip_reduce(mgc_hip_exec *x, int kind, int dtype, long outer, long n, long inner,
                    const void *in, void *out);

/* Index of the first maximum along the middle axis of [outer, n, inner]; int64 output. */
void mgc_hip_argmax(mgc_hip_exec *x, int dtype, long outer, long n, long inner, const void *in,
                    int64_t *out);

/* Softmax or log-softmax along the middle axis of an [outer, n, inner] float tensor. */
void mgc_hip_softmax(mgc_hip_exec *x, long outer, long n, long inner, const float *in,
                     float *out, int log_softmax);

/* Layer normalization of each row of [rows, cols]; scale and bias may be NULL. */
void mgc_hip_layer_norm(mgc_hip_exec *x, long rows, long cols, const float *in,
                        const float *scale, const float *bias, float eps, float *out);

/* Scaled dot-product attention for every (batch b, head h), query s and key j:
 *   t = Q[b, s, h, :] . K[b, j, h, :]
 *   t = scale_div ? t / scale : t * scale;  if (bias) t += bias[b, h, s, j];
 *   if (causal || mask) t = keep(s, j) ? t : fill;
 *   O[b, s, h, :] = sum_j softmax_j(t) V[b, j, h, :]
 * with keep(s, j) = (j <= s) when causal, else ((mask[b, h, s, j] != 0) == mask_keep).
 * Element (b, s, h, d) of X in {Q, K, V, O} is at x + b * x_b + s * x_s + h * x_h + d (d is
 * contiguous); bias and mask elements are at p + b * p_b + h * p_h + s * p_s + j * p_j (strides
 * in elements, 0 for a broadcast dimension; bias float, mask one byte per element).
 * Limits: D <= 64 with D % 4 == 0 (mgc_hip_attention_supported); Q, K and V pointers and row
 * strides must keep 16-byte alignment. S and Skv are unbounded (keys are streamed in blocks
 * with a running softmax). */
typedef struct {
    int B, H, S, Skv, D;
    const float *q, *k, *v;
    long q_b, q_s, q_h, k_b, k_s, k_h, v_b, v_s, v_h;
    float *o;
    long o_b, o_s, o_h;
    float scale;
    int scale_div;
    const float *bias;
    long bias_b, bias_h, bias_s, bias_j;
    const unsigned char *mask;
    long mask_b, mask_h, mask_s, mask_j;
    int mask_keep;
    int causal;
    float fill;
} mgc_hip_attention_args;

int mgc_hip_attention_supported(int S, int Skv, int D);
void mgc_hip_attention(mgc_hip_exec *x, const mgc_hip_attention_args *a);

/* ---------------------------------------------------------------------------------------- */
/* elementwise programs, copies, fills, gathers                                              */
/* ---------------------------------------------------------------------------------------- */

#define MGC_EW_MAX_RANK 6
#define MGC_EW_MAX_LEAVES 16
#define MGC_EW_MAX_INSTR 32

/* Elementwise opcodes (one per reference elementwise operator, ops.py:122-375). */
enum {
    MGC_EW_ADD = 0, MGC_EW_SUB, MGC_EW_MUL, MGC_EW_DIV, MGC_EW_POW, MGC_EW_MAX, MGC_EW_MIN,
    MGC_EW_EQUAL, MGC_EW_LESS, MGC_EW_GREATER, MGC_EW_LESS_EQUAL, MGC_EW_GREATER_EQUAL,
    MGC_EW_AND, MGC_EW_OR, MGC_EW_XOR, MGC_EW_WHERE, MGC_EW_RELU, MGC_EW_SIGMOID, MGC_EW_TANH,
    MGC_EW_ERF, MGC_EW_SQRT, MGC_EW_EXP, MGC_EW_LOG, MGC_EW_NEG, MGC_EW_ABS, MGC_EW_RECIPROCAL,
    MGC_EW_FLOOR, MGC_EW_CEIL, MGC_EW_SIN, MGC_EW_COS, MGC_EW_SOFTPLUS, MGC_EW_IDENTITY,
    MGC_EW_NOT, MGC_EW_GELU, MGC_EW_GELU_TANH, MGC_EW_LEAKY_RELU, MGC_EW_HARD_SIGMOID,
    MGC_EW_CLIP, MGC_EW_CAST, MGC_EW_COUNT
};

typedef struct {
    const void *p;
    int dtype;
    long strides[MGC_EW_MAX_RANK]; /* element strides over the output dims (0 = broadcast) */
} mgc_hip_ew_leaf;

/* One instruction: out_dtype = op(args) where args index the register file (leaves first,
 * then instruction results; -1 = absent). in_dtype is the dtype of the first argument; fa/fb
 * are float attributes (LeakyRelu alpha, HardSigmoid alpha/beta, Clip bounds when args are
 * absent). */
typedef struct {
    int op, in_dtype, out_dtype;
    int args[3];
    float fa, fb;
} mgc_hip_ew_instr;

typedef struct {
    int rank;
    long dims[MGC_EW_MAX_RANK];
    long out_strides[MGC_EW_MAX_RANK];
    long out_base;
    int n_leaves, n_instr;
    mgc_hip_ew_leaf leaf[MGC_EW_MAX_LEAVES];
    mgc_hip_ew_instr instr[MGC_EW_MAX_INSTR];
    void *out;
    int out_dtype;
} mgc_hip_ew_args;

void mgc_hip_elementwise(mgc_hip_exec *x, const mgc_hip_ew_args *e);

/* N-d strided copy: out[o_base + sum i_d * o_st_d] = in[i_base + sum (i_d % mod_d) * i_st_d]
 * over dims (mod_d = 0 means no modulus). Element size in bytes: 1, 2, 4 or 8. */
typedef struct {
    int rank;
    long dims[MGC_EW_MAX_RANK];
    long in_strides[MGC_EW_MAX_RANK];
    long out_strides[MGC_EW_MAX_RANK];
    long in_mod[MGC_EW_MAX_RANK];
    long in_base, out_base;
    const void *in;
    void *out;
    int elem_bytes;
} mgc_hip_copy_args;

void mgc_hip_copy(mgc_hip_exec *x, const mgc_hip_copy_args *c);

/* Space-to-depth of an NCHW float image for a stride-2 convolution over few channels:
 * out[b][i][j][(dy * 2 + dx) * C + c] = in[b][c][2 i + dy][2 j + dx], out contiguous
 * [N][H/2][W/2][4 C]. Requires even H and W and 1 <= C <= 8 (returns without launching and
 * sets the launch error otherwise). No counterpart in the reference: the hip emitter uses it to
 * run the network's stem convolution as a stride-1 convolution with 16-byte operand loads. */
void mgc_hip_space_to_depth(mgc_hip_exec *x, int N, int C, int H, int W, const float *in, float *out);

/* Fill n elements of elem_bytes each with the bit pattern `bits`. */
void mgc_hip_fill(mgc_hip_exec *x, void *out, long n, int elem_bytes, uint64_t bits);

/* out[o, t, :] = src[o, idx[t], :] with negative indices wrapped; an index out of [0, dim)
 * sets the model's error flag (mgc_run then returns MGC_ERR_GATHER_INDEX). */
void mgc_hip_gather(mgc_hip_exec *x, const void *src, const void *idx, int idx_dtype,
                    long outer, long dim, long n, long inner_bytes, void *out);

/* out[o] = start + o * delta for o < n (dtype MGC_F32/F64/I64/I32). */
void mgc_hip_range(mgc_hip_exec *x, int dtype, const void *start, const void *delta, long n,
                   void *out);

/* ---------------------------------------------------------------------------------------- */
/* model runtime                                                                             */
/* ---------------------------------------------------------------------------------------- */

/* The forward function the emitter generates: one launcher call per scheduled node. A, W, in
 * and out are device pointers. */
typedef void (*mgc_hip_forward_fn)(mgc_hip_exec *x, const void *const *in, void *const *out,
                                   unsigned char *A, const unsigned char *W);

typedef struct {
    size_t arena_bytes;
    size_t weights_bytes;
    int n_inputs, n_outputs;
    const size_t *input_bytes;
    const size_t *output_bytes;
    int n_nodes;       /* nodes with profiling markers (0 when compiled without profile) */
    mgc_hip_forward_fn forward;
    void *state;       /* owned by the runtime */
} mgc_hip_model;

/* Allocate one HBM block (arena | weights | input staging | output staging | flags), upload
 * the weights once and return the device arena and weights pointers. Idempotent. */
int mgc_hip_model_init(mgc_hip_model *m, const unsigned char *weights_host, unsigned char **A,
                       unsigned char **W);
/* Host inputs/outputs: H2D copy, replay of the captured hipGraph, D2H copy, synchronize. */
int mgc_hip_model_run(mgc_hip_model *m, const void *const *inputs, void *const *outputs,
                      unsigned char *A, const unsigned char *W);
/* Device inputs/outputs (for example torch tensors); the graph is re-captured when the pointer
 * set changes. Synchronizes and returns the status. */
int mgc_hip_model_run_device(mgc_hip_model *m, const void *const *inputs, void *const *outputs,
                             unsigned char *A, const unsigned char *W);
/* Resident-input execution for benchmarks: upload once, then enqueue replays without copies. */
int mgc_hip_model_upload(mgc_hip_model *m, const void *const *inputs);
int mgc_hip_model_launch(mgc_hip_model *m, int replays);
int mgc_hip_model_sync(mgc_hip_model *m);
int mgc_hip_model_download(mgc_hip_model *m, void *const *outputs);
/* Eager (non-graph) execution on the staged inputs with a hipEvent pair around every profiled
 * node; seconds accumulate into the per-node profile. */
int mgc_hip_model_profile_run(mgc_hip_model *m, int replays);
const double *mgc_hip_model_profile_data(mgc_hip_model *m);
void mgc_hip_model_profile_reset(mgc_hip_model *m);
/* Time `replays` graph replays between two hipEvents on the model stream; milliseconds. */
double mgc_hip_model_time_graph(mgc_hip_model *m, int replays);
void mgc_hip_model_release(mgc_hip_model *m);

/* Profiling markers emitted around each node when the model is compiled with profile=True. */
void mgc_hip_node_begin(mgc_hip_exec *x, int node);
void mgc_hip_node_end(mgc_hip_exec *x, int node);

/* Text of the last HIP error seen by the library (empty when none). */
const char *mgc_hip_last_error(void);
/* Version string of the kernel library. */
const char *mgc_hip_version(void);
/* Number of visible HIP devices (0 without a GPU; never fails). */
int mgc_hip_device_count(void);

#ifdef __cplusplus
}
#endif

#endif /* MGC_HIP_H */
