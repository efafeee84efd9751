/*
 * mira_rocm.h -- C ABI of libmira_rocm.so, the gfx950 (MI355X) kernels behind
 * MIRA's `rocm` target for W8A8 quantized inference.
 *
 * The reference (myramay/MIRA) has no native boundary: every op is a NumPy
 * function in mira/ops.py, called through the Target/Executable protocol
 * (mira/backends/base.py:13-26).  Each entry point below replaces one of those
 * NumPy functions; the comment on each names it (file:line).
 *
 * Conventions
 *  - Every pointer is a device pointer (hipMalloc'd or a torch-ROCm tensor's
 *    data_ptr()).  No entry point allocates, frees or takes ownership.
 *  - `stream` is a hipStream_t passed as void*; NULL means the null stream.
 *    Work is enqueued asynchronously; nothing synchronises.
 *  - Every entry point returns MR_OK (0) or an error code; mr_last_error()
 *    then returns a message (thread-local, valid until the next call).
 *    Arguments are validated on the host before any launch.
 *  - Activations inside a rocm segment live in NHWC order.  int8 NHWC
 *    tensors carry `c_pad` channels per pixel (a multiple of 16, or 4 for
 *    the small-channel stem layout); channels >= c are never read as data
 *    because the packed weights hold zeros there.
 *  - Matmul-shaped tensors are row-major [M, K] with a row stride.
 */
#ifndef MIRA_ROCM_H
#define MIRA_ROCM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MR_ABI_VERSION 12

enum mr_status {
  MR_OK = 0,
  MR_EINVAL = 1,      /* bad argument (shape, pointer, alignment) */
  MR_EHIP = 2,        /* a HIP runtime call failed */
  MR_EUNSUPPORTED = 3 /* valid request the library has no kernel for */
};

/* Epilogue step functions: the fusable ops of mira/passes.py:151-152
 * (UNARY/BINARY tables, mira/ops.py:99-139).  ADD..RELU have exact IEEE-754
 * single-precision semantics (relu == np.maximum(x, 0)).  GELU (the tanh form
 * of mira/ops.py:94-96), SIGMOID (1 / (1 + exp(-x)), :102) and TANH (:103)
 * call the device's expf/tanhf, whose results differ from NumPy's in the last
 * bits: a caller that needs bit-exact results does not use them. */
enum mr_epi_fn {
  MR_EPI_ADD = 1,
  MR_EPI_SUB = 2,
  MR_EPI_MUL = 3,
  MR_EPI_DIV = 4,
  MR_EPI_MAX = 5,
  MR_EPI_MIN = 6,
  MR_EPI_RELU = 7,
  MR_EPI_GELU = 8,
  MR_EPI_SIGMOID = 9,
  MR_EPI_TANH = 10
};

/* How an epilogue operand broadcasts onto the [rows, cols] result
 * (rows = N*OH*OW pixels or matmul rows, cols = output channels). */
enum mr_bcast {
  MR_BC_SCALAR = 0, /* ptr[0]                       (0-d constants, e.g. ReLU6's 6) */
  MR_BC_COL = 1,    /* ptr[col]                     (bias [N], [O,1,1], [1,O,1,1]) */
  MR_BC_ROW = 2,    /* ptr[row * ld]                ([M,1] operands) */
  MR_BC_FULL = 3    /* ptr[row * ld + col]          (residuals, same shape as result) */
};

#define MR_MAX_EPI 8

/* One step of mira/ops.py:192-199 epilogue_ref: acc = fn(acc, other), or
 * fn(other, acc) when swapped; `ptr` is unused for the unary steps
 * (MR_EPI_RELU, MR_EPI_GELU, MR_EPI_SIGMOID, MR_EPI_TANH). */
typedef struct mr_epi_step {
  int32_t fn;
  int32_t swapped;
  int32_t mode;
  int32_t reserved;
  const float* ptr;
  int64_t ld;
} mr_epi_step;

/* What happens to each result element after the contraction:
 *   y = f32(f64(acc) * scale[col])          (mira/ops.py:618,633; skipped when scale == NULL)
 *   y = steps[0..n_steps)(y)                (mira/ops.py:192-199)
 *   y = f32(f16(y))                         (flags & MR_EPI_OUT_F16: the op's result is
 *                                            f16, mira/ops.py:620,634 .astype(float16);
 *                                            round to nearest even, overflow to inf; the
 *                                            value is still stored as f32)
 *   out_f32[row*ldo+col] = y                (if out_f32)
 *   out_i8[row*ldq+col]  = clip(rint(y / out_xs), +-127)
 *                                           (mira/ops.py:602-603, the next q-op's input)
 *   out_acc[row*ldacc+col] = acc            (int32 accumulator, if out_acc)
 * f16 values may also be stored as IEEE halves, which holds them exactly and moves
 * half the bytes (entry points that take these flags say so; others return
 * MR_EUNSUPPORTED):
 *   MR_EPI_OUT_H16   out_f32 points to halves: y is rounded to f16 (as MR_EPI_OUT_F16)
 *                    and stored as a half; ldo counts halves
 *   MR_EPI_FULL_H16  every MR_BC_FULL operand holds halves (ld counts halves) */
#define MR_EPI_OUT_F16 1
#define MR_EPI_OUT_H16 2
#define MR_EPI_FULL_H16 4

typedef struct mr_epilogue {
  int32_t n_steps;
  int32_t flags;      /* MR_EPI_OUT_F16 | MR_EPI_OUT_H16 | MR_EPI_FULL_H16, or 0 */
  mr_epi_step steps[MR_MAX_EPI];
  const double* scale;
  float* out_f32;
  int64_t ldo;
  int8_t* out_i8;
  int64_t ldq;
  float out_xs;
  int32_t reserved1;
  int32_t* out_acc;
  int64_t ldacc;
} mr_epilogue;

/* Geometry of an NHWC convolution (mira/ops.py:225-276 conv_params/_conv2d_infer).
 * `c` real input channels, `c_pad` stored per pixel.  For groups == 1 convs
 * c_pad % 16 == 0, or c_pad == 4 (stem layout: taps of one kernel row are
 * packed 4 channels per tap, row_bytes = 16*ceil(kw/4) bytes per row). */
typedef struct mr_conv_geom {
  int32_t n, h, w, c, c_pad;
  int32_t o, oh, ow;
  int32_t kh, kw;
  int32_t sh, sw;
  int32_t ph, pw;
  int32_t dh, dw;
} mr_conv_geom;

/* ---- library ----------------------------------------------------------- */
int mr_abi_version(void);
const char* mr_last_error(void);
/* sizeof of the ABI structs, so bindings can check their mirrors. */
int64_t mr_sizeof(const char* struct_name);
/* Select the device and read its properties (CU count). */
int mr_init(int device);

/* ---- K1: activation quantize ------------------------------------------ */

/* Replaces mira/ops.py:602-603 quantize_activation on a row-major matrix:
 *   q[r*ldq + c] = clip(rint(x[r*ldx + c] / xs), -127, 127) for c < cols,
 *   q[r*ldq + c] = 0 for cols <= c < ldq.
 * Division is IEEE single precision, rint rounds half to even. */
int mr_quantize_rows(const float* x, int64_t rows, int64_t cols, int64_t ldx,
                     int8_t* q, int64_t ldq, float xs, void* stream);

/* Same arithmetic, NCHW f32 in, NHWC int8 out with c_pad channels per pixel
 * (channels c..c_pad-1 are zero).  Graph inputs of qconv2d
 * (mira/ops.py:630-634) enter the device this way. */
int mr_quantize_nchw_nhwc(const float* x, int32_t n, int32_t c, int32_t h, int32_t w,
                          int8_t* q, int32_t c_pad, float xs, void* stream);

/* The same after the f32 -> f16 cast that MIRA's f16 lowering puts on each
 * graph input (mira/passes.py:220-223, mira/ops.py:405-406): quantizes
 * f32(f16(x)), for an input whose only use is that cast. */
int mr_quantize_f16_nchw_nhwc(const float* x, int32_t n, int32_t c, int32_t h, int32_t w,
                              int8_t* q, int32_t c_pad, float xs, void* stream);

/* ---- K2/K3: int8 GEMM with fused dequant/epilogue/requant -------------- */

/* Replaces mira/ops.py:616-620 _qmatmul_ref (after quantize_activation):
 * acc[M,N] = a[M,K] (int8, row stride lda) x B[N,k_pad]^T (packed int8
 * weights, zero for k >= K and n >= N, N rounded up to n_pad rows),
 * exact int32, then the epilogue.  lda % 16 == 0, k_pad % 64 == 0,
 * n_pad % 32 == 0; a holds M whole rows of lda bytes, and for M > 8 both
 * a (M * lda bytes) and the packed weights are under 2 GiB (MR_EINVAL
 * otherwise).  Every packed weight argument of this library stores the
 * logical B[n_pad][k_pad] K-step-major: byte k of row n at
 * ((k / 64) * n_pad + n) * 64 + k % 64. */
int mr_qmatmul(const int8_t* a, int64_t lda, const int8_t* b, int64_t k_pad, int64_t n_pad,
               int64_t M, int64_t N, int64_t K, const mr_epilogue* epi, void* stream);

/* The same for decode shapes whose activation rows are still f32: mira/ops.py:602-603
 * quantize_activation (x / x_scale, as mr_quantize_rows) fused into :616-620, so a
 * decode step's first layer needs no separate quantize launch.  x is [M, ldx] f32
 * (ldx >= K); results equal mr_quantize_rows + mr_qmatmul bit for bit.  M <= 8 and
 * k_pad <= 4096 (MR_EUNSUPPORTED otherwise). */
int mr_qmatmul_f32in(const float* x, int64_t ldx, float x_scale, const int8_t* b,
                     int64_t k_pad, int64_t n_pad, int64_t M, int64_t N, int64_t K,
                     const mr_epilogue* epi, void* stream);

/* The same when the f32 rows are a layernorm's input and the q-op reads only its
 * int8 copy (a transformer decode step's projections after a layernorm): each row
 * of K elements is normalised as mr_layernorm_f32 does (mira/ops.py:356-360: gain
 * gamma[K], bias beta[K], eps; rounded to f16 when round_f16), quantized with
 * x_scale, then multiplied; bit-exact with mr_layernorm_f32 (int8 output) followed
 * by mr_qmatmul.  M <= 8 and k_pad <= 1024 (MR_EUNSUPPORTED otherwise). */
int mr_qmatmul_lnin(const float* x, int64_t ldx, const float* gamma, const float* beta, float eps,
                    int32_t round_f16, float x_scale, const int8_t* b, int64_t k_pad, int64_t n_pad,
                    int64_t M, int64_t N, int64_t K, const mr_epilogue* epi, void* stream);

/* Replaces, for decode-shaped matmuls of the int8 weight-only mode
 * (mira/quantize.py:45-68), mira/ops.py:217-219 _matmul_ref fed by the
 * dequantize constant of mira/ops.py:581-589:
 * y[M,N] = x[M,K] (f32, row stride ldx) @ W, W[k][n] = fl32(q[k][n] *
 * w_scale[n]) (rounded on to f16 when w_f16 != 0: a dequantize of dtype
 * f16) with q packed as B[n_pad][k_pad] (B[n][k] = q[k][n], stored
 * K-step-major as for mr_qmatmul), f32 multiply-adds, then the epilogue (its
 * scale must be NULL and it writes no int32 accumulators).  Up to 16 rows the
 * weights are streamed once per block of 8 rows (decode shapes); more rows run
 * as 128 x 128 tiles on f32 MFMAs when K and ldx are multiples of 4 and x is
 * under 2 GiB, else as 8-row blocks (M <= 524280).  ldx >= K, x and b 16-byte
 * aligned.  The sums run in another order than NumPy's, so the result matches
 * to f32 rounding (relative 1e-5), not bit for bit. */
int mr_w8_matmul_f32(const float* x, int64_t ldx, const int8_t* b, const float* w_scale, int32_t w_f16,
                     int64_t k_pad, int64_t n_pad, int64_t M, int64_t N, int64_t K, const mr_epilogue* epi,
                     void* stream);

/* Replaces, for convolutions of the int8 weight-only mode (mira/quantize.py:45-68),
 * mira/ops.py:265-276 _conv2d_ref (groups 1) over the dequantize constant of
 * mira/ops.py:581-589: y[n,oh,ow,o] (NHWC rows = output pixels) = the convolution of
 * the NHWC f32 image x (g->c channels per pixel, c % 4 == 0) with
 * W[o][c][kh][kw] = fl32(q * w_scale[o]) (rounded on to f16 when w_f16 != 0), q packed
 * as B[n_pad][k_pad] with k = (kh * kw_count + kw) * g->c_pad + c (c_pad % 4 == 0,
 * channels c..c_pad-1 zero), K-step-major as for mr_qmatmul; then the epilogue (scale
 * NULL, no int32 accumulators).  f32 multiply-adds on MFMAs in another order than
 * NumPy's, so the result matches to f32 rounding (relative 1e-5), not bit for bit.
 * x and the weights each under 2 GiB. */
int mr_w8_conv2d_f32(const float* x, const mr_conv_geom* g, const int8_t* b, const float* w_scale, int32_t w_f16,
                     int64_t k_pad, int64_t n_pad, const mr_epilogue* epi, void* stream);

/* Replaces mira/ops.py:630-634 _qconv2d_ref (after quantize_activation):
 * implicit-GEMM convolution of NHWC int8 x with packed weights
 * B[n_pad][k_pad] (stored K-step-major as for mr_qmatmul) whose k index is
 * (kh, kw, c) with c fastest over c_pad
 * (or the stem row layout when c_pad == 4).  Result rows are NHWC pixels
 * (n, oh, ow), columns output channels.  x (n * h * w * c_pad bytes) and the
 * packed weights are each under 2 GiB (MR_EINVAL otherwise). */
int mr_qconv2d(const int8_t* x, const mr_conv_geom* g, const int8_t* b, int64_t k_pad,
               int64_t n_pad, const mr_epilogue* epi, void* stream);

/* Fused stem: mr_qconv2d of a <= 4-channel input (c_pad == 4, o <= 64,
 * output width <= 128, pooled width <= 60 for a 3-wide and <= 64 for a
 * 2-wide pool, weights packed to n_pad >= 64 rows, k_pad <= 256) whose
 * epilogue result feeds a constant pad (pool_pad_* rows/columns of
 * pad_value, mira/ops.py:461-470) and maxpool2d(pool_size, pool_stride)
 * (mira/ops.py:293-296).  Replaces that qconv2d -> pad -> maxpool2d chain;
 * the convolution result is never stored.  `epi` carries the convolution's
 * scale and epilogue steps, while its outputs (out_f32/ldo, out_i8/ldq/out_xs)
 * receive the pooled [n, poh, pow_, o] result in NHWC rows; out_acc must be
 * NULL.  The pool runs on the accumulators, so every epilogue step must be
 * non-decreasing with a scalar or per-channel operand: add, sub (not
 * swapped), maximum, minimum, relu, and mul whose operand the caller
 * guarantees to be positive and finite (it is not read on the host). */
int mr_qconv2d_maxpool(const int8_t* x, const mr_conv_geom* g, const int8_t* b, int64_t k_pad, int64_t n_pad,
                       const mr_epilogue* epi, int32_t pool_size, int32_t pool_stride, int32_t pool_pad_top,
                       int32_t pool_pad_left, float pad_value, int32_t poh, int32_t pow_, void* stream);

/* The same fused stem reading the f32 NCHW image [n, c, h, w] itself: the
 * activation quantizer of mira/ops.py:602-603 (round(x / x_scale) clipped to
 * +-127, of the f16 rounding of x when round_f16 is set: the f32 -> f16 cast
 * of mira/ops.py:405-406 in an f16 graph) followed by mr_qconv2d_maxpool, as
 * one kernel.  Replaces mr_quantize_nchw_nhwc / mr_quantize_f16_nchw_nhwc +
 * mr_qconv2d_maxpool when the stem is the only reader of the image's int8
 * copy, which is then never written.  Same geometry rules (c_pad == 4
 * describes the packed weights), plus: 7 kernel rows of 5 to 8 taps, no
 * dilation, an even column stride, a row stride of at most 2, and input rows
 * of (ow - 1) * sw + 8 pixels forming at most 64 four-pixel groups (ResNet's
 * 224 x 224 stem: 230 pixels, 58 groups); MR_EUNSUPPORTED otherwise. */
int mr_qconv2d_maxpool_f32in(const float* x, float x_scale, int32_t round_f16, const mr_conv_geom* g,
                             const int8_t* b, int64_t k_pad, int64_t n_pad, const mr_epilogue* epi,
                             int32_t pool_size, int32_t pool_stride, int32_t pool_pad_top, int32_t pool_pad_left,
                             float pad_value, int32_t poh, int32_t pow_, void* stream);

/* ---- K4a: f32 depthwise conv ------------------------------------------ */

/* Replaces mira/ops.py:265-276 _conv2d_ref for groups == C, one output per
 * group: acc = 0; for i, j: acc = acc + x_tap*w[i][j] (separate f32
 * multiply and add, taps in (i, j) order), then the epilogue (scale must be
 * NULL).  x NHWC f32 [n,h,w,c], w f32 [kh][kw][c]. */
int mr_dwconv2d_f32(const float* x, const mr_conv_geom* g, const float* w,
                    const mr_epilogue* epi, void* stream);

/* A 1x1 qconv2d whose f32 result only a 3x3 depthwise conv reads, as one
 * launch (a MobileNet block's expansion and depthwise convolution; replaces
 * mira/ops.py:630-634 followed by mira/ops.py:265-276 with groups == C).  The
 * expansion: x NHWC int8 rows of ldx bytes (K real channels, ldx % 16 == 0),
 * packed weights b [k_pad/64][n_pad][64] with n_pad >= dw->c, and its epilogue
 * epi_expand (the dequant scale, bias -> maximum -> minimum, no outputs: its
 * result is never stored).  The depthwise conv: geometry dw (3x3, padding 1,
 * stride 1 or 2, c == o == c_pad, c % 4 == 0), weights w_dw f32 [3][3][c]
 * and epi_dw (bias -> maximum -> minimum, an int8 output and optionally an f32
 * one).  Bit-exact with mr_qconv2d followed by mr_dwconv2d_f32: the expanded
 * values are recomputed for each output tile's halo with the same arithmetic
 * and never leave the chip.  MR_EUNSUPPORTED for other epilogues, f16
 * rounding or k_pad > 192 (the caller then makes the two launches). */
int mr_qconv1x1_dw3x3(const int8_t* x, int64_t ldx, const int8_t* b, int64_t k_pad, int64_t n_pad, int64_t K,
                      const mr_epilogue* epi_expand, const mr_conv_geom* dw, const float* w_dw,
                      const mr_epilogue* epi_dw, void* stream);

/* The same fusion when the first convolution is a network's 3x3 stem (padding 1,
 * stride 1 or 2) over an image of at most 4 channels stored 4 bytes per pixel
 * (mr_quantize_nchw_nhwc with c_pad 4): `stem` is its geometry (c_pad 4, o ==
 * dw->c, output == the depthwise input), b its packed weights in the stem
 * layout (mira_amd.pack.pack_conv(q, 4): kernel row i in the 16-byte chunk i,
 * k_pad 64).  Everything else as mr_qconv1x1_dw3x3; bit-exact with mr_qconv2d
 * followed by mr_dwconv2d_f32. */
int mr_qstem3x3_dw3x3(const int8_t* x, const mr_conv_geom* stem, const int8_t* b, int64_t k_pad, int64_t n_pad,
                      const mr_epilogue* epi_stem, const mr_conv_geom* dw, const float* w_dw,
                      const mr_epilogue* epi_dw, void* stream);

/* ---- adjuncts ---------------------------------------------------------- */

/* mira/ops.py:293-296 maxpool2d with the -inf/constant pad of
 * mira/ops.py:461-470 folded in: NHWC f32 [n,h,w,c] -> [n,oh,ow,c].
 * Optional int8 copy (quantized with xs) into yq with c_pad channels. */
int mr_maxpool2d_f32(const float* x, int32_t n, int32_t h, int32_t w, int32_t c,
                     int32_t size, int32_t stride, int32_t pad_top, int32_t pad_left,
                     float pad_value, int32_t oh, int32_t ow, float* y,
                     int8_t* yq, int32_t c_pad, float xs, void* stream);

/* Replaces mira/ops.py:405-406 cast of an f32 tensor to f16, and the final
 * .astype(float16) of an f16 op that takes no epilogue descriptor (e.g.
 * reduce_mean): y[i] = f32(f16(x[i])), round to nearest even, over n floats
 * (y == x allowed).  f16 tensors stay stored as f32 on the device. */
int mr_round_f16_f32(const float* x, int64_t n, float* y, void* stream);

/* The functions of mr_elementwise_f32 beyond the epilogue codes MR_EPI_ADD .. MR_EPI_RELU. */
enum mr_ew_fn {
  MR_EW_GREATER = 11,
  MR_EW_GREATER_EQUAL = 12,
  MR_EW_EQUAL = 13,
  MR_EW_NEG = 14,
  MR_EW_ABS = 15
};

/* Replaces mira/ops.py:163-169 for one standalone elementwise op (add, sub, mul, div,
 * maximum, minimum, greater, greater_equal, equal; relu, neg, abs) inside a loop the
 * target runs on the device: y[i] over an output of shape[4] (rank <= 4, leading 1s),
 * a and b read at the element strides a_stride[4] / b_stride[4] (0 on broadcast axes;
 * b and b_stride unused by unary functions), computed in f32 with NumPy's float32
 * semantics (NaN through maximum / minimum, comparisons giving 1 / 0), rounded to f16
 * when round_f16 is set.  Host arrays shape / a_stride / b_stride are read at the call. */
int mr_elementwise_f32(int32_t fn, const float* a, const int64_t* a_stride, const float* b, const int64_t* b_stride,
                       float* y, const int64_t* shape, int32_t round_f16, void* stream);

/* ---- device loops: integer and data-movement ops ------------------------
 * Inside a while / if the target runs on the device, every value is 4 bytes per
 * element: f32, f16 values held as f32, and i32 values held as their own bits in the
 * same buffers.  Positions read from device memory are clamped into range. */

enum mr_dtype { MR_DT_F32 = 0, MR_DT_F16 = 1, MR_DT_I32 = 2 };

/* mr_elementwise_f32 for i32 operands (mira/ops.py:163-169 with integers exact): add,
 * sub, mul wrapping around; maximum, minimum, greater, greater_equal, equal (1 / 0);
 * relu, neg, abs. */
int mr_elementwise_i32(int32_t fn, const int32_t* a, const int64_t* a_stride, const int32_t* b,
                       const int64_t* b_stride, int32_t* y, const int64_t* shape, void* stream);

/* Replaces mira/ops.py:405-406 between i32 and f32 / f16 over n elements: integers round
 * to nearest (to f16 in one rounding); floats truncate toward zero, NaN, infinities and
 * values outside int32 giving INT_MIN (NumPy on x86). */
int mr_cast_32(const void* x, int64_t n, int32_t from, int32_t to, void* y, void* stream);

/* Replaces mira/ops.py:479-484 gather along axis 0: y[i, :] = table[idx[i], :] over rows of
 * row_elems 4-byte elements; negative indices count from the end (NumPy's take), indices
 * still out of range are clamped (NumPy raises). */
int mr_gather_rows_32(const void* table, int64_t rows, int64_t row_elems, const int32_t* idx, int64_t n_idx,
                      void* y, void* stream);

/* Replaces mira/ops.py:551-554: y = x[start : start + size] over shape[4] / size[4] (leading
 * axes 1 up to the value's rank), start a device i32[rank] clamped as mira/ops.py:538-539. */
int mr_dynamic_slice_32(const void* x, const int64_t* shape, const int32_t* start, int32_t rank,
                        const int64_t* size, void* y, void* stream);

/* Replaces mira/ops.py:567-572: y = x with the window [start, start + size) replaced by upd
 * (y != x), start clamped as above. */
int mr_dynamic_update_slice_32(const void* x, const int64_t* shape, const void* upd, const int64_t* size,
                               const int32_t* start, int32_t rank, void* y, void* stream);

/* Replaces mira/ops.py:527-528 argmax over the last axis of rows x n f32 values: the first
 * index of the maximum, the first NaN if there is one. */
int mr_argmax_f32(const float* x, int64_t rows, int64_t n, int32_t* y, void* stream);

/* Replaces mira/ops.py:432-433: y = where(cond != 0, a, b) over shape[4], all three read
 * through broadcast strides; cond_int: cond holds i32 (else f32, true when non-zero or NaN). */
int mr_where_32(const void* cond, int32_t cond_int, const int64_t* c_stride, const void* a, const int64_t* a_stride,
                const void* b, const int64_t* b_stride, void* y, const int64_t* shape, void* stream);

/* mira/ops.py:318-343 reduce_mean over H,W (NumPy order: pairwise f32 sum,
 * then f32(f64(sum) / count)).  NHWC f32 [n,hw,c] -> [n,c]; optional int8.
 * out_f16 != 0: the mean is rounded to f16 first (an f16 graph's reduce_mean,
 * whose .astype(float16) then feeds y and the quantize). */
int mr_mean_hw_f32(const float* x, int32_t n, int32_t hw, int32_t c, float* y,
                   int8_t* yq, int32_t ldq, float xs, int32_t out_f16, void* stream);

/* mira/ops.py:461-470 pad with a constant on H and W of an NHWC tensor. */
int mr_pad_hw_f32(const float* x, int32_t n, int32_t h, int32_t w, int32_t c,
                  int32_t top, int32_t bottom, int32_t left, int32_t right,
                  float value, float* y, void* stream);

/* Layout changes at segment boundaries: NCHW <-> NHWC, f32. */
int mr_nchw_to_nhwc_f32(const float* x, int32_t n, int32_t c, int32_t h, int32_t w,
                        float* y, void* stream);

/* NCHW f32 -> NHWC f32 with c_pad >= c channels per pixel (c_pad % 4 == 0),
 * channels c .. c_pad - 1 zero: the input of a weight-only convolution whose
 * channel count is not a multiple of 4 (a 3-channel stem); exact (a copy). */
int mr_nchw_to_nhwc_pad_f32(const float* x, int32_t n, int32_t c, int32_t h, int32_t w,
                            float* y, int32_t c_pad, void* stream);
int mr_nhwc_to_nchw_f32(const float* x, int32_t n, int32_t c, int32_t h, int32_t w,
                        float* y, void* stream);

/* ---- the float ops of a transformer decode step --------------------------
 * Row-major (C order) f32 tensors; f16 results are rounded and stored as f32
 * when out_f16 is set, as for every other op. */

/* Replaces mira/ops.py:356-360 layernorm over the last axis of x [rows, d],
 * bit for bit: NumPy's pairwise f32 sums for both means, each divided by the
 * count in double precision, var + f32(eps), IEEE sqrt and division.  Writes
 * y [rows, d] (if y) and the int8 copy yq [rows, ldq] = clip(rint(y / xs),
 * +-127) of a following q-op's input (if yq, mira/ops.py:602-603). */
int mr_layernorm_f32(const float* x, int64_t rows, int32_t d, const float* gamma,
                     const float* beta, float eps, int32_t out_f16, float* y,
                     int8_t* yq, int64_t ldq, float xs, void* stream);

/* Replaces mira/ops.py:310-313 softmax over the last axis of x [rows, n]:
 * exp(x - max) / sum.  Approximate: expf and the summation order are not
 * NumPy's (relative error ~1e-6 per element). */
int mr_softmax_f32(const float* x, int64_t rows, int32_t n, int32_t out_f16,
                   float* y, void* stream);

/* Replaces mira/ops.py:217-219 matmul of two float tensors with NumPy's
 * batch broadcasting: for each batch index (nb <= 4 dimensions of extents
 * bdim, element strides sa and sw in a and w, 0 where an operand
 * broadcasts), [M, K] @ [K, N] in f32, then the epilogue over the C-order
 * [batches * M, N] result (scale must be NULL).  Both operands are strided
 * views: mk_strides = {a's M stride, a's K stride, w's K stride, w's N
 * stride} in elements, so transposed operands are read in place.
 * Approximate: fused multiply-adds over interleaved k-groups added by a lane
 * butterfly, not BLAS's summation order. */
int mr_bmm_f32(const float* a, const float* w, int32_t nb, const int64_t* bdim,
               const int64_t* sa, const int64_t* sw, const int64_t* mk_strides,
               int64_t M, int64_t N, int64_t K, const mr_epilogue* epi,
               void* stream);

/* Replaces mira/ops.py:375 transpose (np.ascontiguousarray(np.transpose(x,
 * perm))) for rank 1..4; exact (a copy). */
int mr_transpose_f32(const float* x, int32_t rank, const int64_t* shape,
                     const int32_t* perm, float* y, void* stream);

/* One operand of mira/ops.py:403 concat: x viewed as [outer, inner] is copied
 * into columns [at, at + inner) of y viewed as [outer, ld]; exact.  An empty
 * operand (outer * inner == 0) is a no-op and its pointers may be NULL. */
int mr_copy_rows_f32(const float* x, int64_t outer, int64_t inner, float* y,
                     int64_t ld, int64_t at, void* stream);

/* ---- a decode step's attention and the greedy loop around it (examples/gpt_text.mira:60-82) */

/* Replaces, for one decode step, the chain mira/ops.py:217-219 matmul(q,
 * keys^T) -> mul(scale) -> add(mask) -> mira/ops.py:310-313 softmax -> matmul(
 * ., values), where keys and values are a [B, T, H*hd] cache joined by the
 * step's own [B, H*hd] row (mira/ops.py:403 concat at slot T): per sequence b
 * and head h, s_j = (q_bh . k_j) * scale + mask[j] over the T + 1 keys,
 * p = softmax(s), out_bh = sum_j p_j v_j.  q rows have stride ldq; cache row j
 * of sequence b is at b * c_bs + j * c_ld; the new rows have strides ld_kn, ld_vn;
 * mask has T + 1 entries shared by every sequence and head.  out (f32, row
 * stride ldo) and/or out_i8 (clip(rint(out / xs), +-127), row stride ldq8).
 * Approximate like the ops it replaces (expf, f32 multiply-adds in key order):
 * within f32 rounding of NumPy, not bit for bit.  hd in {16, 32, 64},
 * T + 1 <= 1024; strides multiples of 4 floats, operands 16-byte aligned. */
int mr_attention_decode_f32(const float* q, int64_t ldq, const float* k_cache,
                            const float* v_cache, int64_t c_ld, int64_t c_bs,
                            const float* k_new, int64_t ld_kn, const float* v_new,
                            int64_t ld_vn, const float* mask, float scale, int64_t B, int32_t H,
                            int32_t hd, int32_t T, float* out, int64_t ldo,
                            int8_t* out_i8, int64_t ldq8, float xs, void* stream);

#define MR_DECODE_MAX_CACHES 16

/* Start of one step of the greedy decode loop of examples/gpt_text.mira:66-81
 * (the reference runs it on the host through mira/backends/cpu.py:44-51), at
 * position t = *t_io (device int32): h[b, :] = emb[tokens[b, t]] + pos[t]
 * (one f32 add), the step's mask over the T cache rows and its own row
 * (mask[j] = 0 for j < t and j == T, neg otherwise), and *t_cur = t for the
 * step's end.  tokens is [B, ld_tok] int32; emb [V, D], pos [T, D] f32.
 * Token ids are clamped to [0, V) and t to [0, T) on the device so no read
 * leaves its table; the caller keeps them in range. */
int mr_decode_embed(const int32_t* tokens, int64_t ld_tok, const int32_t* t_io,
                    int32_t* t_cur, const float* emb, int32_t V, const float* pos,
                    int32_t T, int32_t D, float* h, int64_t B, float* mask,
                    float neg, void* stream);

/* End of that step at t = *t_cur: rows[k][b, :D] (row stride ld_rows[k]) is
 * stored at row t of caches[k] (row b * c_bs + t * c_ld) for each of the
 * n_caches key/value rows; tokens[b, t + 1] becomes the argmax of
 * logits[b, :V] (NumPy's: first maximum, a NaN first) when t + 1 >= prompt_len
 * (the prompt's own tokens stay otherwise); *t_io = t + 1.  `rows`, `ld_rows`
 * and `caches` are host arrays of n_caches <= MR_DECODE_MAX_CACHES entries. */
int mr_decode_commit(const float* logits, int64_t ldl, int32_t V, int32_t n_caches,
                     const float* const* rows, const int64_t* ld_rows,
                     float* const* caches, int64_t c_ld, int64_t c_bs, int32_t D,
                     int32_t* tokens, int64_t ld_tok, int32_t* t_io,
                     const int32_t* t_cur, int32_t prompt_len, int32_t T,
                     int64_t B, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MIRA_ROCM_H */
