// Bandwidth-bound f32 kernels around the int8 contractions:
//   K4a depthwise conv (mira/ops.py:265-276 with groups == C),
//   maxpool with the pad folded in (mira/ops.py:293-296, 461-470),
//   reduce_mean over H,W in NumPy's summation order (mira/ops.py:318-343),
//   constant pad, and NCHW <-> NHWC layout changes at segment boundaries.
// All tensors are NHWC inside a segment; threads run along channels so
// every global access coalesces.
#include "mr_common.hpp"
#include "np_sum.hpp"

namespace mr {

static int grid_1d(int64_t total, int block) {
  int64_t g = (total + block - 1) / block;
  const int64_t cap = int64_t(device_cu_count()) * 64;
  if (g > cap) g = cap;
  if (g < 1) g = 1;
  return static_cast<int>(g);
}

// ---------------------------------------------------------------- depthwise conv

// One thread per output element (pixel, channel).  acc starts at +0 and
// adds each tap's product in (i, j) order with separate roundings, exactly
// like `acc += einsum(...)` per tap in the reference; taps that fall into
// the zero padding still add 0 * w.
// Idx is uint32_t when every index fits (the host checks), else uint64_t:
// 64-bit division is a long software sequence on the GPU.
template <typename Idx>
__global__ void __launch_bounds__(256) dwconv_kernel(const float* __restrict__ x, mr_conv_geom G,
                                                     const float* __restrict__ w, const EpiDev e) {
  const Idx total = Idx(G.n) * G.oh * G.ow * G.c;
  for (Idx t = blockIdx.x * Idx(blockDim.x) + threadIdx.x; t < total; t += Idx(gridDim.x) * blockDim.x) {
    const int c = static_cast<int>(t % Idx(G.c));
    const Idx pix = t / Idx(G.c);
    const int ow = static_cast<int>(pix % Idx(G.ow));
    const Idx r = pix / Idx(G.ow);
    const int oh = static_cast<int>(r % Idx(G.oh));
    const int64_t img = r / Idx(G.oh);
    // Loads go to clamped (always valid) addresses and are selected afterwards,
    // so every tap's load is in flight at once instead of one after another.
    float acc = 0.0f;
    for (int i = 0; i < G.kh; ++i) {
      const int ih = oh * G.sh - G.ph + i * G.dh;
      const bool row_ok = unsigned(ih) < unsigned(G.h);
      const int ihc = min(max(ih, 0), G.h - 1);
      for (int j = 0; j < G.kw; ++j) {
        const int iw = ow * G.sw - G.pw + j * G.dw;
        const int iwc = min(max(iw, 0), G.w - 1);
        const float v = x[((img * G.h + ihc) * G.w + iwc) * G.c + c];
        const float xv = (row_ok && unsigned(iw) < unsigned(G.w)) ? v : 0.0f;
        acc = __fadd_rn(acc, __fmul_rn(xv, w[(i * G.kw + j) * G.c + c]));
      }
    }
    const float y = epi_steps(e, acc, int64_t(pix), c);
    epi_store(e, y, int64_t(pix), c);
  }
}

// 3x3 depthwise convolution, dilation 1, stride SW in both directions,
// C % 4 == 0: a thread owns 4 channels (one 16-byte run of an NHWC pixel) of
// OWT adjacent output columns (4 for stride-1 maps wider than 28 columns, else
// 2: measured on the MobileNetV2 layers) of OHT adjacent output rows, loads each
// of the (OHT-1)*SW + 3 input rows' (OWT-1)*SW + 3 columns once for all of them
// (walking the input rows top to bottom), and keeps its 9 weight runs in
// registers.  Per output element the arithmetic is the one above: +0, then each
// tap's product added in (i, j) order with separate roundings (an output row
// meets its tap rows in that order as the input rows go down).
// EF: EF_GENERIC runs each element's epilogue through epi_steps (any legal
// epilogue); EF_SPEC | flags is a compiled fixed form -- bias, NumPy maximum /
// minimum with a wave-uniform bound, f32 and/or int8 out -- run as
// straight-line code on constants loaded once per thread.
template <int SW, int OWT, int EF, int OHT>
__global__ void __launch_bounds__(256) dwconv3x3_kernel(const float* __restrict__ x, mr_conv_geom G,
                                                        const float* __restrict__ w, const EpiDev e, int cg4,
                                                        int wtiles, bool vec_out) {
  constexpr int KH = 3, KW = 3, IWN = (OWT - 1) * SW + KW, IHN = (OHT - 1) * SW + KH;
  const int item = blockIdx.x * 256 + threadIdx.x;
  if (item >= cg4 * wtiles) return;
  const int oh0 = blockIdx.y * OHT;
  const int64_t img = blockIdx.z;
  const int wt = item / cg4;
  const int c0 = (item - wt * cg4) * 4;
  const int ow0 = wt * OWT;

  float4 wv[KH][KW];
#pragma unroll
  for (int i = 0; i < KH; ++i)
#pragma unroll
    for (int j = 0; j < KW; ++j) wv[i][j] = *reinterpret_cast<const float4*>(w + (i * KW + j) * G.c + c0);

  float acc[OHT][OWT][4];
#pragma unroll
  for (int t = 0; t < OHT; ++t)
#pragma unroll
    for (int k = 0; k < OWT; ++k)
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[t][k][q] = 0.0f;

#pragma unroll
  for (int r = 0; r < IHN; ++r) {   // input rows top to bottom
    const int ih = oh0 * G.sh - G.ph + r;
    const bool row_ok = unsigned(ih) < unsigned(G.h);
    const float* xr = x + ((img * G.h + min(max(ih, 0), G.h - 1)) * G.w) * G.c + c0;
    float4 xin[IWN];
#pragma unroll
    for (int q = 0; q < IWN; ++q) {   // clamped addresses, selected after the load: all in flight at once
      const int iw = ow0 * SW - G.pw + q;
      const float4 v = *reinterpret_cast<const float4*>(xr + int64_t(min(max(iw, 0), G.w - 1)) * G.c);
      xin[q] = row_ok && unsigned(iw) < unsigned(G.w) ? v : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
#pragma unroll
    for (int t = 0; t < OHT; ++t) {   // output row oh0 + t takes this input row as tap row i
      const int i = r - t * SW;
      if (i < 0 || i >= KH) continue;
#pragma unroll
      for (int j = 0; j < KW; ++j)
#pragma unroll
        for (int k = 0; k < OWT; ++k) {
          const float4 xv = xin[k * SW + j];
          acc[t][k][0] = __fadd_rn(acc[t][k][0], __fmul_rn(xv.x, wv[i][j].x));
          acc[t][k][1] = __fadd_rn(acc[t][k][1], __fmul_rn(xv.y, wv[i][j].y));
          acc[t][k][2] = __fadd_rn(acc[t][k][2], __fmul_rn(xv.z, wv[i][j].z));
          acc[t][k][3] = __fadd_rn(acc[t][k][3], __fmul_rn(xv.w, wv[i][j].w));
        }
    }
  }

  if constexpr (EF >= EF_SPEC) {
    constexpr bool S_COL = EF & SF_COL, S_LO = EF & SF_LO, S_HI = EF & SF_HI, S_F32 = EF & SF_F32, S_I8 = EF & SF_I8;
    static_assert(!(EF & SF_FULL), "no full-size operand in the compiled depthwise forms");
    const float4 cv = S_COL ? *reinterpret_cast<const float4*>(e.col_ptr + c0) : make_float4(0.f, 0.f, 0.f, 0.f);
    const float col[4] = {cv.x, cv.y, cv.z, cv.w};
    const float lo = S_LO && e.lo_ptr ? e.lo_ptr[0] : 0.0f;
    const float hi = S_HI ? e.hi_ptr[0] : 0.0f;
    const bool lo_nan = lo != lo, hi_nan = hi != hi;
#pragma unroll
    for (int t = 0; t < OHT; ++t) {
      const int oh = oh0 + t;
      if (oh >= G.oh) break;
#pragma unroll
      for (int k = 0; k < OWT; ++k) {
        const int ow = ow0 + k;
        if (ow >= G.ow) break;
        const int64_t pix = (img * G.oh + oh) * G.ow + ow;
        float y[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float v = acc[t][k][q];
          if constexpr (S_COL) v = __fadd_rn(v, col[q]);
          if constexpr (S_LO) v = max_bound(v, lo, lo_nan);
          if constexpr (S_HI) v = min_bound(v, hi, hi_nan);
          y[q] = v;
        }
        if constexpr (S_F32) *reinterpret_cast<float4*>(e.out_f32 + pix * e.ldo + c0) = make_float4(y[0], y[1], y[2], y[3]);
        if constexpr (S_I8) {
          uint32_t packed = 0;
#pragma unroll
          for (int q = 0; q < 4; ++q) packed |= uint32_t(uint8_t(quantize_rcp(y[q], e.out_rxs))) << (8 * q);
          *reinterpret_cast<uint32_t*>(e.out_i8 + pix * e.ldq + c0) = packed;
        }
      }
    }
    return;
  }
#pragma unroll 1
  for (int t = 0; t < OHT; ++t) {
    const int oh = oh0 + t;
    if (oh >= G.oh) break;
#pragma unroll 1
    for (int k = 0; k < OWT; ++k) {
      const int ow = ow0 + k;
      if (ow >= G.ow) break;
      const int64_t pix = (img * G.oh + oh) * G.ow + ow;
      float y[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) y[q] = epi_steps(e, acc[t][k][q], pix, c0 + q);
      if (vec_out) {   // 16-byte f32 and 4-byte int8 runs (alignment checked on the host)
        if (e.out_f32) *reinterpret_cast<float4*>(e.out_f32 + pix * e.ldo + c0) = make_float4(y[0], y[1], y[2], y[3]);
        if (e.out_i8) {
          uint32_t packed = 0;
#pragma unroll
          for (int q = 0; q < 4; ++q) packed |= uint32_t(uint8_t(quantize_rcp(y[q], e.out_rxs))) << (8 * q);
          *reinterpret_cast<uint32_t*>(e.out_i8 + pix * e.ldq + c0) = packed;
        }
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) epi_store(e, y[q], pix, c0 + q);
      }
    }
  }
}

// ---------------------------------------------------------------- f16 rounding

// y[i] = f32(f16(x[i])): a cast to f16 (mira/ops.py:405-406) or the final
// .astype(float16) of an op without an epilogue descriptor, on f32 storage.
__global__ void __launch_bounds__(256) round_f16_kernel(const float* __restrict__ x, int64_t n, float* y) {
  const int64_t stride = int64_t(gridDim.x) * 256;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride) y[i] = round_f16(x[i]);
}

// ---------------------------------------------------------------- standalone elementwise

// An elementwise op over an output of rank <= 4 (dims n[0..3], leading 1s), each operand
// read through element strides (0 on its broadcast axes): mira/ops.py:163-169, computed in
// f32 as NumPy does for float32 operands, then rounded to f16 for an f16 op.  Comparisons
// give 1 / 0 (mira/ops.py:134-140).
struct EwShape {
  int64_t n[4];
  int64_t sa[4];
  int64_t sb[4];
};

__device__ __forceinline__ float ew_apply(int fn, float a, float b) {
  switch (fn) {
    case MR_EPI_RELU: return np_maximum(a, 0.0f);
    case MR_EW_GREATER: return a > b ? 1.0f : 0.0f;
    case MR_EW_GREATER_EQUAL: return a >= b ? 1.0f : 0.0f;
    case MR_EW_EQUAL: return a == b ? 1.0f : 0.0f;
    case MR_EW_NEG: return -a;
    case MR_EW_ABS: return fabsf(a);
    default: return epi_binary(fn, a, b);
  }
}

__global__ void __launch_bounds__(256) elementwise_kernel(int fn, const float* __restrict__ a,
                                                          const float* __restrict__ b, float* __restrict__ y,
                                                          const EwShape sh, int64_t total, int f16) {
  const int64_t stride = int64_t(gridDim.x) * 256;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < total; i += stride) {
    int64_t r = i, ia = 0, ib = 0;
#pragma unroll
    for (int d = 3; d >= 0; --d) {
      const int64_t c = r % sh.n[d];
      r /= sh.n[d];
      ia += c * sh.sa[d];
      ib += c * sh.sb[d];
    }
    float v = ew_apply(fn, a[ia], b ? b[ib] : 0.0f);
    y[i] = f16 ? round_f16(v) : v;
  }
}

// ---------------------------------------------------------------- maxpool

template <typename Idx>
__global__ void __launch_bounds__(256) maxpool_kernel(const float* __restrict__ x, int n, int h, int w, int c,
                                                      int size, int stride, int pt, int pl, float pad_value, int oh,
                                                      int ow, float* __restrict__ y, int8_t* __restrict__ yq,
                                                      int c_pad, float xs) {
  const Idx total = Idx(n) * oh * ow * c;
  for (Idx t = blockIdx.x * Idx(blockDim.x) + threadIdx.x; t < total; t += Idx(gridDim.x) * blockDim.x) {
    const int ch = static_cast<int>(t % Idx(c));
    const int64_t pix = t / Idx(c);
    const int ox = static_cast<int>(Idx(pix) % Idx(ow));
    const Idx r = Idx(pix) / Idx(ow);
    const int oy = static_cast<int>(r % Idx(oh));
    const int64_t img = r / Idx(oh);
    float m = 0.0f;
    for (int i = 0; i < size; ++i) {
      const int ih = oy * stride - pt + i;
      const int ihc = min(max(ih, 0), h - 1);
      for (int j = 0; j < size; ++j) {
        const int iw = ox * stride - pl + j;
        const int iwc = min(max(iw, 0), w - 1);
        const float ld = x[((img * h + ihc) * w + iwc) * c + ch];   // unpredicated: all taps in flight
        const float v = (unsigned(ih) < unsigned(h) && unsigned(iw) < unsigned(w)) ? ld : pad_value;
        m = (i == 0 && j == 0) ? v : np_maximum(m, v);
      }
    }
    if (y) y[pix * c + ch] = m;
    if (yq) yq[pix * c_pad + ch] = quantize_one(m, xs);
  }
}

// ---------------------------------------------------------------- mean over H*W

// y[img, ch] = f32(f64(pairwise_sum) / f64(hw)): NumPy's mean divides the f32
// sum by the intp count in a double-precision loop and casts back.
__global__ void __launch_bounds__(256) mean_hw_kernel(const float* __restrict__ x, int n, int hw, int c,
                                                      float* __restrict__ y, int8_t* __restrict__ yq, int ldq,
                                                      float xs, int out_f16) {
  const int64_t total = int64_t(n) * c;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int ch = static_cast<int>(t % c);
    const int64_t img = t / c;
    const float s = pairwise_sum(x + img * hw * c + ch, hw, c);
    float m = static_cast<float>(__ddiv_rn(static_cast<double>(s), static_cast<double>(hw)));
    if (out_f16) m = round_f16(m);   // an f16 op's .astype(float16), before the next q-op's quantize
    if (y) y[t] = m;
    if (yq) yq[img * ldq + ch] = quantize_one(m, xs);
  }
}

// ---------------------------------------------------------------- pad / layout

template <typename Idx>
__global__ void __launch_bounds__(256) pad_kernel(const float* __restrict__ x, int n, int h, int w, int c, int top,
                                                  int left, int oh, int ow, float value, float* __restrict__ y) {
  const Idx total = Idx(n) * oh * ow * c;
  for (Idx t = blockIdx.x * Idx(blockDim.x) + threadIdx.x; t < total; t += Idx(gridDim.x) * blockDim.x) {
    const int ch = static_cast<int>(t % Idx(c));
    const Idx pix = t / Idx(c);
    const int ox = static_cast<int>(pix % Idx(ow));
    const Idx r = pix / Idx(ow);
    const int oy = static_cast<int>(r % Idx(oh));
    const int64_t img = r / Idx(oh);
    const int ih = oy - top, iw = ox - left;
    y[t] = (unsigned(ih) < unsigned(h) && unsigned(iw) < unsigned(w)) ? x[((img * h + ih) * w + iw) * c + ch]
                                                                       : value;
  }
}

// Tiled transpose of a [rows, cols] matrix per image (32x32 tiles in LDS):
// NCHW -> NHWC is rows = C, cols = H*W; NHWC -> NCHW swaps them.
__global__ void __launch_bounds__(256) transpose_kernel(const float* __restrict__ x, int rows, int cols,
                                                        float* __restrict__ y) {
  __shared__ float tile[32][33];
  const int64_t img = blockIdx.z;
  const float* xi = x + img * int64_t(rows) * cols;
  float* yi = y + img * int64_t(rows) * cols;
  const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
  for (int i = threadIdx.y; i < 32; i += 8) {
    const int r = r0 + i, cc = c0 + threadIdx.x;
    if (r < rows && cc < cols) tile[i][threadIdx.x] = xi[int64_t(r) * cols + cc];
  }
  __syncthreads();
  for (int i = threadIdx.y; i < 32; i += 8) {
    const int cc = c0 + i, r = r0 + threadIdx.x;
    if (r < rows && cc < cols) yi[int64_t(cc) * rows + r] = tile[threadIdx.x][i];
  }
}

// NCHW f32 -> NHWC f32 with c_pad >= c channels per pixel, channels c .. c_pad - 1 zero:
// thread t writes one 16-byte group of 4 channels of one pixel (c_pad % 4 == 0).
__global__ void __launch_bounds__(256) nchw_to_nhwc_pad_kernel(const float* __restrict__ x, int c, int64_t hw,
                                                               int c_pad, int64_t total, float* __restrict__ y) {
  const int groups = c_pad >> 2;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
    const int g = static_cast<int>(t % groups);
    const int64_t pix = t / groups;           // image * hw + p
    const int64_t img = pix / hw, p = pix - img * hw;
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int ch = 4 * g + j;
      v[j] = ch < c ? x[(img * c + ch) * hw + p] : 0.0f;
    }
    *reinterpret_cast<float4*>(y + pix * c_pad + 4 * g) = make_float4(v[0], v[1], v[2], v[3]);
  }
}

static int transpose(const float* x, int n, int rows, int cols, float* y, hipStream_t s) {
  dim3 grid((cols + 31) / 32, (rows + 31) / 32, n);
  hipLaunchKernelGGL(transpose_kernel, grid, dim3(32, 8), 0, s, x, rows, cols, y);
  MR_LAUNCH_CHECK("transpose");
  return MR_OK;
}

}  // namespace mr

extern "C" {

int mr_dwconv2d_f32(const float* x, const mr_conv_geom* cg, const float* w, const mr_epilogue* epi, void* stream) {
  MR_REQUIRE(x && cg && w, "mr_dwconv2d_f32: NULL argument");
  const mr_conv_geom& G = *cg;
  MR_REQUIRE(G.n >= 0 && G.h > 0 && G.w > 0 && G.c > 0, "mr_dwconv2d_f32: bad shape");
  MR_REQUIRE(G.o == G.c && G.c_pad == G.c, "mr_dwconv2d_f32: depthwise needs o == c == c_pad");
  MR_REQUIRE(G.kh > 0 && G.kw > 0 && G.sh > 0 && G.sw > 0 && G.dh > 0 && G.dw > 0 && G.ph >= 0 && G.pw >= 0,
             "mr_dwconv2d_f32: bad kernel/stride/padding/dilation");
  const int32_t oh = (G.h + 2 * G.ph - G.dh * (G.kh - 1) - 1) / G.sh + 1;
  const int32_t ow = (G.w + 2 * G.pw - G.dw * (G.kw - 1) - 1) / G.sw + 1;
  MR_REQUIRE(oh == G.oh && ow == G.ow && oh > 0 && ow > 0, "mr_dwconv2d_f32: output size mismatch");
  mr::EpiDev e;
  const int rc = mr::make_epi(epi, G.c, false, &e);
  if (rc != MR_OK) return rc;
  MR_REQUIRE(!epi->out_acc, "mr_dwconv2d_f32: no int32 accumulators");
  const int64_t total = int64_t(G.n) * oh * ow * G.c;
  if (total == 0) return MR_OK;
  const int64_t in_total = int64_t(G.n) * G.h * G.w * G.c;
  // 3x3, dilation 1, equal strides 1 or 2, 16-byte channel runs: the vectorized kernel
  if (G.kh == 3 && G.kw == 3 && G.dh == 1 && G.dw == 1 && G.sh == G.sw && (G.sh == 1 || G.sh == 2) &&
      G.c % 4 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0 &&
      G.n <= 65535 && oh <= 65535) {
    const int cg4 = G.c / 4;
    const int owt = G.sh == 1 && ow > 28 ? 4 : 2;
    const int wtiles = (ow + owt - 1) / owt;
    const bool vec_out = (!e.out_f32 || (e.ldo % 4 == 0 && reinterpret_cast<uintptr_t>(e.out_f32) % 16 == 0)) &&
                         (!e.out_i8 || (e.ldq % 4 == 0 && reinterpret_cast<uintptr_t>(e.out_i8) % 4 == 0));
    // two output rows per thread with a compiled epilogue (11 % faster than one over the MobileNetV2 layers),
    // one with the step interpreter (where two measured 10 % slower)
    auto grid = [&](int oht) {
      return dim3(static_cast<unsigned>((int64_t(cg4) * wtiles + 255) / 256),
                  static_cast<unsigned>((oh + oht - 1) / oht), static_cast<unsigned>(G.n));
    };
    // compiled forms: bias + ReLU6 / ReLU (maximum, minimum with scalars) to f32 and/or int8
    int form = vec_out && (!e.f_col || reinterpret_cast<uintptr_t>(e.col_ptr) % 16 == 0) ? mr::spec_form(e) : -1;
    constexpr int R6 = mr::SF_COL | mr::SF_LO | mr::SF_HI, R = mr::SF_COL | mr::SF_LO;
#define MR_DW_LAUNCH(SWV, OWTV, EFV)                                                                    \
  hipLaunchKernelGGL((mr::dwconv3x3_kernel<SWV, OWTV, (EFV), (EFV) == mr::EF_GENERIC ? 1 : 2>),               \
                     grid((EFV) == mr::EF_GENERIC ? 1 : 2), dim3(256), 0, static_cast<hipStream_t>(stream), x, G, w, \
                     e, cg4, wtiles, vec_out)
#define MR_DW_FORMS(SWV, OWTV)                                                                             \
  switch (form) {                                                                                          \
    case R6 | mr::SF_F32 | mr::SF_I8: MR_DW_LAUNCH(SWV, OWTV, mr::EF_SPEC | R6 | mr::SF_F32 | mr::SF_I8); break; \
    case R6 | mr::SF_I8: MR_DW_LAUNCH(SWV, OWTV, mr::EF_SPEC | R6 | mr::SF_I8); break;                     \
    case R6 | mr::SF_F32: MR_DW_LAUNCH(SWV, OWTV, mr::EF_SPEC | R6 | mr::SF_F32); break;                   \
    case R | mr::SF_F32 | mr::SF_I8: MR_DW_LAUNCH(SWV, OWTV, mr::EF_SPEC | R | mr::SF_F32 | mr::SF_I8); break; \
    case R | mr::SF_I8: MR_DW_LAUNCH(SWV, OWTV, mr::EF_SPEC | R | mr::SF_I8); break;                       \
    default: MR_DW_LAUNCH(SWV, OWTV, mr::EF_GENERIC); break;                                              \
  }
    if (G.sh == 2) {
      MR_DW_FORMS(2, 2)
    } else if (owt == 4) {
      MR_DW_FORMS(1, 4)
    } else {
      MR_DW_FORMS(1, 2)
    }
#undef MR_DW_FORMS
#undef MR_DW_LAUNCH
    MR_LAUNCH_CHECK("dwconv2d");
    return MR_OK;
  }
  if (total < (int64_t(1) << 32) - 65536 * 256 && in_total < (int64_t(1) << 32))
    hipLaunchKernelGGL(mr::dwconv_kernel<uint32_t>, dim3(mr::grid_1d(total, 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), x, G, w, e);
  else
    hipLaunchKernelGGL(mr::dwconv_kernel<uint64_t>, dim3(mr::grid_1d(total, 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), x, G, w, e);
  MR_LAUNCH_CHECK("dwconv2d");
  return MR_OK;
}

int mr_maxpool2d_f32(const float* x, int32_t n, int32_t h, int32_t w, int32_t c, int32_t size, int32_t stride,
                     int32_t pad_top, int32_t pad_left, float pad_value, int32_t oh, int32_t ow, float* y,
                     int8_t* yq, int32_t c_pad, float xs, void* stream) {
  MR_REQUIRE(x && (y || yq), "mr_maxpool2d_f32: NULL argument");
  MR_REQUIRE(n >= 0 && h > 0 && w > 0 && c > 0 && size > 0 && stride > 0 && pad_top >= 0 && pad_left >= 0,
             "mr_maxpool2d_f32: bad shape");
  MR_REQUIRE(oh > 0 && ow > 0, "mr_maxpool2d_f32: empty output");
  // every window must start inside the padded extent the host described
  MR_REQUIRE((oh - 1) * stride - pad_top < h && (ow - 1) * stride - pad_left < w,
             "mr_maxpool2d_f32: output %dx%d too large for input %dx%d", oh, ow, h, w);
  if (yq) {
    MR_REQUIRE(c_pad >= c, "mr_maxpool2d_f32: c_pad < c");
    MR_REQUIRE(xs > 0.0f, "mr_maxpool2d_f32: requant scale must be positive");
  }
  const int64_t total = int64_t(n) * oh * ow * c;
  if (total == 0) return MR_OK;
  if (total < (int64_t(1) << 32) - 65536 * 256)
    hipLaunchKernelGGL(mr::maxpool_kernel<uint32_t>, dim3(mr::grid_1d(total, 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), x, n, h, w, c, size, stride, pad_top, pad_left, pad_value,
                       oh, ow, y, yq, c_pad, xs);
  else
    hipLaunchKernelGGL(mr::maxpool_kernel<uint64_t>, dim3(mr::grid_1d(total, 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), x, n, h, w, c, size, stride, pad_top, pad_left, pad_value,
                       oh, ow, y, yq, c_pad, xs);
  MR_LAUNCH_CHECK("maxpool2d");
  return MR_OK;
}

int mr_mean_hw_f32(const float* x, int32_t n, int32_t hw, int32_t c, float* y, int8_t* yq, int32_t ldq, float xs,
                   int32_t out_f16, void* stream) {
  MR_REQUIRE(x && (y || yq), "mr_mean_hw_f32: NULL argument");
  MR_REQUIRE(n >= 0 && hw > 0 && c > 0, "mr_mean_hw_f32: bad shape");
  if (yq) {
    MR_REQUIRE(ldq >= c, "mr_mean_hw_f32: ldq < c");
    MR_REQUIRE(xs > 0.0f, "mr_mean_hw_f32: requant scale must be positive");
  }
  const int64_t total = int64_t(n) * c;
  if (total == 0) return MR_OK;
  hipLaunchKernelGGL(mr::mean_hw_kernel, dim3(mr::grid_1d(total, 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, n, hw, c, y, yq, ldq, xs, out_f16 != 0);
  MR_LAUNCH_CHECK("mean_hw");
  return MR_OK;
}

int mr_pad_hw_f32(const float* x, int32_t n, int32_t h, int32_t w, int32_t c, int32_t top, int32_t bottom,
                  int32_t left, int32_t right, float value, float* y, void* stream) {
  MR_REQUIRE(x && y, "mr_pad_hw_f32: NULL argument");
  MR_REQUIRE(n >= 0 && h > 0 && w > 0 && c > 0 && top >= 0 && bottom >= 0 && left >= 0 && right >= 0,
             "mr_pad_hw_f32: bad shape");
  const int oh = h + top + bottom, ow = w + left + right;
  const int64_t total = int64_t(n) * oh * ow * c;
  if (total == 0) return MR_OK;
  if (total < (int64_t(1) << 32) - 65536 * 256)
    hipLaunchKernelGGL(mr::pad_kernel<uint32_t>, dim3(mr::grid_1d(total, 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), x, n, h, w, c, top, left, oh, ow, value, y);
  else
    hipLaunchKernelGGL(mr::pad_kernel<uint64_t>, dim3(mr::grid_1d(total, 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), x, n, h, w, c, top, left, oh, ow, value, y);
  MR_LAUNCH_CHECK("pad_hw");
  return MR_OK;
}

int mr_round_f16_f32(const float* x, int64_t n, float* y, void* stream) {
  MR_REQUIRE(x && y, "mr_round_f16_f32: NULL argument");
  MR_REQUIRE(n >= 0, "mr_round_f16_f32: bad size");
  if (n == 0) return MR_OK;
  hipLaunchKernelGGL(mr::round_f16_kernel, dim3(mr::grid_1d(n, 256)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     x, n, y);
  MR_LAUNCH_CHECK("round_f16");
  return MR_OK;
}

int mr_elementwise_f32(int32_t fn, const float* a, const int64_t* a_stride, const float* b, const int64_t* b_stride,
                       float* y, const int64_t* shape, int32_t round_f16, void* stream) {
  const bool unary = fn == MR_EPI_RELU || fn == MR_EW_NEG || fn == MR_EW_ABS;
  const bool binary = (fn >= MR_EPI_ADD && fn <= MR_EPI_MIN) || fn == MR_EW_GREATER || fn == MR_EW_GREATER_EQUAL ||
                      fn == MR_EW_EQUAL;
  MR_REQUIRE(unary || binary, "mr_elementwise_f32: unknown function %d", fn);
  MR_REQUIRE(a && a_stride && y && shape, "mr_elementwise_f32: NULL argument");
  MR_REQUIRE(!binary || (b && b_stride), "mr_elementwise_f32: a binary function needs b and its strides");
  mr::EwShape sh = {};
  int64_t total = 1;
  for (int d = 0; d < 4; ++d) {
    MR_REQUIRE(shape[d] >= 0 && a_stride[d] >= 0 && (!binary || b_stride[d] >= 0), "mr_elementwise_f32: bad shape");
    sh.n[d] = shape[d];
    sh.sa[d] = a_stride[d];
    sh.sb[d] = binary ? b_stride[d] : 0;
    total *= shape[d];
  }
  if (total == 0) return MR_OK;
  hipLaunchKernelGGL(mr::elementwise_kernel, dim3(mr::grid_1d(total, 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), fn, a, binary ? b : nullptr, y, sh, total, round_f16 ? 1 : 0);
  MR_LAUNCH_CHECK("elementwise");
  return MR_OK;
}

int mr_nchw_to_nhwc_f32(const float* x, int32_t n, int32_t c, int32_t h, int32_t w, float* y, void* stream) {
  MR_REQUIRE(x && y && x != y, "mr_nchw_to_nhwc_f32: bad pointers");
  MR_REQUIRE(n >= 0 && c > 0 && h > 0 && w > 0 && n < 65536, "mr_nchw_to_nhwc_f32: bad shape");
  if (n == 0) return MR_OK;
  return mr::transpose(x, n, c, h * w, y, static_cast<hipStream_t>(stream));
}

int mr_nchw_to_nhwc_pad_f32(const float* x, int32_t n, int32_t c, int32_t h, int32_t w, float* y, int32_t c_pad,
                            void* stream) {
  MR_REQUIRE(x && y && x != y, "mr_nchw_to_nhwc_pad_f32: bad pointers");
  MR_REQUIRE(n >= 0 && c > 0 && h > 0 && w > 0, "mr_nchw_to_nhwc_pad_f32: bad shape");
  MR_REQUIRE(c_pad >= c && c_pad % 4 == 0, "mr_nchw_to_nhwc_pad_f32: c_pad %d must be >= c and a multiple of 4",
             c_pad);
  MR_REQUIRE(reinterpret_cast<uintptr_t>(y) % 16 == 0, "mr_nchw_to_nhwc_pad_f32: y must be 16-byte aligned");
  const int64_t total = int64_t(n) * h * w * (c_pad / 4);
  if (total == 0) return MR_OK;
  hipLaunchKernelGGL(mr::nchw_to_nhwc_pad_kernel, dim3(mr::grid_1d(total, 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, c, int64_t(h) * w, c_pad, total, y);
  MR_LAUNCH_CHECK("nchw_to_nhwc_pad");
  return MR_OK;
}

int mr_nhwc_to_nchw_f32(const float* x, int32_t n, int32_t c, int32_t h, int32_t w, float* y, void* stream) {
  MR_REQUIRE(x && y && x != y, "mr_nhwc_to_nchw_f32: bad pointers");
  MR_REQUIRE(n >= 0 && c > 0 && h > 0 && w > 0 && n < 65536, "mr_nhwc_to_nchw_f32: bad shape");
  if (n == 0) return MR_OK;
  return mr::transpose(x, n, h * w, c, y, static_cast<hipStream_t>(stream));
}

}  // extern "C"
