// Fused stem: int8 implicit-GEMM convolution of a <= 4-channel NHWC input
// (mira/ops.py:630-634), its epilogue (bias, ReLU: mira/ops.py:192-199), the
// -inf pad (mira/ops.py:461-470) and max pooling (mira/ops.py:293-296), for
// graphs such as ResNet's 7x7/2 stem followed by a 3x3/2 max pool.
//
// Unfused, the convolution writes its full-resolution f32 output
// (822 MB for ResNet-18 at batch 256) only for the pool to read it back.
// Here a workgroup owns POOL_ROWS output rows of the pool for one image; it
// computes the convolution rows their windows cover, one row at a time
// (<= 128 output pixels x 64 channels: 4 waves x one 32-row MFMA block row),
// applies the epilogue, stages the f32 row in LDS, pools it horizontally and
// folds it into running window maxima kept in registers.  Only the pooled
// f32 / int8 results reach memory.  Max is exact in any order for the
// non-NaN values an epilogue of a finite accumulator produces, so the
// result equals the reference's window maximum bit for bit.
//
// A fragments are loaded straight from global memory (one dword per tap of
// 4 channels, zero outside the image); the weights (<= 64 x k_pad bytes) are
// copied to LDS once per workgroup.
#include "mr_common.hpp"

namespace mr {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int POOL_ROWS = 2;      // pooled output rows per workgroup

// Source of every padding tap: loads are never predicated, their address is
// (a select before the load keeps all of a row's loads in flight at once).
__device__ __attribute__((aligned(64))) int32_t g_stem_zero[16];
constexpr int CROW_LD = 64 + 1;   // f32 stride of a staged convolution row (bank offset)
constexpr int BROW_PAD = 16;      // bytes added to each weight row in LDS (16 rows hit 16 bank groups)

struct StemArgs {
  const int8_t* x;     // NHWC int8, 4 bytes per pixel
  const int8_t* b;     // packed weights [64][k_pad]
  int32_t k_pad;
  int32_t row_bytes;   // packed bytes per kernel row
  int32_t N, H, W, O, OH, OW, KH, KW, SH, SW, PH, PW, DH, DW;
  int32_t pk, ps, ppt, ppl, POH, POW;  // pool size, stride, top/left pad, pooled size
  float pad_value;
};

template <int KSUB, int RB, bool FIXED>
__global__ void __launch_bounds__(256) stem_pool_kernel(const StemArgs a, const EpiDev e) {
  constexpr int KB = KSUB * 32;                // k_pad
  constexpr int BLD = KB + BROW_PAD;
  __shared__ float crow[128 * CROW_LD];
  __shared__ __attribute__((aligned(16))) int8_t bs[64 * BLD];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int img = blockIdx.x / ((a.POH + POOL_ROWS - 1) / POOL_ROWS);
  const int pr0 = (blockIdx.x - img * ((a.POH + POOL_ROWS - 1) / POOL_ROWS)) * POOL_ROWS;

  // weights to LDS: 64 rows x KB bytes, 16 bytes per thread per step
  for (int c = threadIdx.x; c < 64 * KB / 16; c += 256) {
    const int row = c / (KB / 16), k16 = c - row * (KB / 16);
    *reinterpret_cast<v4i*>(bs + row * BLD + k16 * 16) =
        *reinterpret_cast<const v4i*>(a.b + int64_t(row) * a.k_pad + k16 * 16);
  }

  // per-column constants (the column index is lane-fixed): dequant scale and,
  // for the fixed epilogue form, the per-column operand and the scalar bounds
  double scale[2];
  float colv[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int col = min(j * 32 + (lane & 31), a.O - 1);
    scale[j] = e.scale[col];
    colv[j] = FIXED && e.f_col ? e.col_ptr[col] : 0.0f;
  }
  const float lo = FIXED && e.f_lo && e.lo_ptr ? e.lo_ptr[0] : 0.0f;
  const float hi = FIXED && e.f_hi ? e.hi_ptr[0] : 0.0f;

  // running window maxima: this thread owns pooled positions idx = t + 256*i.
  // A window that reaches above or below the convolution output includes the
  // pad value; otherwise it starts empty (-inf is max's identity).
  constexpr int PER_T = (64 * 64 + 255) / 256;   // POW <= 64 positions x 64 channels
  float pmax[POOL_ROWS][PER_T];
#pragma unroll
  for (int r = 0; r < POOL_ROWS; ++r) {
    const int top = (pr0 + r) * a.ps - a.ppt;
    const float init = (top < 0 || top + a.pk > a.OH) ? a.pad_value : -INFINITY;
#pragma unroll
    for (int i = 0; i < PER_T; ++i) pmax[r][i] = init;
  }

  // convolution rows the band's windows touch
  const int cr_lo = max(pr0 * a.ps - a.ppt, 0);
  const int cr_hi = min((pr0 + POOL_ROWS - 1) * a.ps - a.ppt + a.pk - 1, a.OH - 1);
  const int ow = wave * 32 + (lane & 31);           // this lane's A row (output column)
  const int iw0 = ow * a.SW - a.PW;

  // A fragments of convolution row cr straight from global memory.  A 32-byte
  // K step is one kernel row of up to 8 taps (RB == 2: lane halves take taps
  // 0-3 / 4-7) or two kernel rows of up to 4 taps (RB == 1: one row per half).
  const int32_t* ximg = reinterpret_cast<const int32_t*>(a.x) + int64_t(img) * a.H * a.W;
  auto load_row = [&](int cr, v4i (&af)[KSUB]) {
    const int ih0 = cr * a.SH - a.PH;
#pragma unroll
    for (int s = 0; s < KSUB; ++s) {
      const int kh = RB == 2 ? s : 2 * s + (lane >> 5);
      const int kw0 = RB == 2 ? 4 * (lane >> 5) : 0;
      const int ih = ih0 + kh * a.DH;
      const bool row_ok = ow < a.OW && kh < a.KH && unsigned(ih) < unsigned(a.H);
      const int32_t* p = ximg + int64_t(row_ok ? ih : 0) * a.W;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int kw = kw0 + q;
        const int iw = iw0 + kw * a.DW;
        const bool ok = row_ok && kw < a.KW && unsigned(iw) < unsigned(a.W);
        af[s][q] = *(ok ? p + iw : g_stem_zero);
      }
    }
  };

  v4i anext[KSUB];
  if (cr_lo <= cr_hi) load_row(cr_lo, anext);
  for (int cr = cr_lo; cr <= cr_hi; ++cr) {
    v4i afrag[KSUB];
#pragma unroll
    for (int s = 0; s < KSUB; ++s) afrag[s] = anext[s];
    if (cr < cr_hi) load_row(cr + 1, anext);   // in flight during this row's MFMA, epilogue and pooling
    v16i acc[2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][r] = 0;
    __syncthreads();   // weights staged (first row) / previous row's pooling reads done
#pragma unroll
    for (int s = 0; s < KSUB; ++s)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const v4i bf = *reinterpret_cast<const v4i*>(bs + (j * 32 + (lane & 31)) * BLD + s * 32 + (lane >> 5) * 16);
        acc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(afrag[s], bf, acc[j], 0, 0, 0);
      }

    // ---- epilogue of the convolution row, staged in LDS as f32
    // Every lane stores all 32 of its values: rows >= OW and columns >= O land
    // in the padded part of the row buffer and are never read; their operand
    // indices are clamped so every load stays inside the operand.
    const int64_t pix_base = (int64_t(img) * a.OH + cr) * a.OW;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = j * 32 + (lane & 31);
      const int colc = min(col, a.O - 1);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int rw = wave * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        const int64_t pix = pix_base + min(rw, a.OW - 1);
        float y = dequant(acc[j][r], scale[j]);
        if constexpr (FIXED) {
          if (e.f_col) y = __fadd_rn(y, colv[j]);
          if (e.f_full) y = __fadd_rn(y, e.full_ptr[pix * e.full_ld + colc]);
          if (e.f_lo) y = np_maximum(y, lo);
          if (e.f_hi) y = np_minimum(y, hi);
        } else {
          y = epi_generic(e, y, pix, colc);
        }
        crow[rw * CROW_LD + col] = y;
      }
    }
    __syncthreads();

    // ---- pool horizontally and fold into the windows containing this row.
    // Branch-free: positions past the pooled row (pc >= POW) or channel count
    // compute on clamped indices and are simply never stored.
    bool in_win[POOL_ROWS];
#pragma unroll
    for (int r = 0; r < POOL_ROWS; ++r) {
      const int top = (pr0 + r) * a.ps - a.ppt;
      in_win[r] = cr >= top && cr < top + a.pk;
    }
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      const int idx = threadIdx.x + 256 * i;
      const int pc = min(idx >> 6, a.POW - 1), ch = min(idx & 63, a.O - 1);
      float h = -INFINITY;
      for (int t = 0; t < a.pk; ++t) {
        const int c = pc * a.ps - a.ppl + t;
        const float v = crow[min(max(c, 0), a.OW - 1) * CROW_LD + ch];
        h = np_maximum(h, unsigned(c) < unsigned(a.OW) ? v : a.pad_value);
      }
#pragma unroll
      for (int r = 0; r < POOL_ROWS; ++r) pmax[r][i] = in_win[r] ? np_maximum(pmax[r][i], h) : pmax[r][i];
    }
  }

  // ---- pooled results
#pragma unroll
  for (int r = 0; r < POOL_ROWS; ++r) {
    const int pr = pr0 + r;
    if (pr >= a.POH) break;
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      const int idx = threadIdx.x + 256 * i;
      const int pc = idx >> 6, ch = idx & 63;
      if (pc >= a.POW || ch >= a.O) continue;
      const int64_t pix = (int64_t(img) * a.POH + pr) * a.POW + pc;
      epi_store(e, pmax[r][i], pix, ch);
    }
  }
}

template <int KS, int RBV>
static void launch_stem(dim3 grid, hipStream_t s, const StemArgs& a, const EpiDev& e) {
  if (e.fixed)
    hipLaunchKernelGGL((stem_pool_kernel<KS, RBV, true>), grid, dim3(256), 0, s, a, e);
  else
    hipLaunchKernelGGL((stem_pool_kernel<KS, RBV, false>), grid, dim3(256), 0, s, a, e);
}

}  // namespace mr

extern "C" {

int mr_qconv2d_maxpool(const int8_t* x, const mr_conv_geom* cg, const int8_t* b, int64_t k_pad, int64_t n_pad,
                       const mr_epilogue* epi, int32_t pool_size, int32_t pool_stride, int32_t pool_pad_top,
                       int32_t pool_pad_left, float pad_value, int32_t poh, int32_t pow_, void* stream) {
  MR_REQUIRE(x && cg && b, "mr_qconv2d_maxpool: NULL argument");
  const mr_conv_geom& G = *cg;
  MR_REQUIRE(G.n >= 0 && G.h > 0 && G.w > 0 && G.c > 0 && G.c <= 4 && G.c_pad == 4,
             "mr_qconv2d_maxpool: input must hold <= 4 channels in the 4-byte pixel layout");
  MR_REQUIRE(G.o > 0 && G.o <= 64 && n_pad >= 64 && n_pad % 32 == 0,
             "mr_qconv2d_maxpool: needs o <= 64 and weights packed to 64 rows");
  MR_REQUIRE(G.kh > 0 && G.kw > 0 && G.sh > 0 && G.sw > 0 && G.dh > 0 && G.dw > 0 && G.ph >= 0 && G.pw >= 0,
             "mr_qconv2d_maxpool: bad kernel/stride/padding/dilation");
  const int32_t oh = (G.h + 2 * G.ph - G.dh * (G.kh - 1) - 1) / G.sh + 1;
  const int32_t ow = (G.w + 2 * G.pw - G.dw * (G.kw - 1) - 1) / G.sw + 1;
  MR_REQUIRE(oh == G.oh && ow == G.ow && oh > 0 && ow > 0 && ow <= 128,
             "mr_qconv2d_maxpool: convolution output must match the geometry and be <= 128 wide");
  const int32_t row_bytes = 16 * ((G.kw + 3) / 4);
  MR_REQUIRE(row_bytes <= 32, "mr_qconv2d_maxpool: kernels wider than 8 taps are not supported");
  MR_REQUIRE(k_pad >= G.kh * row_bytes && k_pad % 64 == 0 && k_pad <= 256,
             "mr_qconv2d_maxpool: k_pad %lld must cover kh*row_bytes, be a multiple of 64 and <= 256",
             (long long)k_pad);
  MR_REQUIRE(pool_size > 0 && pool_stride > 0 && pool_pad_top >= 0 && pool_pad_left >= 0 &&
                 pool_pad_top < pool_size && pool_pad_left < pool_size,
             "mr_qconv2d_maxpool: bad pool parameters");
  MR_REQUIRE(poh > 0 && pow_ > 0 && pow_ <= 64 && (poh - 1) * pool_stride - pool_pad_top < oh &&
                 (pow_ - 1) * pool_stride - pool_pad_left < ow,
             "mr_qconv2d_maxpool: pooled size %dx%d does not fit the %dx%d convolution output", poh, pow_, oh, ow);
  MR_REQUIRE(reinterpret_cast<uintptr_t>(x) % 4 == 0 && reinterpret_cast<uintptr_t>(b) % 16 == 0,
             "mr_qconv2d_maxpool: misaligned operands");
  mr::EpiDev e;
  const int rc = mr::make_epi(epi, G.o, true, &e);
  if (rc != MR_OK) return rc;
  MR_REQUIRE(!epi->out_acc, "mr_qconv2d_maxpool: no int32 accumulator output (the convolution is not stored)");
  if (G.n == 0) return MR_OK;
  mr::StemArgs a = {};
  a.x = x;
  a.b = b;
  a.k_pad = static_cast<int32_t>(k_pad);
  a.row_bytes = row_bytes;
  a.N = G.n;
  a.H = G.h;
  a.W = G.w;
  a.O = G.o;
  a.OH = oh;
  a.OW = ow;
  a.KH = G.kh;
  a.KW = G.kw;
  a.SH = G.sh;
  a.SW = G.sw;
  a.PH = G.ph;
  a.PW = G.pw;
  a.DH = G.dh;
  a.DW = G.dw;
  a.pk = pool_size;
  a.ps = pool_stride;
  a.ppt = pool_pad_top;
  a.ppl = pool_pad_left;
  a.POH = poh;
  a.POW = pow_;
  a.pad_value = pad_value;
  const int64_t bands = (poh + mr::POOL_ROWS - 1) / mr::POOL_ROWS;
  const int64_t blocks = int64_t(G.n) * bands;
  MR_REQUIRE(blocks < (int64_t(1) << 31), "mr_qconv2d_maxpool: too many images");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool rb2 = row_bytes == 32;   // kw 5..8 (else kw <= 4, 16 bytes per kernel row)
  const dim3 grid(static_cast<unsigned>(blocks));
  switch (k_pad / 32) {
    case 2: rb2 ? mr::launch_stem<2, 2>(grid, s, a, e) : mr::launch_stem<2, 1>(grid, s, a, e); break;
    case 4: rb2 ? mr::launch_stem<4, 2>(grid, s, a, e) : mr::launch_stem<4, 1>(grid, s, a, e); break;
    case 6: rb2 ? mr::launch_stem<6, 2>(grid, s, a, e) : mr::launch_stem<6, 1>(grid, s, a, e); break;
    default: rb2 ? mr::launch_stem<8, 2>(grid, s, a, e) : mr::launch_stem<8, 1>(grid, s, a, e); break;
  }
  MR_LAUNCH_CHECK("qconv2d_maxpool");
  return MR_OK;
}

}  // extern "C"
