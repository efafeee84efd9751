// Fused stem: int8 implicit-GEMM convolution of a <= 4-channel NHWC input
// (mira/ops.py:630-634), its epilogue (mira/ops.py:192-199), a constant pad
// (mira/ops.py:461-470) and max pooling (mira/ops.py:293-296), for graphs such
// as ResNet's 7x7/2 stem followed by a 3x3/2 max pool.
//
// Unfused, the convolution writes its full-resolution result (822 MB of f32
// for ResNet-18 at batch 256) only for the pool to read it back.  Here the
// pool runs on the int32 accumulators and the epilogue only on the pooled
// values: for a fixed output channel the epilogue is a non-decreasing
// function of the accumulator (dequant by a positive scale, then adds,
// subtractions of a constant, maximum/minimum with constants: the host only
// fuses such epilogues), so the maximum over a window commutes with it, and
// max(f(a1), .., f(ak)) == f(max(a1, .., ak)) bit for bit (the values are never
// NaN unless an epilogue operand is, in which case both sides are NaN).  The
// pad value joins a window through NumPy's maximum after the epilogue.
//
// A workgroup owns BAND pooled rows of one image.  It walks the convolution
// rows their windows cover, one at a time: 4 waves x one 32-pixel MFMA block
// row (<= 128 output columns x 64 channels, weights held in registers), the
// int32 row goes to LDS as [channel][column], and each lane (one channel)
// max-pools its wave's 16 pooled columns horizontally and folds them into the
// running maxima of the pooled rows whose windows contain the row.  A pooled
// row is finished (epilogue, f32 and int8 stores, 64 channels per store)
// when its last convolution row has been folded in.
#include "mr_common.hpp"

#include <climits>

namespace mr {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int BAND = 8;           // pooled rows per workgroup
constexpr int CRW = 132;          // int32 slots per channel in a staged row: columns -4 .. 127
constexpr int COL_OFF = 4;        // slot of convolution column 0
constexpr int BUF_DWORD3 = 0x00020000;   // buffer resource word 3 for raw 32-bit loads on gfx9

// Source of every padding tap: loads are never predicated, their address is
// (a select before the load keeps all of a row's loads in flight at once).
__device__ __attribute__((aligned(64))) int32_t g_stem_zero[16];

struct StemArgs {
  const int8_t* x;     // NHWC int8, 4 bytes per pixel
  const int8_t* b;     // packed weights, K-step-major [k_pad / 64][n_pad >= 64][64]
  int32_t k_pad, n_pad;
  int32_t row_bytes;   // packed bytes per kernel row
  int32_t N, H, W, O, OH, OW, KH, KW, SH, SW, PH, PW, DH, DW;
  int32_t ppt, POH, POW;  // pool top pad, pooled size
  float pad_value;
};

// KSUB: 32-byte K steps holding kernel rows; RB: 16-byte chunks per kernel
// row; PK: pool window (3: rows/columns 2p-1 .. 2p+1, pad 1; 2: 2p .. 2p+1,
// pad 0), stride 2.
template <int KSUB, int RB, int PK, int EF>
__global__ void __launch_bounds__(256) stem_pool_kernel(const StemArgs a, const EpiDev e) {
  constexpr int PS = 2;
  constexpr int PPL = PK == 3 ? 1 : 0;
  // pooled columns of wave w: 16w .. 16w+15; their windows read staged slots
  // [RD0 + 32w, + 4*NRD) of the lane's channel
  constexpr int SPAN_LO = COL_OFF - PPL;                  // slot of the first window column of pooled column 0
  constexpr int RD0 = SPAN_LO & ~3;                       // aligned start of a wave's reads (wave 0)
  constexpr int REL = SPAN_LO - RD0;                      // first window slot relative to the read start
  constexpr int NRD = (REL + 15 * PS + PK + 3) / 4;       // 16-byte reads per lane
  static_assert(RD0 + 48 * PS + 4 * NRD <= CRW, "pool reads stay inside the staged row");

  __shared__ __attribute__((aligned(16))) int32_t crow[2][64 * CRW];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform: keeps per-wave values scalar
  const int bands = (a.POH + BAND - 1) / BAND;
  const int img = blockIdx.x / bands;
  const int pr0 = (blockIdx.x - img * bands) * BAND;
  const int pr_end = min(pr0 + BAND, a.POH);

  // weights: lane holds rows (32j + lane%32), K bytes 32s + 16*(lane/32) .. +16
  v4i bw[KSUB][2];
#pragma unroll
  for (int s = 0; s < KSUB; ++s)
#pragma unroll
    for (int j = 0; j < 2; ++j)
      bw[s][j] = *reinterpret_cast<const v4i*>(a.b + (int64_t(s >> 1) * a.n_pad + j * 32 + (lane & 31)) * 64 +
                                               (s & 1) * 32 + (lane >> 5) * 16);

  // pool-phase role: this lane is output channel `lane`
  const int ch = lane;
  const int chc = min(ch, a.O - 1);
  const double scale = e.scale[chc];
  constexpr bool FIXED = EF != EF_GENERIC;
  const float colv = FIXED && e.f_col ? e.col_ptr[chc] : 0.0f;
  const float lo = FIXED && e.f_lo && e.lo_ptr ? e.lo_ptr[0] : 0.0f;
  const float hi = FIXED && e.f_hi ? e.hi_ptr[0] : 0.0f;

  const int ow = wave * 32 + (lane & 31);           // this lane's A row (output column)
  const int iw0 = ow * a.SW - a.PW;

  // A fragments of convolution row cr straight from global memory.  A 32-byte
  // K step is one kernel row of up to 8 taps (RB == 2: lane halves take taps
  // 0-3 / 4-7) or two kernel rows of up to 4 taps (RB == 1: one row per half).
  // Each input row is read through a buffer resource spanning exactly that row
  // (none for rows outside the image), and each lane's tap columns are fixed
  // byte offsets into it: the hardware returns 0 for every tap outside the
  // image, so the loads need no address arithmetic, masking or branches.  Taps
  // past the kernel (kh >= KH, kw >= KW) read whatever is there: their packed
  // weights are zero.
  const int32_t* ximg = reinterpret_cast<const int32_t*>(a.x) + int64_t(img) * a.H * a.W;
  const int kw0 = RB == 2 ? 4 * (lane >> 5) : 0;
  int cofs[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) cofs[q] = (iw0 + (kw0 + q) * a.DW) * 4;   // negative -> out of range
  auto load_row = [&](int cr, v4i (&af)[KSUB]) {
#pragma unroll
    for (int s = 0; s < KSUB; ++s) {
      if constexpr (RB == 2) {
        const int ih = cr * a.SH - a.PH + s * a.DH;
        const bool ok = unsigned(ih) < unsigned(a.H);
        const __amdgpu_buffer_rsrc_t row = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<int32_t*>(ximg + int64_t(ok ? ih : 0) * a.W), 0, ok ? a.W * 4 : 0, BUF_DWORD3);
#pragma unroll
        for (int q = 0; q < 4; ++q) af[s][q] = __builtin_amdgcn_raw_buffer_load_b32(row, cofs[q], 0, 0);
      } else {
        // lane halves read different kernel rows 2s and 2s+1
        const int ih = cr * a.SH - a.PH + (2 * s + (lane >> 5)) * a.DH;
        const bool ok = unsigned(ih) < unsigned(a.H);
        const int32_t* rp = ximg + int64_t(ok ? ih : 0) * a.W;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int v = rp[min(max(cofs[q] / 4, 0), a.W - 1)];
          af[s][q] = ok && unsigned(cofs[q] / 4) < unsigned(a.W) ? v : 0;
        }
      }
    }
  };

  // Columns outside the convolution output read as INT_MIN (max's identity):
  // the slots of columns -4..-1 and OW4..127 (OW4 = OW rounded down to a
  // multiple of 4) are set once here and never staged into; a last group
  // of 1..3 real columns is staged with its tail masked.
  const int ow4 = a.OW & ~3;
  for (int i = threadIdx.x; i < 2 * 64 * CRW; i += 256) {
    const int slot = i % CRW;
    if (slot < COL_OFF || slot >= COL_OFF + ow4) crow[i / (64 * CRW)][i % (64 * CRW)] = INT_MIN;
  }

  // Convolution row cr -> h[j]: this lane's channel, max over the window
  // columns of pooled column 16*wave + j.  The A fragments of row cr are in
  // afrag on entry; those of row `next` are on their way on return.
  v4i afrag[KSUB];
  auto conv_row = [&](int cr, int next, int (&h)[16]) {
    int32_t* buf = crow[cr & 1];
    {
      v16i acc[2];
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[j][r] = 0;
#pragma unroll
      for (int s = 0; s < KSUB; ++s)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(afrag[s], bw[s][j], acc[j], 0, 0, 0);
      load_row(next, afrag);   // in flight during the staging and pooling of this row
      // stage as [channel][column]: the lane's 4 consecutive rows (columns) per group
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int col = wave * 32 + 8 * g + 4 * (lane >> 5);
          v4i v = {acc[j][4 * g], acc[j][4 * g + 1], acc[j][4 * g + 2], acc[j][4 * g + 3]};
          int32_t* dst = buf + (j * 32 + (lane & 31)) * CRW + COL_OFF + col;
          if (col < ow4) {
            *reinterpret_cast<v4i*>(dst) = v;
          } else if (col < a.OW) {
#pragma unroll
            for (int b = 0; b < 4; ++b) dst[b] = col + b < a.OW ? v[b] : INT_MIN;
          }
        }
    }
    __syncthreads();   // the row is staged; the other buffer's readers (row cr-1) are done
    v4i rd[NRD];
    const int32_t* src = buf + ch * CRW + RD0 + wave * 16 * PS;
#pragma unroll
    for (int q = 0; q < NRD; ++q) rd[q] = *reinterpret_cast<const v4i*>(src + 4 * q);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      int m = INT_MIN;
#pragma unroll
      for (int t = 0; t < PK; ++t) {
        const int slot = REL + j * PS + t;                   // compile-time
        m = max(m, rd[slot >> 2][slot & 3]);
      }
      h[j] = m;
    }
  };

  // Finish pooled row p from its window maxima v[j]: epilogue on the pooled
  // accumulators, the pad value where the window covers padding, stores (the
  // 64 lanes of a wave write one pooled pixel's channels).  Windows reaching
  // into the left/right padding: bit j of pad_cols.  Stores go through buffer
  // resources spanning the npx finished pixels of the pooled row; lanes past
  // the channel count get an offset out of range, so the hardware drops them.
  const int npx = max(0, min(16, a.POW - wave * 16));   // pooled pixels this wave stores (0 past POW)
  uint32_t pad_cols = 0;
  for (int j = 0; j < 16; ++j) {
    const int left = (wave * 16 + j) * PS - PPL;
    if (left < 0 || left + PK > a.OW) pad_cols |= 1u << j;
  }
  const bool pad_inert = a.pad_value == -INFINITY;   // max with -inf changes nothing
  const uint32_t vf = ch < a.O ? uint32_t(ch) * 4u : 0x80000000u;
  const uint32_t vq = ch < a.O ? uint32_t(ch) : 0x80000000u;
  // With a finite scale and bias and no NaN bound (the usual case, checked once
  // for the whole wave) the epilogue values are never NaN, NumPy's
  // maximum/minimum reduce to one compare and select, and the int8 clamp to a
  // median.
  const bool nan_free = FIXED && !__any(!(fabs(scale) < INFINITY) || !(fabsf(colv) < INFINITY) || lo != lo ||
                                        hi != hi) && !(a.pad_value != a.pad_value);
  auto finish = [&](int p, const int (&v)[16]) {
    const int top = p * PS - PPL;
    const bool pad_rows = top < 0 || top + PK > a.OH;
    const int64_t row0 = (int64_t(img) * a.POH + p) * a.POW + wave * 16;
    const __amdgpu_buffer_rsrc_t rf = __builtin_amdgcn_make_buffer_rsrc(
        e.out_f32 + row0 * e.ldo, 0, e.out_f32 ? npx * int(e.ldo) * 4 : 0, BUF_DWORD3);
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
        e.out_i8 + row0 * e.ldq, 0, e.out_i8 ? npx * int(e.ldq) : 0, BUF_DWORD3);
    auto store = [&](int j, float y, int8_t q) {   // pixels j >= npx fall outside the resources
      if (e.out_f32) __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(y), rf, vf + uint32_t(j * e.ldo * 4), 0, 0);
      if (e.out_i8) __builtin_amdgcn_raw_buffer_store_b8(q, rq, vq + uint32_t(j * e.ldq), 0, 0);
    };
    if constexpr (EF >= EF_SPEC) {
      if (nan_free && pad_inert) {   // steps and outputs known at compile time: straight-line code
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          float y = dequant(v[j], scale);
          if constexpr ((EF & SF_COL) != 0) y = __fadd_rn(y, colv);
          if constexpr ((EF & SF_LO) != 0) y = y > lo ? y : lo;
          if constexpr ((EF & SF_HI) != 0) y = y < hi ? y : hi;
          if constexpr ((EF & SF_F32) != 0)
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(y), rf, vf + uint32_t(j * e.ldo * 4), 0, 0);
          if constexpr ((EF & SF_I8) != 0) {
            const float t = rintf(static_cast<float>(__dmul_rn(static_cast<double>(y), e.out_rxs)));
            __builtin_amdgcn_raw_buffer_store_b8(static_cast<int8_t>(static_cast<int>(__builtin_amdgcn_fmed3f(t, -127.0f, 127.0f))),
                                                 rq, vq + uint32_t(j * e.ldq), 0, 0);
          }
        }
        return;
      }
    }
    if (nan_free) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        float y = dequant(v[j], scale);
        if (e.f_col) y = __fadd_rn(y, colv);
        if (e.f_lo) y = y > lo ? y : lo;
        if (e.f_hi) y = y < hi ? y : hi;
        if (!pad_inert && (pad_rows || ((pad_cols >> j) & 1))) y = y > a.pad_value ? y : a.pad_value;
        const float t = rintf(static_cast<float>(__dmul_rn(static_cast<double>(y), e.out_rxs)));
        store(j, y, static_cast<int8_t>(static_cast<int>(__builtin_amdgcn_fmed3f(t, -127.0f, 127.0f))));
      }
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        float y = dequant(v[j], scale);
        if constexpr (FIXED) {
          if (e.f_col) y = __fadd_rn(y, colv);
          if (e.f_lo) y = np_maximum(y, lo);
          if (e.f_hi) y = np_minimum(y, hi);
        } else {
          y = epi_generic(e, y, row0 + j, chc);
        }
        if (!pad_inert) y = np_maximum(y, pad_rows || ((pad_cols >> j) & 1) ? a.pad_value : -INFINITY);
        store(j, y, quantize_rcp(y, e.out_rxs));
      }
    }
  };

  // Pooled row p takes convolution rows 2p-1 (PK == 3), 2p and 2p+1; the host
  // guarantees 2p - PPL < OH for every pooled row.  Rows are walked in order,
  // row 2p+1 carrying over into pooled row p+1.
  const int cr_first = max(2 * pr0 - PPL, 0);
  const int cr_last = min(2 * (pr_end - 1) + 1, a.OH - 1);
  int carry[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) carry[j] = INT_MIN;
  load_row(cr_first, afrag);
  if (PK == 3 && pr0 > 0) conv_row(2 * pr0 - 1, min(2 * pr0, cr_last), carry);
  for (int p = pr0; p < pr_end; ++p) {
    const int r0 = 2 * p, r1 = 2 * p + 1;
    int v[16], h[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = PK == 3 ? carry[j] : INT_MIN;
    if (r0 < a.OH) {
      conv_row(r0, min(r1, cr_last), h);
#pragma unroll
      for (int j = 0; j < 16; ++j) v[j] = max(v[j], h[j]);
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) carry[j] = INT_MIN;
    if (r1 < a.OH) {
      conv_row(r1, min(r1 + 1, cr_last), carry);
#pragma unroll
      for (int j = 0; j < 16; ++j) v[j] = max(v[j], carry[j]);
    }
    finish(p, v);
  }
}

template <int KS, int RBV, int PK>
static void launch_stem(dim3 grid, hipStream_t s, const StemArgs& a, const EpiDev& e) {
  if (spec_form(e) == SPEC_RELU_F32_I8)
    hipLaunchKernelGGL((stem_pool_kernel<KS, RBV, PK, EF_SPEC | SPEC_RELU_F32_I8>), grid, dim3(256), 0, s, a, e);
  else if (e.fixed)
    hipLaunchKernelGGL((stem_pool_kernel<KS, RBV, PK, EF_FIXED>), grid, dim3(256), 0, s, a, e);
  else
    hipLaunchKernelGGL((stem_pool_kernel<KS, RBV, PK, EF_GENERIC>), grid, dim3(256), 0, s, a, e);
}

template <int PK>
static bool launch_stem_pool(int ksub, bool rb2, dim3 grid, hipStream_t s, const StemArgs& a, const EpiDev& e) {
  if (rb2) {
    switch (ksub) {
      case 5: launch_stem<5, 2, PK>(grid, s, a, e); return true;
      case 6: launch_stem<6, 2, PK>(grid, s, a, e); return true;
      case 7: launch_stem<7, 2, PK>(grid, s, a, e); return true;
      case 8: launch_stem<8, 2, PK>(grid, s, a, e); return true;
      default: return false;
    }
  }
  switch (ksub) {
    case 1: launch_stem<1, 1, PK>(grid, s, a, e); return true;
    case 2: launch_stem<2, 1, PK>(grid, s, a, e); return true;
    default: return false;
  }
}

// The pool commutes with the epilogue only if every step is a non-decreasing
// function of the value with an operand that is the same across a window
// (a scalar or a per-channel vector).
static bool monotone_epilogue(const mr_epilogue* epi) {
  for (int i = 0; i < epi->n_steps; ++i) {
    const mr_epi_step& st = epi->steps[i];
    if (st.fn == MR_EPI_RELU) continue;
    if (st.mode != MR_BC_SCALAR && st.mode != MR_BC_COL) return false;
    switch (st.fn) {
      case MR_EPI_ADD: case MR_EPI_MAX: case MR_EPI_MIN: break;
      case MR_EPI_SUB: if (st.swapped) return false; break;
      default: return false;
    }
  }
  return true;
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
  const bool pool_3_2_1 = pool_size == 3 && pool_stride == 2 && pool_pad_left == 1 && pool_pad_top == 1;
  const bool pool_2_2_0 = pool_size == 2 && pool_stride == 2 && pool_pad_left == 0 && pool_pad_top == 0;
  if (!pool_3_2_1 && !pool_2_2_0) {
    mr::set_error("mr_qconv2d_maxpool: pool %dx%d/%d with top/left pad %d/%d has no kernel (3/2 pad 1 and 2/2 pad 0 "
                  "do)", pool_size, pool_size, pool_stride, pool_pad_top, pool_pad_left);
    return MR_EUNSUPPORTED;
  }
  MR_REQUIRE(epi != nullptr, "mr_qconv2d_maxpool: NULL epilogue");
  if (!mr::monotone_epilogue(epi)) {
    mr::set_error("mr_qconv2d_maxpool: the epilogue must be non-decreasing with scalar or per-channel operands "
                  "(add, sub, maximum, minimum, relu)");
    return MR_EUNSUPPORTED;
  }
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
  a.n_pad = static_cast<int32_t>(n_pad);
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
  a.ppt = pool_pad_top;
  a.POH = poh;
  a.POW = pow_;
  a.pad_value = pad_value;
  const int64_t bands = (poh + mr::BAND - 1) / mr::BAND;
  const int64_t blocks = int64_t(G.n) * bands;
  MR_REQUIRE(blocks < (int64_t(1) << 31), "mr_qconv2d_maxpool: too many images");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool rb2 = row_bytes == 32;   // kw 5..8 (else kw <= 4, 16 bytes per kernel row)
  const dim3 grid(static_cast<unsigned>(blocks));
  const int ksub = rb2 ? G.kh : (G.kh + 1) / 2;        // 32-byte K steps holding real kernel rows
  const bool launched = pool_3_2_1 ? mr::launch_stem_pool<3>(ksub, rb2, grid, s, a, e)
                                   : mr::launch_stem_pool<2>(ksub, rb2, grid, s, a, e);
  if (!launched) {
    mr::set_error("mr_qconv2d_maxpool: %dx%d kernels have no kernel here (kh 1-4 with kw <= 4, kh 5-8 with kw 5-8)",
                  G.kh, G.kw);
    return MR_EUNSUPPORTED;
  }
  MR_LAUNCH_CHECK("qconv2d_maxpool");
  return MR_OK;
}

}  // extern "C"
