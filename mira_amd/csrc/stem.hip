// Fused stem: int8 implicit-GEMM convolution of a <= 4-channel NHWC input
// (mira/ops.py:630-634), its epilogue (mira/ops.py:192-199), a constant pad
// (mira/ops.py:461-470) and max pooling (mira/ops.py:293-296), for graphs such
// as ResNet's 7x7/2 stem followed by a 3x3/2 max pool.
//
// Unfused, the convolution writes its full-resolution result (822 MB of f32
// for ResNet-18 at batch 256) only for the pool to read it back.  Here the
// pool runs on the int32 accumulators and the epilogue only on the pooled
// values: for a fixed output channel the epilogue is a non-decreasing
// function of the accumulator (dequant by a positive scale, then products
// with positive constants, adds, subtractions of a constant, maximum/minimum
// with constants: the host only fuses such epilogues), so the maximum over a window commutes with it, and
// max(f(a1), .., f(ak)) == f(max(a1, .., ak)) bit for bit (the values are never
// NaN unless an epilogue operand is, in which case both sides are NaN).  The
// pad value joins a window through NumPy's maximum after the epilogue.
//
// The input is either the int8 NHWC image with 4 bytes per pixel (XIN_I8),
// read from global memory row by row, or the f32 NCHW image itself (XIN_F32,
// XIN_F16: quantized from its f16 rounding).  Then the workgroup first fills
// LDS with its band's input rows, quantized exactly as quantize_nchw_nhwc4
// does (mira/ops.py:602-603) into the same 4-byte pixel layout, padding taps
// included as zeros, and the convolution reads its taps from there: the
// separate quantize pass (a full int8 copy of the image written and read
// back) disappears, and so does the global-load latency of the main loop.
//
// A workgroup owns a band of pooled rows of one image (BAND of them, fewer when the
// batch is too small to give every CU a workgroup).  It walks the convolution
// rows their windows cover, one at a time; each of its 4 waves computes, as
// one 32-pixel MFMA block row (x 64 channels, weights in LDS), the 32
// convolution columns that its pooled columns' windows cover (for a 3-wide
// pool, 15 pooled columns from 32 columns: neighbouring waves overlap by two
// columns), so the waves never exchange data.  A lane holds 16 columns of
// one channel per channel block; it trades 8 of them with its partner lane
// (lane ^ 32) so that each half of the wave holds the consecutive columns of
// its 8 pooled columns, max-pools them in registers and folds them into the
// running maxima of the pooled rows whose windows contain the row.  A pooled
// row is finished (epilogue, f32 and int8 stores) when its last convolution
// row has been folded in.
#include "mr_common.hpp"

#include <algorithm>
#include <climits>
#include <type_traits>

namespace mr {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int BAND = 8;           // pooled rows per workgroup, at most
// f32-input kernels: input rows live in an LDS ring of STEM_RING rows; each
// convolution row fetches the rows the one STEM_PD rows later needs
constexpr int STEM_RING = 16;
constexpr int STEM_PD = 4;

// Source of every padding tap: loads are never predicated, their address is
// (a select before the load keeps all of a row's loads in flight at once).
__device__ __attribute__((aligned(64))) int32_t g_stem_zero[16];

enum { XIN_I8 = 0, XIN_F32 = 1, XIN_F16 = 2 };

struct StemArgs {
  const int8_t* x;     // NHWC int8, 4 bytes per pixel (XIN_I8)
  const float* xf;     // NCHW f32 with C channels (XIN_F32 / XIN_F16)
  double rxs;          // fl64(1 / x_scale) (XIN_F32 / XIN_F16)
  int32_t C, lds_w;    // input channels; LDS pixels per input row: (OW - 1) * SW + 8
  const int8_t* b;     // packed weights, K-step-major [k_pad / 64][n_pad >= 64][64]
  int32_t k_pad, n_pad;
  int32_t row_bytes;   // packed bytes per kernel row
  int32_t N, H, W, O, OH, OW, KH, KW, SH, SW, PH, PW, DH, DW;
  int32_t ppt, POH, POW;  // pool top pad, pooled size
  int32_t band;           // pooled rows per workgroup (1 .. BAND)
  float pad_value;
};

// KSUB: 32-byte K steps holding kernel rows; RB: 16-byte chunks per kernel
// row; PK: pool window (3: rows/columns 2p-1 .. 2p+1, pad 1; 2: 2p .. 2p+1,
// pad 0), stride 2.
template <int KSUB, int RB, int PK, int EF, int XIN>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) stem_pool_kernel(const StemArgs a,
                                                                                      const EpiDev e) {
  static_assert(XIN == XIN_I8 || RB == 2, "the f32 input path reads 8-tap kernel rows");
  constexpr int PS = 2;
  constexpr int PPL = PK == 3 ? 1 : 0;   // window columns/rows left of / above 2p
  constexpr int PPW = PK == 3 ? 15 : 16; // pooled columns per wave
  constexpr bool FIXED = EF != EF_GENERIC;

  __shared__ v4i bw_lds[KSUB][2][64];    // weights, one MFMA B fragment per (K step, channel block, lane)
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform: keeps per-wave values scalar
  const int half = lane >> 5;
  const int bands = (a.POH + a.band - 1) / a.band;
  const int img = blockIdx.x / bands;
  const int pr0 = (blockIdx.x - img * bands) * a.band;
  const int pr_end = min(pr0 + a.band, a.POH);
  // the convolution rows this band walks
  const int cr_first = max(2 * pr0 - PPL, 0);
  const int cr_last = min(2 * (pr_end - 1) + 1, a.OH - 1);

  // K step s of channel block j: lane holds row 32j + lane%32, K bytes 32s + 16*(lane/32) .. +16
  for (int i = threadIdx.x; i < KSUB * 2 * 64; i += 256) {
    const int s = i >> 7, j = (i >> 6) & 1, l = i & 63;
    bw_lds[s][j][l] = *reinterpret_cast<const v4i*>(a.b + (int64_t(s >> 1) * a.n_pad + j * 32 + (l & 31)) * 64 +
                                                    (s & 1) * 32 + (l >> 5) * 16);
  }

  // XIN_F32 / XIN_F16: the input rows the band's convolution rows read,
  // ih_first + r for r < rows, pass through a ring of STEM_RING rows in LDS as
  // int8 pixels (row r in slot r % STEM_RING); LDS pixel px of a row is input
  // column px - PW, so every tap of every lane lies inside the row and padding
  // taps read the zeros stored for them.  A load unit is 4 pixels (columns
  // 4g - lg .. 4g - lg + 3; lg: PW rounded up to a multiple of 4, so no unit
  // straddles column 0) of one channel plane of one row, read with one 16-byte
  // load through a buffer resource spanning that plane row: columns past the
  // row's end and rows outside the image (no records) read 0, which quantizes
  // to the 0 of the convolution's zero padding.  The SH * C * groups units of
  // SH consecutive rows (<= 512) are spread over the workgroup, two per
  // thread; each writes its plane's 4 bytes, so the ring is zeroed once and
  // channel bytes past C stay 0.  Loads and stores are issued without branches
  // (a store with nothing to write goes to a sink byte), so every load of a
  // batch is in flight at once.  One image is under 2 GiB (checked on the host).
  extern __shared__ int32_t xin[];
  __shared__ int32_t sink[64];
  const int ih_first = cr_first * a.SH - a.PH;
  const int rows = (cr_last - cr_first) * a.SH + a.KH;
  const int lg = (a.PW + 3) & ~3;
  const int groups = XIN != XIN_I8 ? (a.lds_w - a.PW + lg + 3) >> 2 : 64;   // <= 64 (host)
  const int units = a.SH * a.C * groups;
  int u_row[2], u_ch[2], u_col[2];
  bool u_on[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int u = threadIdx.x + 256 * q;
    u_on[q] = u < units;
    const int cg = u % (a.C * groups);
    u_row[q] = u / (a.C * groups);
    u_ch[q] = cg / groups;
    u_col[q] = 4 * (cg - u_ch[q] * groups) - lg;
  }
  // One buffer resource spanning the image (uniform: a resource that differs
  // between lanes would make the compiler loop over its distinct values, one
  // load at a time).  A unit outside the image (a row above or below it, a
  // group left of column 0, a plane past C) gets an offset out of range and
  // reads 0; the dwords of a group past column W - 1 read the next row (or 0
  // past the image) and are replaced by 0.
  const __amdgpu_buffer_rsrc_t xrsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(a.xf + int64_t(img) * a.C * a.H * a.W), 0, XIN != XIN_I8 ? a.C * a.H * a.W * 4 : 0,
      BUF_DWORD3);
  // rows r0 + u_row[q] (the SH rows from r0) of this thread's two units
  auto fetch = [&](int r0, float4 (&v)[2]) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int r = r0 + u_row[q];
      const int ih = ih_first + r;
      const bool ok = u_on[q] && r < rows && unsigned(ih) < unsigned(a.H) && u_col[q] >= 0;
      const int off = ok ? ((u_ch[q] * a.H + ih) * a.W + u_col[q]) * 4 : int(0x80000000u);
      v[q] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(xrsrc, off, 0, 0));
    }
  };
  auto commit = [&](int r0, bool active, const float4 (&v)[2]) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      int8_t* dst = reinterpret_cast<int8_t*>(xin + ((r0 + u_row[q]) & (STEM_RING - 1)) * a.lds_w);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float xv = j == 0 ? v[q].x : j == 1 ? v[q].y : j == 2 ? v[q].z : v[q].w;
        const float x = u_col[q] + j < a.W ? xv : 0.0f;
        const int8_t b = quantize_rcp(XIN == XIN_F16 ? round_f16(x) : x, a.rxs);
        const int px = u_col[q] + a.PW + j;
        *(active && u_on[q] && unsigned(px) < unsigned(a.lds_w)
              ? dst + 4 * px + u_ch[q]
              : reinterpret_cast<int8_t*>(sink) + (threadIdx.x & 63) * 4) = b;
      }
    }
  };
  if constexpr (XIN != XIN_I8) {
    for (int i = threadIdx.x; i < STEM_RING * a.lds_w; i += 256) xin[i] = 0;
    __syncthreads();
    // rows 0 .. STEM_RING - 1: everything the first STEM_PD + 1 convolution
    // rows read (SH * STEM_PD + KH <= STEM_RING, host): batches of SH rows,
    // 8 batches in flight at once (two rounds when SH == 1)
    constexpr int PR = 8;
    for (int k0 = 0; k0 * a.SH < STEM_RING; k0 += PR) {
      float4 v[PR][2];
#pragma unroll
      for (int k = 0; k < PR; ++k) fetch((k0 + k) * a.SH, v[k]);
#pragma unroll
      for (int k = 0; k < PR; ++k) commit((k0 + k) * a.SH, (k0 + k) * a.SH < STEM_RING, v[k]);
    }
  }

  // pool-phase role: channels lane%32 and 32 + lane%32, pooled columns
  // wave*PPW + 8*half + t (t < 8; the upper half of a PK == 3 wave has 7)
  int chc[2];
  double scale[2];
  float mulv[2], colv[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    chc[j] = min(j * 32 + (lane & 31), a.O - 1);
    scale[j] = e.scale[chc[j]];
    mulv[j] = FIXED && e.f_mul ? e.mul_ptr[chc[j]] : 1.0f;
    colv[j] = FIXED && e.f_col ? e.col_ptr[chc[j]] : 0.0f;
  }
  const float lo = FIXED && e.f_lo && e.lo_ptr ? e.lo_ptr[0] : 0.0f;
  const float hi = FIXED && e.f_hi ? e.hi_ptr[0] : 0.0f;

  // The wave's 32 convolution columns: cw0 .. cw0 + 31, cw0 = 2 * PPW * wave - PPL,
  // so its pooled columns' windows lie inside them (neighbouring waves overlap
  // by two columns for PK == 3).  Lane l is A row (column) cw0 + l % 32,
  // clamped to [0, OW): a column outside the output recomputes its nearest
  // output column, which every window that reaches past the edge also
  // covers (a window starts at 2p - PPL <= OW - 1 and is at most 3 wide), so
  // the maxima are those over the window's real columns.
  const int cw0 = 2 * PPW * wave - PPL;
  const int ow = min(max(cw0 + (lane & 31), 0), a.OW - 1);
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
  const int kw0 = RB == 2 ? 4 * half : 0;
  int cofs[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) cofs[q] = (iw0 + (kw0 + q) * a.DW) * 4;   // negative -> out of range
  const bool left_edge = cofs[0] < 0 || a.DW != 1;   // taps not one contiguous 16-byte run from the row
  auto load_row = [&](int cr, v4i (&af)[KSUB]) {
    if constexpr (XIN != XIN_I8) {
      // LDS pixel of the lane's first tap: (ow * SW - PW + kw0) + PW; SW and the
      // row length are even, so the 16 bytes are two 8-byte aligned halves
      const int r0 = (cr - cr_first) * a.SH;
#pragma unroll
      for (int s = 0; s < KSUB; ++s) {
        const int2* p2 = reinterpret_cast<const int2*>(xin + ((r0 + s) & (STEM_RING - 1)) * a.lds_w + ow * a.SW + kw0);
        const int2 lo = p2[0], hi = p2[1];
        af[s] = v4i{lo.x, lo.y, hi.x, hi.y};
      }
      return;
    }
#pragma unroll
    for (int s = 0; s < KSUB; ++s) {
      if constexpr (RB == 2) {
        const int ih = cr * a.SH - a.PH + s * a.DH;
        const bool ok = unsigned(ih) < unsigned(a.H);
        const __amdgpu_buffer_rsrc_t row = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<int32_t*>(ximg + int64_t(ok ? ih : 0) * a.W), 0, ok ? a.W * 4 : 0, BUF_DWORD3);
        // the 4 taps are 16 contiguous bytes: one load, range-checked per
        // dword (taps right of the image read 0); a lane whose first tap is
        // left of the image (negative offset: the whole load would read 0)
        // loads its taps one by one
        af[s] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(row, cofs[0], 0, 0));
        if (left_edge) {
#pragma unroll
          for (int q = 0; q < 4; ++q) af[s][q] = __builtin_amdgcn_raw_buffer_load_b32(row, cofs[q], 0, 0);
        }
      } else {
        // lane halves read different kernel rows 2s and 2s+1
        const int ih = cr * a.SH - a.PH + (2 * s + half) * a.DH;
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

  // Convolution row cr -> h[j][t]: channel 32j + lane%32, max over the window
  // columns of pooled column wave*PPW + 8*half + t.  The A fragments of rows
  // cr and cr + 1 are in afr[cr & 1] and afr[(cr + 1) & 1] on entry (two rows
  // in flight hide the input's latency); those of row cr + 2 replace row cr's.
  v4i afr[2][KSUB];
  __syncthreads();   // weights in LDS
  auto conv_row = [&](auto par, int cr, int (&h)[2][8]) {
    constexpr int P = decltype(par)::value;
    // XIN_F32 / XIN_F16: fetch the SH input rows that convolution row cr + STEM_PD
    // adds (in flight during this row's MFMAs and pooling), and read this
    // row's taps from the ring
    const int pf_row = (cr - cr_first + STEM_PD) * a.SH + a.KH - a.SH;
    v4i af[KSUB];
    float4 pbuf[2];
    if constexpr (XIN != XIN_I8) {
      fetch(pf_row, pbuf);
      load_row(cr, af);
    }
    v16i acc[2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][r] = 0;
#pragma unroll
    for (int s = 0; s < KSUB; ++s)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        acc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(XIN != XIN_I8 ? af[s] : afr[P][s], bw_lds[s][j][lane], acc[j],
                                                       0, 0, 0);
    if constexpr (XIN == XIN_I8) {
      if (cr + 2 <= cr_last) load_row(cr + 2, afr[P]);   // in flight during the next rows
    }
    // Register r of a lane holds column 8*(r/4) + 4*half + r%4: the lower
    // half has columns 0-3, 8-11, 16-19, 24-27, the upper 4-7, ..., 28-31.
    // v_permlane32_swap(X, Y) exchanges X's upper 32 lanes with Y's lower 32
    // lanes; applied to (r, 8 + r) for r < 8 it leaves both halves holding
    // their 16 consecutive columns (16*half + 0..15) in the same registers:
    // X'[0..3], Y'[0..3], X'[4..7], Y'[4..7].  The lower half's pools also
    // need column 16, its register 8 before the swap.
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      int w[17];
      w[16] = acc[j][8];
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const auto xy = __builtin_amdgcn_permlane32_swap(static_cast<unsigned>(acc[j][r]),
                                                         static_cast<unsigned>(acc[j][8 + r]), false, false);
        w[(r >> 2) * 8 + (r & 3)] = static_cast<int>(xy[0]);
        w[(r >> 2) * 8 + 4 + (r & 3)] = static_cast<int>(xy[1]);
      }
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        int m = max(w[2 * t], w[2 * t + 1]);
        if constexpr (PK == 3) m = max(m, w[2 * t + 2]);
        h[j][t] = m;
      }
    }
    if constexpr (XIN != XIN_I8) {
      // the fetched rows replace rows STEM_RING lower, which no convolution row
      // from cr on reads; the barrier makes them visible before row cr + 1 (and
      // keeps every wave within one row of the others); nothing is scheduled
      // across the fence, so the loads have the whole row to arrive
      __builtin_amdgcn_sched_barrier(0);
      commit(pf_row, true, pbuf);
      __syncthreads();
    }
  };

  // Finish pooled row p from its window maxima v[j][t]: epilogue on the pooled
  // accumulators, the pad value where the window covers padding, stores.
  // Stores go through buffer resources spanning the pooled row; elements
  // without a pooled column or a channel get an offset out of range, so the
  // hardware drops them.
  const bool pad_inert = a.pad_value == -INFINITY;   // max with -inf changes nothing
  uint32_t pad_cols = 0, col_ok = 0;
  for (int t = 0; t < 8; ++t) {
    const int pc = wave * PPW + 8 * half + t;
    const int left = pc * PS - PPL;
    if (left < 0 || left + PK > a.OW) pad_cols |= 1u << t;
    if (pc < a.POW && 8 * half + t < PPW) col_ok |= 1u << t;
  }
  // With a finite scale and bias and no NaN bound (the usual case, checked once
  // for the whole wave) the epilogue values are never NaN, NumPy's
  // maximum/minimum reduce to one compare and select, and the int8 clamp to a
  // median.
  const bool nan_free = FIXED && !__any(!(fabs(scale[0]) < INFINITY) || !(fabs(scale[1]) < INFINITY) ||
                                        !(fabsf(colv[0]) < INFINITY) || !(fabsf(colv[1]) < INFINITY) ||
                                        !(fabsf(mulv[0]) < INFINITY) || !(fabsf(mulv[1]) < INFINITY) ||
                                        lo != lo || hi != hi) && !(a.pad_value != a.pad_value);
  auto finish = [&](int p, const int (&v)[2][8]) {
    const int top = p * PS - PPL;
    const bool pad_rows = top < 0 || top + PK > a.OH;
    const int64_t row0 = (int64_t(img) * a.POH + p) * a.POW;
    // f32 results, or (an f16 graph's values stored as halves) 2-byte halves
    const int fb = e.out_h16 ? 2 : 4;
    const __amdgpu_buffer_rsrc_t rf = __builtin_amdgcn_make_buffer_rsrc(
        reinterpret_cast<char*>(e.out_f32) + row0 * e.ldo * fb, 0, e.out_f32 ? a.POW * int(e.ldo) * fb : 0,
        BUF_DWORD3);
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
        e.out_i8 + row0 * e.ldq, 0, e.out_i8 ? a.POW * int(e.ldq) : 0, BUF_DWORD3);
    auto store_f = [&](float y, __amdgpu_buffer_rsrc_t r, uint32_t of) __attribute__((always_inline)) {
      if (e.out_h16)
        __builtin_amdgcn_raw_buffer_store_b16(__half_as_ushort(__float2half_rn(y)), r, of, 0, 0);
      else
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(y), r, of, 0, 0);
    };
    auto offs = [&](int j, int t, uint32_t& of, uint32_t& oq) __attribute__((always_inline)) {
      const int ch = j * 32 + (lane & 31);
      const int pc = wave * PPW + 8 * half + t;
      const bool ok = ((col_ok >> t) & 1) && ch < a.O;
      of = ok ? uint32_t((pc * int(e.ldo) + ch) * fb) : 0x80000000u;
      oq = ok ? uint32_t(pc * int(e.ldq) + ch) : 0x80000000u;
    };
    if constexpr (EF >= EF_SPEC) {
      if (nan_free && pad_inert) {   // steps and outputs known at compile time: straight-line code
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int t = 0; t < 8; ++t) {
            uint32_t of, oq;
            offs(j, t, of, oq);
            float y = dequant(v[j][t], scale[j]);
            if constexpr ((EF & SF_COL) != 0) y = __fadd_rn(y, colv[j]);
            if constexpr ((EF & SF_LO) != 0) y = y > lo ? y : lo;
            if constexpr ((EF & SF_HI) != 0) y = y < hi ? y : hi;
            if constexpr ((EF & SF_F16) != 0) y = round_f16(y);
            if constexpr ((EF & SF_F32) != 0) store_f(y, rf, of);
            if constexpr ((EF & SF_I8) != 0) {
              const float tq = rintf(static_cast<float>(__dmul_rn(static_cast<double>(y), e.out_rxs)));
              __builtin_amdgcn_raw_buffer_store_b8(
                  static_cast<int8_t>(static_cast<int>(__builtin_amdgcn_fmed3f(tq, -127.0f, 127.0f))), rq, oq, 0, 0);
            }
          }
        return;
      }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        uint32_t of, oq;
        offs(j, t, of, oq);
        float y = dequant(v[j][t], scale[j]);
        const bool padded = pad_rows || ((pad_cols >> t) & 1);
        if (nan_free) {
          if (e.f_mul) y = __fmul_rn(y, mulv[j]);
          if (e.f_col) y = __fadd_rn(y, colv[j]);
          if (e.f_lo) y = y > lo ? y : lo;
          if (e.f_hi) y = y < hi ? y : hi;
          if (e.f16) y = round_f16(y);
          if (!pad_inert && padded) y = y > a.pad_value ? y : a.pad_value;
        } else {
          if constexpr (FIXED) {
            if (e.f_mul) y = __fmul_rn(y, mulv[j]);
            if (e.f_col) y = __fadd_rn(y, colv[j]);
            if (e.f_lo) y = np_maximum(y, lo);
            if (e.f_hi) y = np_minimum(y, hi);
          } else {
            const int pc = wave * PPW + 8 * half + t;
            y = epi_generic(e, y, row0 + min(pc, a.POW - 1), chc[j]);
          }
          if (e.f16) y = round_f16(y);
          if (!pad_inert) y = np_maximum(y, padded ? a.pad_value : -INFINITY);
        }
        if (e.out_f32) store_f(y, rf, of);
        if (e.out_i8) __builtin_amdgcn_raw_buffer_store_b8(quantize_rcp(y, e.out_rxs), rq, oq, 0, 0);
      }
  };

  // Pooled row p takes convolution rows 2p-1 (PK == 3), 2p and 2p+1; the host
  // guarantees 2p - PPL < OH for every pooled row.  Rows are walked in order,
  // row 2p+1 carrying over into pooled row p+1.
  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  int carry[2][8];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int t = 0; t < 8; ++t) carry[j][t] = INT_MIN;
  if constexpr (XIN == XIN_I8) {
    if (cr_first & 1) load_row(cr_first, afr[1]); else load_row(cr_first, afr[0]);
    if (cr_first + 1 <= cr_last) {
      if (cr_first & 1) load_row(cr_first + 1, afr[0]); else load_row(cr_first + 1, afr[1]);
    }
  }
  if (PK == 3 && pr0 > 0) conv_row(P1{}, 2 * pr0 - 1, carry);   // 2 * pr0 - 1 is odd
  for (int p = pr0; p < pr_end; ++p) {
    const int r0 = 2 * p, r1 = 2 * p + 1;
    int v[2][8], h[2][8];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int t = 0; t < 8; ++t) v[j][t] = PK == 3 ? carry[j][t] : INT_MIN;
    if (r0 < a.OH) {
      conv_row(P0{}, r0, h);
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int t = 0; t < 8; ++t) v[j][t] = max(v[j][t], h[j][t]);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int t = 0; t < 8; ++t) carry[j][t] = INT_MIN;
    if (r1 < a.OH) {
      conv_row(P1{}, r1, carry);
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int t = 0; t < 8; ++t) v[j][t] = max(v[j][t], carry[j][t]);
    }
    finish(p, v);
  }
}

template <int KS, int RBV, int PK, int XIN>
static void launch_stem(dim3 grid, size_t lds, hipStream_t s, const StemArgs& a, const EpiDev& e) {
  // the stem stores halves (out_h16) through a run-time branch of its own
  const int form = spec_form(e) & ~SF_H16O;
  if (form == SPEC_RELU_F32_I8)
    hipLaunchKernelGGL((stem_pool_kernel<KS, RBV, PK, EF_SPEC | SPEC_RELU_F32_I8, XIN>), grid, dim3(256), lds, s, a,
                       e);
  else if (form == (SPEC_RELU_F32_I8 | SF_F16))
    hipLaunchKernelGGL((stem_pool_kernel<KS, RBV, PK, EF_SPEC | SPEC_RELU_F32_I8 | SF_F16, XIN>), grid, dim3(256), lds,
                       s, a, e);
  else if (e.fixed)
    hipLaunchKernelGGL((stem_pool_kernel<KS, RBV, PK, EF_FIXED, XIN>), grid, dim3(256), lds, s, a, e);
  else
    hipLaunchKernelGGL((stem_pool_kernel<KS, RBV, PK, EF_GENERIC, XIN>), grid, dim3(256), lds, s, a, e);
}

template <int PK>
static bool launch_stem_pool(int ksub, bool rb2, dim3 grid, hipStream_t s, const StemArgs& a, const EpiDev& e) {
  if (rb2) {
    switch (ksub) {
      case 5: launch_stem<5, 2, PK, XIN_I8>(grid, 0, s, a, e); return true;
      case 6: launch_stem<6, 2, PK, XIN_I8>(grid, 0, s, a, e); return true;
      case 7: launch_stem<7, 2, PK, XIN_I8>(grid, 0, s, a, e); return true;
      case 8: launch_stem<8, 2, PK, XIN_I8>(grid, 0, s, a, e); return true;
      default: return false;
    }
  }
  switch (ksub) {
    case 1: launch_stem<1, 1, PK, XIN_I8>(grid, 0, s, a, e); return true;
    case 2: launch_stem<2, 1, PK, XIN_I8>(grid, 0, s, a, e); return true;
    default: return false;
  }
}

// The f32-input kernels: 8-tap kernel rows (kw 5..8), the 7-row ResNet-style stem.
template <int PK, int XIN>
static bool launch_stem_pool_f32in(int ksub, dim3 grid, size_t lds, hipStream_t s, const StemArgs& a,
                                   const EpiDev& e) {
  if (ksub != 7) return false;
  launch_stem<7, 2, PK, XIN>(grid, lds, s, a, e);
  return true;
}

// The pool commutes with the epilogue only if every step is a non-decreasing
// function of the value with an operand that is the same across a window
// (a scalar or a per-channel vector).  A mul step is non-decreasing only for a
// positive operand, which lives in device memory: the caller guarantees it.
static bool monotone_epilogue(const mr_epilogue* epi) {
  for (int i = 0; i < epi->n_steps; ++i) {
    const mr_epi_step& st = epi->steps[i];
    if (st.fn == MR_EPI_RELU) continue;
    if (st.mode != MR_BC_SCALAR && st.mode != MR_BC_COL) return false;
    switch (st.fn) {
      case MR_EPI_ADD: case MR_EPI_MUL: case MR_EPI_MAX: case MR_EPI_MIN: break;
      case MR_EPI_SUB: if (st.swapped) return false; break;
      default: return false;
    }
  }
  return true;
}

// Validates a fused-stem call and fills the kernel arguments; MR_OK or the error code.
static int stem_setup(const char* who, const mr_conv_geom* cg, const int8_t* b, int64_t k_pad, int64_t n_pad,
                      const mr_epilogue* epi, int32_t pool_size, int32_t pool_stride, int32_t pool_pad_top,
                      int32_t pool_pad_left, float pad_value, int32_t poh, int32_t pow_, StemArgs* out, EpiDev* e,
                      bool* pool3) {
  MR_REQUIRE(cg && b, "%s: NULL argument", who);
  const mr_conv_geom& G = *cg;
  MR_REQUIRE(G.n >= 0 && G.h > 0 && G.w > 0 && G.c > 0 && G.c <= 4 && G.c_pad == 4,
             "%s: input must hold <= 4 channels in the 4-byte pixel layout", who);
  MR_REQUIRE(G.o > 0 && G.o <= 64 && n_pad >= 64 && n_pad % 32 == 0, "%s: needs o <= 64 and weights packed to 64 rows",
             who);
  MR_REQUIRE(G.kh > 0 && G.kw > 0 && G.sh > 0 && G.sw > 0 && G.dh > 0 && G.dw > 0 && G.ph >= 0 && G.pw >= 0,
             "%s: bad kernel/stride/padding/dilation", who);
  const int32_t oh = (G.h + 2 * G.ph - G.dh * (G.kh - 1) - 1) / G.sh + 1;
  const int32_t ow = (G.w + 2 * G.pw - G.dw * (G.kw - 1) - 1) / G.sw + 1;
  MR_REQUIRE(oh == G.oh && ow == G.ow && oh > 0 && ow > 0 && ow <= 128,
             "%s: convolution output must match the geometry and be <= 128 wide", who);
  const int32_t row_bytes = 16 * ((G.kw + 3) / 4);
  MR_REQUIRE(row_bytes <= 32, "%s: kernels wider than 8 taps are not supported", who);
  MR_REQUIRE(k_pad >= G.kh * row_bytes && k_pad % 64 == 0 && k_pad <= 256,
             "%s: k_pad %lld must cover kh*row_bytes, be a multiple of 64 and <= 256", who, (long long)k_pad);
  MR_REQUIRE(pool_size > 0 && pool_stride > 0 && pool_pad_top >= 0 && pool_pad_left >= 0 &&
                 pool_pad_top < pool_size && pool_pad_left < pool_size,
             "%s: bad pool parameters", who);
  MR_REQUIRE(poh > 0 && pow_ > 0 && pow_ <= (pool_size == 3 ? 60 : 64) && (poh - 1) * pool_stride - pool_pad_top < oh &&
                 (pow_ - 1) * pool_stride - pool_pad_left < ow,
             "%s: pooled size %dx%d does not fit the %dx%d convolution output", who, poh, pow_, oh, ow);
  const bool pool_3_2_1 = pool_size == 3 && pool_stride == 2 && pool_pad_left == 1 && pool_pad_top == 1;
  const bool pool_2_2_0 = pool_size == 2 && pool_stride == 2 && pool_pad_left == 0 && pool_pad_top == 0;
  if (!pool_3_2_1 && !pool_2_2_0) {
    set_error("%s: pool %dx%d/%d with top/left pad %d/%d has no kernel (3/2 pad 1 and 2/2 pad 0 do)", who, pool_size,
              pool_size, pool_stride, pool_pad_top, pool_pad_left);
    return MR_EUNSUPPORTED;
  }
  MR_REQUIRE(epi != nullptr, "%s: NULL epilogue", who);
  if (!monotone_epilogue(epi)) {
    set_error("%s: the epilogue must be non-decreasing with scalar or per-channel operands (add, sub, positive mul, "
              "maximum, minimum, relu)", who);
    return MR_EUNSUPPORTED;
  }
  MR_REQUIRE(reinterpret_cast<uintptr_t>(b) % 16 == 0, "%s: misaligned weights", who);
  const int rc = make_epi(epi, G.o, true, e, true);
  if (rc != MR_OK) return rc;
  MR_REQUIRE(!epi->out_acc, "%s: no int32 accumulator output (the convolution is not stored)", who);
  StemArgs a = {};
  a.b = b;
  a.k_pad = static_cast<int32_t>(k_pad);
  a.n_pad = static_cast<int32_t>(n_pad);
  a.row_bytes = row_bytes;
  a.N = G.n;
  a.H = G.h;
  a.W = G.w;
  a.C = G.c;
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
  // BAND pooled rows per workgroup, or fewer where that leaves CUs without two
  // workgroups (ResNet-18 at batch 1: 56 workgroups of one pooled row, not 7 of 8)
  const int64_t cus = device_cu_count();
  a.band = static_cast<int32_t>(std::min<int64_t>(BAND, std::max<int64_t>(1, (int64_t(G.n) * poh + 2 * cus - 1) /
                                                                                   (2 * cus))));
  const int64_t bands = (poh + a.band - 1) / a.band;
  MR_REQUIRE(int64_t(G.n) * bands < (int64_t(1) << 31), "%s: too many images", who);
  *out = a;
  *pool3 = pool_3_2_1;
  return MR_OK;
}

}  // namespace mr

extern "C" {

int mr_qconv2d_maxpool(const int8_t* x, const mr_conv_geom* cg, const int8_t* b, int64_t k_pad, int64_t n_pad,
                       const mr_epilogue* epi, int32_t pool_size, int32_t pool_stride, int32_t pool_pad_top,
                       int32_t pool_pad_left, float pad_value, int32_t poh, int32_t pow_, void* stream) {
  MR_REQUIRE(x, "mr_qconv2d_maxpool: NULL argument");
  MR_REQUIRE(reinterpret_cast<uintptr_t>(x) % 4 == 0, "mr_qconv2d_maxpool: misaligned operands");
  mr::StemArgs a;
  mr::EpiDev e;
  bool pool3 = false;
  const int rc = mr::stem_setup("mr_qconv2d_maxpool", cg, b, k_pad, n_pad, epi, pool_size, pool_stride, pool_pad_top,
                                pool_pad_left, pad_value, poh, pow_, &a, &e, &pool3);
  if (rc != MR_OK) return rc;
  if (a.N == 0) return MR_OK;
  a.x = x;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool rb2 = a.row_bytes == 32;   // kw 5..8 (else kw <= 4, 16 bytes per kernel row)
  const dim3 grid(static_cast<unsigned>(int64_t(a.N) * ((poh + a.band - 1) / a.band)));
  const int ksub = rb2 ? a.KH : (a.KH + 1) / 2;        // 32-byte K steps holding real kernel rows
  const bool launched = pool3 ? mr::launch_stem_pool<3>(ksub, rb2, grid, s, a, e)
                              : mr::launch_stem_pool<2>(ksub, rb2, grid, s, a, e);
  if (!launched) {
    mr::set_error("mr_qconv2d_maxpool: %dx%d kernels have no kernel here (kh 1-4 with kw <= 4, kh 5-8 with kw 5-8)",
                  a.KH, a.KW);
    return MR_EUNSUPPORTED;
  }
  MR_LAUNCH_CHECK("qconv2d_maxpool");
  return MR_OK;
}

int mr_qconv2d_maxpool_f32in(const float* x, float x_scale, int32_t round_f16, const mr_conv_geom* cg,
                             const int8_t* b, int64_t k_pad, int64_t n_pad, const mr_epilogue* epi, int32_t pool_size,
                             int32_t pool_stride, int32_t pool_pad_top, int32_t pool_pad_left, float pad_value,
                             int32_t poh, int32_t pow_, void* stream) {
  MR_REQUIRE(x, "mr_qconv2d_maxpool_f32in: NULL argument");
  MR_REQUIRE(x_scale > 0.0f && x_scale < INFINITY, "mr_qconv2d_maxpool_f32in: x_scale must be positive and finite");
  mr::StemArgs a;
  mr::EpiDev e;
  bool pool3 = false;
  const int rc = mr::stem_setup("mr_qconv2d_maxpool_f32in", cg, b, k_pad, n_pad, epi, pool_size, pool_stride,
                                pool_pad_top, pool_pad_left, pad_value, poh, pow_, &a, &e, &pool3);
  if (rc != MR_OK) return rc;
  // one image's f32 planes are read through a buffer resource with 32-bit byte offsets
  MR_REQUIRE(int64_t(a.C) * a.H * a.W * 4 < (int64_t(1) << 31),
             "mr_qconv2d_maxpool_f32in: an f32 image of 2 GiB or more is not supported");
  if (a.KH != 7 || a.KW < 5 || a.DH != 1 || a.DW != 1 || a.SW % 2 != 0) {
    mr::set_error("mr_qconv2d_maxpool_f32in: needs a 7-row kernel of 5 to 8 taps, no dilation and an even column "
                  "stride (got %dx%d, stride %d, dilation %dx%d)", a.KH, a.KW, a.SW, a.DH, a.DW);
    return MR_EUNSUPPORTED;
  }
  // LDS: a ring of STEM_RING input rows of (OW - 1) * SW + 8 pixels (every tap
  // of the last column's lane: 8 taps from (OW - 1) * SW - PW), loaded as
  // 4-pixel column groups with at least 4 rows side by side; the ring holds the
  // rows of STEM_PD + 1 convolution rows
  a.lds_w = (a.OW - 1) * a.SW + 8;
  const int32_t lg = (a.PW + 3) & ~3;
  const int32_t groups = (a.lds_w - a.PW + lg + 3) >> 2;
  if (groups > 64 || a.SH * mr::STEM_PD + a.KH > mr::STEM_RING) {
    mr::set_error("mr_qconv2d_maxpool_f32in: needs at most 64 four-pixel column groups per input row "
                  "((ow - 1) * sw + 8 = %d pixels) and a row stride of at most 2 (got %d)", a.lds_w, a.SH);
    return MR_EUNSUPPORTED;
  }
  const size_t lds = size_t(mr::STEM_RING) * a.lds_w * 4;
  if (a.N == 0) return MR_OK;
  a.xf = x;
  a.rxs = 1.0 / static_cast<double>(x_scale);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(int64_t(a.N) * ((poh + a.band - 1) / a.band)));
  const int xin = round_f16 ? mr::XIN_F16 : mr::XIN_F32;
  if (pool3) {
    if (xin == mr::XIN_F16) mr::launch_stem_pool_f32in<3, mr::XIN_F16>(a.KH, grid, lds, s, a, e);
    else mr::launch_stem_pool_f32in<3, mr::XIN_F32>(a.KH, grid, lds, s, a, e);
  } else {
    if (xin == mr::XIN_F16) mr::launch_stem_pool_f32in<2, mr::XIN_F16>(a.KH, grid, lds, s, a, e);
    else mr::launch_stem_pool_f32in<2, mr::XIN_F32>(a.KH, grid, lds, s, a, e);
  }
  MR_LAUNCH_CHECK("qconv2d_maxpool_f32in");
  return MR_OK;
}

}  // extern "C"
