// Fused MobileNet-style expansion and depthwise convolution.  A 1x1 int8
// convolution (mira/ops.py:630-634: int32 sums, f64 dequant, then its epilogue:
// bias, ReLU6) whose f32 result only a 3x3 depthwise f32 convolution reads
// (mira/ops.py:265-276 with groups == C, then its own bias, ReLU6 and the int8
// quantize of the next 1x1 convolution's input, mira/ops.py:602-603).  The two
// launches move the expanded f32 tensor through HBM twice (6x the channels of
// the block's input, 1.2 GB for the first 112x112 block of MobileNetV2 at batch
// 128); here it never leaves the chip.
//
// A workgroup owns a T x T tile of the depthwise output of one image.  It loads
// the tile's input region ((T-1)*S + 3 pixels square, the halo included) of the
// int8 expansion input into LDS once, then walks 32-channel blocks of the
// expanded tensor: the 1x1 product of the region's pixels with the block's 32
// weight columns on v_mfma_i32_32x32x32_i8, the expansion epilogue on each
// accumulator in registers, the f32 values into LDS (+0 for region pixels
// outside the image, the depthwise zero padding), and the depthwise taps from
// there.  The halo pixels' expansion is recomputed by the neighbouring tiles,
// with the same instructions, so every value is the one the two launches make:
// bit-exact (the accumulation order of each depthwise output is the row-major
// tap order of dwconv3x3_kernel, a separate multiply and add per tap).
#include <algorithm>
#include <type_traits>

#include "mr_common.hpp"

namespace mr {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

struct ExpandDwArgs {
  const int8_t* x;      // expansion input, NHWC int8 rows of ldx bytes (K real channels)
  const int8_t* b;      // packed 1x1 weights [KP / 64][n_pad][64]
  const float* wdw;     // depthwise weights [3][3][C]
  int32_t ldx, n_pad;
  int32_t H, W, C, OH, OW;
  int32_t tiles_w, tiles;   // output tiles per tile row, per image
  int32_t total;            // tiles of the whole batch
  int32_t Hin, Win, SS;     // STEM: the 3x3 convolution's input size and stride
};

// S: depthwise stride; T: output tile edge; KP: k_pad of the 1x1 weights;
// DF32: the depthwise result is also stored as f32 (besides its int8 copy).
// STEM: the first convolution is instead a 3x3 one (padding 1, stride SS) over a
// 4-byte-per-pixel image (3 channels and a zero), its weights in the stem layout
// (kernel row ki in the 16-byte chunk ki: three 4-byte taps and a zero word), so
// the A row of a region pixel is its nine input pixels gathered into those chunks.
// F16: an f16 graph's pair: each expanded value and each depthwise result rounded to f16
// after its epilogue, as the two launches round them (the taps stay exact f32 products of
// f16 values, summed in f32).
// blockIdx.y: the 32-channel block, whose weights and column constants a
// workgroup loads once; it then walks tiles blockIdx.x, + gridDim.x, ..., loading
// the next tile's region into registers while it computes the current one.  The
// region bytes (read by the MFMAs) and the f32 tile (written after every wave's
// MFMAs are done) share the LDS.
// workgroups of this LDS footprint that fit on a CU (160 KB), at most 4: the waves per
// SIMD the register budget is set for
template <int S, int T, int KP>
constexpr int ed_occupancy() {
  constexpr int IR = (T - 1) * S + 3, P = IR * IR, A = (P + 31) / 32 * 32 * (KP + 16), E = (P + 31) / 32 * 32 * 144;
  constexpr int bytes = (A > E ? A : E) + 32 * (KP + 16);
  return 163840 / bytes >= 4 ? 4 : 163840 / bytes;
}

template <int S, int T, int KP, bool DF32, bool STEM, bool F16>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(ed_occupancy<S, T, KP>())))
expand_dw_kernel(const ExpandDwArgs a, const EpiDev ex, const EpiDev dw) {
  constexpr int IR = (T - 1) * S + 3;   // input region edge
  constexpr int P = IR * IR;            // region pixels
  constexpr int PB = (P + 31) / 32;     // 32-pixel MFMA row blocks
  constexpr int AST = KP + 16;          // LDS row strides: A and B in bytes, E in floats
  constexpr int EST = 36;
  constexpr int KC = KP / 16;           // 16-byte chunks per region pixel
  constexpr int NA = (P * KC + 255) / 256;
  constexpr int NB = (32 * KC + 255) / 256;
  constexpr int NSLOT = (T * T + 31) / 32;   // depthwise pixels per thread
  constexpr int RPW = (PB + 3) / 4;          // MFMA row blocks per wave
  constexpr int A_BYTES = PB * 32 * AST, E_BYTES = PB * 32 * EST * 4;   // E rows past P: written, unread
  constexpr int AE_BYTES = A_BYTES > E_BYTES ? A_BYTES : E_BYTES;
  __shared__ __attribute__((aligned(16))) int8_t smem[AE_BYTES + 32 * AST];
  __shared__ __attribute__((aligned(16))) float4 wl[10][8];   // depthwise taps and bias, 8 channel quads
  int8_t* const A = smem;
  float* const E = reinterpret_cast<float*>(smem);
  int8_t* const B = smem + AE_BYTES;

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int c_base = blockIdx.y * 32;

  // the region of tile `id` (zeros outside the image and past ldx) into registers
  v4i va[NA];
  auto load_region = [&](int id) __attribute__((always_inline)) {
    const int img = id / a.tiles, tile = id - img * a.tiles;
    const int th = tile / a.tiles_w;
    const int ih0 = th * T * S - 1, iw0 = (tile - th * a.tiles_w) * T * S - 1;
#pragma unroll
    for (int u = 0; u < NA; ++u) {
      const int i = t + u * 256;
      const int p = i / KC, kc = i - p * KC;
      const int ih = ih0 + p / IR, iw = iw0 + p % IR;
      va[u] = v4i{0, 0, 0, 0};
      if constexpr (STEM) {
        // kernel row kc of region pixel (ih, iw)'s 3x3 window: three 4-byte input pixels
        const int iy = ih * a.SS - 1 + kc, ix0 = iw * a.SS - 1;
        if (i < P * KC && kc < 3 && unsigned(iy) < unsigned(a.Hin)) {
          const int32_t* row = reinterpret_cast<const int32_t*>(a.x) + (int64_t(img) * a.Hin + iy) * a.Win;
#pragma unroll
          for (int j = 0; j < 3; ++j)
            if (unsigned(ix0 + j) < unsigned(a.Win)) va[u][j] = row[ix0 + j];
        }
      } else {
        if (i < P * KC && unsigned(ih) < unsigned(a.H) && unsigned(iw) < unsigned(a.W) && kc * 16 < a.ldx)
          va[u] = *reinterpret_cast<const v4i*>(a.x + ((int64_t(img) * a.H + ih) * a.W + iw) * a.ldx + kc * 16);
      }
    }
  };
  int id = blockIdx.x;
  load_region(id);

  // this workgroup's 32 weight columns (64-byte K steps of 32 adjacent packed rows) and
  // the column constants: the expansion's for the lane's column, the depthwise ones for
  // the thread's channel quad
  {
    v4i vb[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int i = t + u * 256;
      const int ks = i >> 7, col = (i >> 2) & 31, part = i & 3;
      if (i < 32 * KC)
        vb[u] = *reinterpret_cast<const v4i*>(a.b + (int64_t(ks) * a.n_pad + c_base + col) * 64 + part * 16);
    }
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int i = t + u * 256;
      const int ks = i >> 7, col = (i >> 2) & 31, part = i & 3;
      if (i < 32 * KC) *reinterpret_cast<v4i*>(B + col * AST + ks * 64 + part * 16) = vb[u];
    }
  }
  const int ecol = min(c_base + (lane & 31), a.C - 1);
  const double escale = ex.scale[ecol];
  const float ebias = ex.col_ptr[ecol];
  const int q = t & 7;
  const int cq = c_base + 4 * q;
  const bool qok = cq < a.C;
  if (t < 80) {   // the block's depthwise taps [9][8 quads] and bias [8 quads] into LDS
    const int k = t >> 3, c4 = c_base + 4 * (t & 7);
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (c4 < a.C) v = *reinterpret_cast<const float4*>(k < 9 ? a.wdw + k * a.C + c4 : dw.col_ptr + c4);
    wl[k][t & 7] = v;
  }
  const float ex_lo = ex.lo_ptr ? ex.lo_ptr[0] : 0.0f, ex_hi = ex.hi_ptr[0];
  const float dw_lo = dw.lo_ptr ? dw.lo_ptr[0] : 0.0f, dw_hi = dw.hi_ptr[0];
  const bool ex_lo_nan = ex_lo != ex_lo, ex_hi_nan = ex_hi != ex_hi;
  const bool dw_lo_nan = dw_lo != dw_lo, dw_hi_nan = dw_hi != dw_hi;
  auto expand = [&](int32_t v) __attribute__((always_inline)) {
    float y = dequant(v, escale);
    y = __fadd_rn(y, ebias);
    y = max_bound(y, ex_lo, ex_lo_nan);
    y = min_bound(y, ex_hi, ex_hi_nan);
    return F16 ? round_f16(y) : y;
  };
  // With a finite bias and bounds lo <= hi the expanded value is never NaN, and the two
  // bounds are one median (v_med3_f32): equal to them up to the sign of a zero result, which
  // the depthwise sums cannot see (they start from +0, and +0 + -0 = +0 in round to
  // nearest).  Taken when every lane of the wave qualifies.
  const bool ex_med3 = __all(isfinite(ebias) && !ex_lo_nan && !ex_hi_nan && ex_lo <= ex_hi);
  auto expand_med3 = [&](int32_t v) __attribute__((always_inline)) {
    const float y = __builtin_amdgcn_fmed3f(__fadd_rn(dequant(v, escale), ebias), ex_lo, ex_hi);
    return F16 ? round_f16(y) : y;
  };

  for (; id < a.total; id += gridDim.x) {
    const int img = id / a.tiles, tile = id - img * a.tiles;
    const int th = tile / a.tiles_w;
    const int oh0 = th * T, ow0 = (tile - th * a.tiles_w) * T;
    const int ih0 = oh0 * S - 1, iw0 = ow0 * S - 1;   // padding 1
    // a region wholly inside the image needs no per-pixel bounds (most tiles)
    const bool interior = ih0 >= 0 && iw0 >= 0 && ih0 + IR <= a.H && iw0 + IR <= a.W;

    block_barrier();   // the last tile's E reads are done: A may overwrite them
#pragma unroll
    for (int u = 0; u < NA; ++u) {
      const int i = t + u * 256;
      const int p = i / KC, kc = i - p * KC;
      if (i < P * KC) *reinterpret_cast<v4i*>(A + p * AST + kc * 16) = va[u];
    }
    lds_store_barrier();   // A (and, the first time, B) written
    if (id + int(gridDim.x) < a.total) load_region(id + gridDim.x);   // in flight during this tile

    // the 1x1 product on the region's row blocks (a wave takes blocks wave, wave + 4, ...)
    v16i acc[RPW];
#pragma unroll
    for (int j = 0; j < RPW; ++j) {
      const int rb = wave + 4 * j;
      acc[j] = v16i{};
      if (rb >= PB) continue;
#pragma unroll
      for (int kk = 0; kk < KP / 32; ++kk) {
        const v4i av = *reinterpret_cast<const v4i*>(A + (rb * 32 + (lane & 31)) * AST + kk * 32 + (lane >> 5) * 16);
        const v4i bv = *reinterpret_cast<const v4i*>(B + (lane & 31) * AST + kk * 32 + (lane >> 5) * 16);
        acc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv, acc[j], 0, 0, 0);
      }
    }
    block_barrier();   // every wave's A reads are done: E may overwrite them

    // the expansion epilogue (lane: column lane % 32, rows 8 (r / 4) + 4 (lane / 32) + r % 4
    // of each block) into E, every row of the blocks (region pixels outside the image are
    // zeroed afterwards)
    if (ex_med3) {
#pragma unroll
      for (int j = 0; j < RPW; ++j) {
        const int rb = wave + 4 * j;
        if (rb >= PB) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r)
          E[(rb * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * EST + (lane & 31)] = expand_med3(acc[j][r]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < RPW; ++j) {
        const int rb = wave + 4 * j;
        if (rb >= PB) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r)
          E[(rb * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * EST + (lane & 31)] = expand(acc[j][r]);
      }
    }
    lds_store_barrier();   // E written
    if (!interior) {
      // the depthwise zero padding: region pixels outside the image read as +0 (a tile at the
      // image's edge; the same for the whole workgroup)
#pragma unroll 1
      for (int p = t >> 3; p < P; p += 32) {
        const int pr = p / IR;
        if (unsigned(ih0 + pr) >= unsigned(a.H) || unsigned(iw0 + p - pr * IR) >= unsigned(a.W))
          *reinterpret_cast<float4*>(E + p * EST + 4 * q) = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
      lds_store_barrier();
    }

    // the depthwise taps: quad q of output pixels t / 8, t / 8 + 32, ...
    if (qok) {
      float4 w9[9];
#pragma unroll
      for (int k = 0; k < 9; ++k) w9[k] = wl[k][q];
      const float4 dbias = wl[9][q];
      // int8 only, finite biases and bounds lo <= hi: the sums are finite, so the bounds are
      // one median, exact up to the sign of a zero, which quantizes to the same byte
      const bool dw_med3 = !DF32 && __all(isfinite(dbias.x) && isfinite(dbias.y) && isfinite(dbias.z) &&
                                          isfinite(dbias.w) && !dw_lo_nan && !dw_hi_nan && dw_lo <= dw_hi);
      auto slots = [&](auto med3) __attribute__((always_inline)) {
#pragma unroll 1
        for (int sl = 0; sl < NSLOT; ++sl) {
          const int pi = (t >> 3) + sl * 32;
          if (pi >= T * T) break;
          const int oy = pi / T, ox = pi - oy * T;
          const int oh = oh0 + oy, ow = ow0 + ox;
          if (oh >= a.OH || ow >= a.OW) continue;
          float acc4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int ki = 0; ki < 3; ++ki)
#pragma unroll
            for (int kj = 0; kj < 3; ++kj) {
              const float4 xv = *reinterpret_cast<const float4*>(E + ((oy * S + ki) * IR + ox * S + kj) * EST + 4 * q);
              const float4 w = w9[ki * 3 + kj];
              acc4[0] = __fadd_rn(acc4[0], __fmul_rn(xv.x, w.x));
              acc4[1] = __fadd_rn(acc4[1], __fmul_rn(xv.y, w.y));
              acc4[2] = __fadd_rn(acc4[2], __fmul_rn(xv.z, w.z));
              acc4[3] = __fadd_rn(acc4[3], __fmul_rn(xv.w, w.w));
            }
          const float bias[4] = {dbias.x, dbias.y, dbias.z, dbias.w};
          float y[4];
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const float v = __fadd_rn(acc4[c], bias[c]);
            if constexpr (decltype(med3)::value)
              y[c] = __builtin_amdgcn_fmed3f(v, dw_lo, dw_hi);
            else
              y[c] = min_bound(max_bound(v, dw_lo, dw_lo_nan), dw_hi, dw_hi_nan);
            if constexpr (F16) y[c] = round_f16(y[c]);
          }
          const int64_t pix = (int64_t(img) * a.OH + oh) * a.OW + ow;
          if constexpr (DF32)
            *reinterpret_cast<float4*>(dw.out_f32 + pix * dw.ldo + cq) = make_float4(y[0], y[1], y[2], y[3]);
          uint32_t packed = 0;
#pragma unroll
          for (int c = 0; c < 4; ++c) packed |= uint32_t(uint8_t(quantize_rcp(y[c], dw.out_rxs))) << (8 * c);
          *reinterpret_cast<uint32_t*>(dw.out_i8 + pix * dw.ldq + cq) = packed;
        }
      };
      if (dw_med3)
        slots(std::true_type{});
      else
        slots(std::false_type{});
    }
  }
}

template <int S, int T, int KP, bool STEM = false>
static void expand_dw_launch(const ExpandDwArgs& a, const EpiDev& ex, const EpiDev& dw, dim3 grid,
                             hipStream_t stream) {
  if (dw.f16) {
    if (dw.out_f32)
      hipLaunchKernelGGL((expand_dw_kernel<S, T, KP, true, STEM, true>), grid, dim3(256), 0, stream, a, ex, dw);
    else
      hipLaunchKernelGGL((expand_dw_kernel<S, T, KP, false, STEM, true>), grid, dim3(256), 0, stream, a, ex, dw);
  } else {
    if (dw.out_f32)
      hipLaunchKernelGGL((expand_dw_kernel<S, T, KP, true, STEM, false>), grid, dim3(256), 0, stream, a, ex, dw);
    else
      hipLaunchKernelGGL((expand_dw_kernel<S, T, KP, false, STEM, false>), grid, dim3(256), 0, stream, a, ex, dw);
  }
}

template <int S, int T>
static int expand_dw_kp(int64_t k_pad, const ExpandDwArgs& a, const EpiDev& ex, const EpiDev& dw, dim3 grid,
                        hipStream_t stream) {
  if (k_pad == 64) expand_dw_launch<S, T, 64>(a, ex, dw, grid, stream);
  else if (k_pad == 128) expand_dw_launch<S, T, 128>(a, ex, dw, grid, stream);
  else expand_dw_launch<S, T, 192>(a, ex, dw, grid, stream);
  return MR_OK;
}

static bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

// bias (per column) -> maximum -> minimum, nothing else
static bool relu6_form(const EpiDev& e) {
  return e.fixed && !e.f_mul && e.f_col && !e.f_full && e.f_lo && e.f_hi && !e.out_acc;
}

// Checks and launch shared by both entry points: the depthwise geometry, both epilogues,
// the launch (stem: the first convolution's 3x3 geometry, else the 1x1 expansion's).
static int expand_dw_run(const char* fn, const int8_t* x, int64_t ldx, const int8_t* b, int64_t k_pad,
                         int64_t n_pad, const mr_epilogue* epi_expand, const mr_conv_geom* dwg, const float* w_dw,
                         const mr_epilogue* epi_dw, void* stream, const mr_conv_geom* stem) {
  MR_REQUIRE(x && b && epi_expand && dwg && w_dw && epi_dw, "%s: NULL argument", fn);
  const mr_conv_geom& G = *dwg;
  MR_REQUIRE(G.n >= 0 && G.h > 0 && G.w > 0 && G.c > 0 && G.o == G.c && G.c_pad == G.c,
             "%s: bad depthwise geometry (o == c == c_pad)", fn);
  MR_REQUIRE(G.kh == 3 && G.kw == 3 && G.dh == 1 && G.dw == 1 && G.ph == 1 && G.pw == 1 && G.sh == G.sw &&
                 (G.sh == 1 || G.sh == 2),
             "%s: the depthwise convolution must be 3x3, padding 1, stride 1 or 2", fn);
  const int32_t oh = (G.h + 2 - 3) / G.sh + 1, ow = (G.w + 2 - 3) / G.sw + 1;
  MR_REQUIRE(oh == G.oh && ow == G.ow, "%s: output %dx%d does not match (%dx%d)", fn, G.oh, G.ow, oh, ow);
  MR_REQUIRE(G.c % 4 == 0, "%s: channel count %d must be a multiple of 4", fn, G.c);
  MR_REQUIRE(n_pad >= G.c && n_pad % 32 == 0, "%s: n_pad %lld must be >= c and a multiple of 32", fn,
             (long long)n_pad);
  MR_REQUIRE(aligned16(x) && aligned16(b) && aligned16(w_dw), "%s: x, b and w_dw must be 16-byte aligned", fn);
  MR_REQUIRE(!epi_expand->out_f32 && !epi_expand->out_i8 && !epi_expand->out_acc,
             "%s: the first convolution's result is not stored (its epilogue has no outputs)", fn);
  MR_REQUIRE(epi_dw->out_i8 != nullptr, "%s: the depthwise result needs its int8 copy", fn);
  EpiDev ex, dw;
  int rc = make_epi(epi_expand, G.c, true, &ex, false, false);
  if (rc != MR_OK) return rc;
  rc = make_epi(epi_dw, G.c, false, &dw);
  if (rc != MR_OK) return rc;
  if (k_pad > 192 || !relu6_form(ex) || !relu6_form(dw) || ex.f16 != dw.f16) {
    set_error("%s: compiled for k_pad <= 192 and bias -> maximum -> minimum epilogues on both convolutions, "
              "both with or both without f16 rounding", fn);
    return MR_EUNSUPPORTED;
  }
  MR_REQUIRE(dw.ldq % 4 == 0 && reinterpret_cast<uintptr_t>(dw.out_i8) % 4 == 0 &&
                 (!dw.out_f32 || (dw.ldo % 4 == 0 && aligned16(dw.out_f32))) && aligned16(dw.col_ptr),
             "%s: depthwise outputs and bias must be aligned for 4-channel runs", fn);
  if (G.n == 0) return MR_OK;
  const int T = G.sh == 1 && oh >= 14 ? 14 : 7;
  ExpandDwArgs a = {};
  a.x = x;
  a.b = b;
  a.wdw = w_dw;
  a.ldx = static_cast<int32_t>(ldx);
  a.n_pad = static_cast<int32_t>(n_pad);
  a.H = G.h; a.W = G.w; a.C = G.c; a.OH = oh; a.OW = ow;
  if (stem) {
    a.Hin = stem->h; a.Win = stem->w; a.SS = stem->sh;
  }
  a.tiles_w = (ow + T - 1) / T;
  a.tiles = a.tiles_w * ((oh + T - 1) / T);
  const int n_cb = (G.c + 31) / 32;
  const int64_t total = int64_t(G.n) * a.tiles;
  MR_REQUIRE(total < (int64_t(1) << 31), "%s: too many tiles", fn);
  a.total = static_cast<int32_t>(total);
  // workgroups per channel block: about eight per CU over all blocks, each walking its
  // share of the tiles
  const int64_t per_cb = std::max<int64_t>(1, std::min<int64_t>(total, (8 * device_cu_count() + n_cb - 1) / n_cb));
  const dim3 grid(static_cast<unsigned>(per_cb), static_cast<unsigned>(n_cb));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (stem) {
    if (G.sh == 2) expand_dw_launch<2, 7, 64, true>(a, ex, dw, grid, s);
    else if (T == 14) expand_dw_launch<1, 14, 64, true>(a, ex, dw, grid, s);
    else expand_dw_launch<1, 7, 64, true>(a, ex, dw, grid, s);
  } else {
    if (G.sh == 2) expand_dw_kp<2, 7>(k_pad, a, ex, dw, grid, s);
    else if (T == 14) expand_dw_kp<1, 14>(k_pad, a, ex, dw, grid, s);
    else expand_dw_kp<1, 7>(k_pad, a, ex, dw, grid, s);
  }
  MR_LAUNCH_CHECK(fn);
  return MR_OK;
}

}  // namespace mr

extern "C" int mr_qconv1x1_dw3x3(const int8_t* x, int64_t ldx, const int8_t* b, int64_t k_pad, int64_t n_pad,
                                 int64_t K, const mr_epilogue* epi_expand, const mr_conv_geom* dwg,
                                 const float* w_dw, const mr_epilogue* epi_dw, void* stream) {
  MR_REQUIRE(K > 0 && ldx >= K && ldx % 16 == 0, "mr_qconv1x1_dw3x3: ldx %lld must be >= K and a multiple of 16",
             (long long)ldx);
  MR_REQUIRE(k_pad >= K && k_pad % 64 == 0, "mr_qconv1x1_dw3x3: k_pad %lld must be >= K and a multiple of 64",
             (long long)k_pad);
  return mr::expand_dw_run("mr_qconv1x1_dw3x3", x, ldx, b, k_pad, n_pad, epi_expand, dwg, w_dw, epi_dw, stream,
                           nullptr);
}

extern "C" int mr_qstem3x3_dw3x3(const int8_t* x, const mr_conv_geom* stem, const int8_t* b, int64_t k_pad,
                                 int64_t n_pad, const mr_epilogue* epi_stem, const mr_conv_geom* dwg,
                                 const float* w_dw, const mr_epilogue* epi_dw, void* stream) {
  MR_REQUIRE(stem && dwg, "mr_qstem3x3_dw3x3: NULL geometry");
  const mr_conv_geom& g = *stem;
  MR_REQUIRE(g.kh == 3 && g.kw == 3 && g.c > 0 && g.c <= 4 && g.c_pad == 4 && g.ph == 1 && g.pw == 1 &&
                 g.dh == 1 && g.dw == 1 && g.sh == g.sw && (g.sh == 1 || g.sh == 2),
             "mr_qstem3x3_dw3x3: the first convolution must be 3x3, padding 1, stride 1 or 2, over at most 4 "
             "channels stored 4 per pixel");
  MR_REQUIRE(g.h > 0 && g.w > 0 && g.oh == (g.h - 1) / g.sh + 1 && g.ow == (g.w - 1) / g.sw + 1,
             "mr_qstem3x3_dw3x3: output %dx%d does not match the input %dx%d", g.oh, g.ow, g.h, g.w);
  MR_REQUIRE(g.n == dwg->n && g.o == dwg->c && g.oh == dwg->h && g.ow == dwg->w,
             "mr_qstem3x3_dw3x3: the depthwise input must be the first convolution's output");
  MR_REQUIRE(k_pad == 64, "mr_qstem3x3_dw3x3: the stem-layout weights have k_pad 64, not %lld", (long long)k_pad);
  MR_REQUIRE(int64_t(g.n) * g.h * g.w < (int64_t(1) << 31), "mr_qstem3x3_dw3x3: image too large");
  return mr::expand_dw_run("mr_qstem3x3_dw3x3", x, 4, b, k_pad, n_pad, epi_stem, dwg, w_dw, epi_dw, stream, stem);
}
