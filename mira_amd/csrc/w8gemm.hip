// Weight-only int8 matmul for batches of rows (the int8 weight-only mode,
// mira/quantize.py:45-68): y[M,N] = x[M,K] (f32) @ W, where W is the
// dequantize constant W[k][n] = fl32(q[k][n] * scale[n]) (mira/ops.py:581-589,
// rounded on to f16 when the dequantize has dtype f16), then the epilogue
// (mira/ops.py:217-219).  The weight-streaming kernel of qgemv.hip reads the
// weights once per 8 rows; this one tiles the product on f32 MFMAs
// (v_mfma_f32_32x32x2_f32), so the weights cross HBM once per 128 rows.
//
// A workgroup owns a 128 x 128 tile and walks K in 64-element stages (one
// 64-byte step of the packed weights).  Each stage's x slice (128 rows x 256
// bytes of f32) and weight slice (128 rows x 64 int8) move global -> LDS by
// buffer loads straight into LDS, double buffered; rows past M, columns past
// n_pad and K past K carry an offset past the buffers' ranges and read zeros.
// Every weight byte is dequantized once per wave that reads it, exactly as the
// reference does, in the fragment that feeds the MFMA.
//
// MFMA K order.  Integer order does not matter for f32 either way: the sum
// runs in another order than NumPy's BLAS, so the result matches to f32
// rounding, not bit for bit.  Within a stage the lanes of half h (lane / 32)
// take K elements 32h .. 32h + 31, one per MFMA step, so each lane reads its
// x values as 16-byte runs and its weights as 16-byte runs.
//
// CONV: the same product as an implicit-GEMM convolution (the weight-only mode's f32
// conv2d over a dequantize weight, mira/ops.py:265-276): x is an NHWC f32 image with C
// channels per pixel (C % 4 == 0), row m of the product is output pixel (n, oh, ow), and
// K element k is (tap (kh, kw), channel c) with k = (kh * KW + kw) * c_pad + c, the
// packed weights' order.  Each lane's 16-byte run keeps its (kh, kw, c) and steps it 64
// elements per stage; taps outside the image and channels >= C read zeros.
//
// LDS layout.  x rows are 256 bytes (16 chunks of 16 bytes; chunk c of row r
// sits at position c ^ (r & 15)), weight rows 64 bytes (chunk c of row n at
// c ^ ((n >> 2) & 3)): 16 consecutive rows of one chunk land on 16 distinct
// 16-byte bank groups.
#include "mr_common.hpp"

namespace mr {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void w8_lds_void;

constexpr int W8T = 128;                        // tile rows and columns
constexpr int W8K = 64;                         // K elements per stage
constexpr int W8_A_BYTES = W8T * W8K * 4;       // f32 x slice: 32 KB
constexpr int W8_STAGE = W8_A_BYTES + W8T * W8K;   // + int8 weight slice: 8 KB
constexpr uint32_t W8_OOB = 0x80000000u;        // an offset past every buffer's range

struct W8GemmArgs {
  const float* x;
  const int8_t* b;        // packed weights [k_pad / 64][n_pad][64]
  const float* ws;        // per-column weight scales
  int32_t ldx, k_pad, n_pad, M, N, K, w16;
  int32_t tiles_m;
  uint32_t x_bytes, b_bytes;
  // CONV geometry (x NHWC with C channels per pixel; k = (kh * KW + kw) * c_pad + c)
  int32_t H, W, C, c_pad, OH, OW, KH, KW, SH, SW, PH, PW, DH, DW;
};

template <bool CONV>
__global__ void __launch_bounds__(256) w8gemm_f32_kernel(const W8GemmArgs g, const EpiDev e) {
  __shared__ __attribute__((aligned(1024))) int8_t lds[2 * W8_STAGE];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;       // 2 x 2 waves of 64 x 64
  const int half = lane >> 5, l32 = lane & 31;
  // column tiles outermost: consecutive workgroups share a weight slice in L2
  const int tile_n = blockIdx.x / g.tiles_m;
  const int tile_m = blockIdx.x - tile_n * g.tiles_m;
  const int m0 = tile_m * W8T, n0 = tile_n * W8T;

  const __amdgpu_buffer_rsrc_t rx =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(g.x), 0, g.x_bytes, BUF_DWORD3);
  const __amdgpu_buffer_rsrc_t rb =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(g.b), 0, g.b_bytes, BUF_DWORD3);

  // x loader: 32 DMAs of 1 KB (4 rows) per stage, 8 per wave; lane l of DMA o fills LDS
  // chunk position l % 16 of row 4o + l / 16, i.e. global chunk (l % 16) ^ (row & 15)
  uint32_t x_row[8];
  int32_t x_k[8];
  // CONV: the row's top-left input pixel and the run's tap and channel at the next stage
  int32_t cv_img[CONV ? 8 : 1], cv_ih[CONV ? 8 : 1], cv_iw[CONV ? 8 : 1];
  int32_t cv_kh[CONV ? 8 : 1], cv_kw[CONV ? 8 : 1], cv_c[CONV ? 8 : 1];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int o = wave * 8 + j;
    const int r = o * 4 + (lane >> 4);
    const int c = (lane & 15) ^ (r & 15);
    x_k[j] = c * 4;
    x_row[j] = m0 + r < g.M ? static_cast<uint32_t>((m0 + r) * g.ldx * 4) : W8_OOB;
    if constexpr (CONV) {
      const int m = min(m0 + r, g.M - 1);
      const int img = m / (g.OH * g.OW);
      const int rem = m - img * g.OH * g.OW;
      const int oh = rem / g.OW;
      cv_img[j] = m0 + r < g.M ? img : -1;
      cv_ih[j] = oh * g.SH - g.PH;
      cv_iw[j] = (rem - oh * g.OW) * g.SW - g.PW;
      // k = c * 4 at stage 0: tap and channel of that K element
      const int tap = (c * 4) / g.c_pad;
      cv_c[j] = c * 4 - tap * g.c_pad;
      cv_kh[j] = tap / g.KW;
      cv_kw[j] = tap - cv_kh[j] * g.KW;
    }
  }
  // weight loader: 8 DMAs of 1 KB (16 rows) per stage, 2 per wave
  uint32_t b_vo[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int o = wave * 2 + j;
    const int n = o * 16 + (lane >> 2);
    const int c = (lane & 3) ^ ((n >> 2) & 3);
    b_vo[j] = n0 + n < g.n_pad ? static_cast<uint32_t>((n0 + n) * 64 + c * 16) : W8_OOB;
  }
  auto issue = [&](int kt, int buf) __attribute__((always_inline)) {
    int8_t* As = lds + buf * W8_STAGE;
    const int k0 = kt * W8K;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      uint32_t off;
      if constexpr (CONV) {
        const int ih = cv_ih[j] + cv_kh[j] * g.DH, iw = cv_iw[j] + cv_kw[j] * g.DW;
        const bool ok = cv_img[j] >= 0 && cv_kh[j] < g.KH && cv_c[j] < g.C && unsigned(ih) < unsigned(g.H) &&
                        unsigned(iw) < unsigned(g.W);
        off = ok ? static_cast<uint32_t>((((cv_img[j] * g.H + ih) * g.W + iw) * g.C + cv_c[j]) * 4) : W8_OOB;
        // on to the next stage's element of this run: 64 channels later, across taps
        cv_c[j] += W8K;
        while (cv_c[j] >= g.c_pad) {
          cv_c[j] -= g.c_pad;
          if (++cv_kw[j] == g.KW) {
            cv_kw[j] = 0;
            ++cv_kh[j];
          }
        }
      } else {
        const int k = k0 + x_k[j];
        // K % 4 == 0 (checked on the host): a 16-byte chunk is all below K or all past it
        off = (k < g.K && x_row[j] != W8_OOB) ? x_row[j] + static_cast<uint32_t>(k * 4) : W8_OOB;
      }
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (w8_lds_void*)(As + (wave * 8 + j) * 1024), 16, off, 0, 0, 0);
    }
    const uint32_t soff = static_cast<uint32_t>(kt * g.n_pad * 64);
#pragma unroll
    for (int j = 0; j < 2; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (w8_lds_void*)(As + W8_A_BYTES + (wave * 2 + j) * 1024), 16,
                                               b_vo[j], soff, 0, 0);
  };

  // this lane's two weight columns and their scales
  float sc[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) sc[j] = g.ws[min(n0 + wn * 64 + j * 32 + l32, g.N - 1)];

  v16f acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  auto compute = [&](int buf) __attribute__((always_inline)) {
    const int8_t* As = lds + buf * W8_STAGE;
    const int8_t* Bs = As + W8_A_BYTES;
#pragma unroll
    for (int q16 = 0; q16 < 2; ++q16) {
      // 16 weights of each column: K elements 32h + 16q16 .. +15 (chunk 2h + q16 of the row)
      v4i braw[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int n = wn * 64 + j * 32 + l32;
        const int pos = (half * 2 + q16) ^ ((n >> 2) & 3);
        braw[j] = *reinterpret_cast<const v4i*>(Bs + n * 64 + pos * 16);
      }
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        // 4 x values of each row: K elements 32h + 16q16 + 4s4 .. +3
        v4f a[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int r = wm * 64 + i * 32 + l32;
          const int pos = (half * 8 + q16 * 4 + s4) ^ (r & 15);
          a[i] = *reinterpret_cast<const v4f*>(As + r * 256 + pos * 16);
        }
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          float w[2];
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const int byte = __builtin_amdgcn_sbfe(braw[j][s4], kk * 8, 8);   // sign-extended int8
            w[j] = __fmul_rn(static_cast<float>(byte), sc[j]);
            if (g.w16) w[j] = round_f16(w[j]);
          }
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][kk], w[j], acc[i][j], 0, 0, 0);
        }
      }
    }
  };

  const int KT = g.k_pad / W8K;
  issue(0, 0);
  __builtin_amdgcn_s_waitcnt(0);               // the first stage has landed
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    // the other buffer's stage was read before the last barrier
    if (kt + 1 < KT) issue(kt + 1, (kt + 1) & 1);
    compute(kt & 1);
    __builtin_amdgcn_s_waitcnt(0);             // the next stage has landed, this one is read
    __syncthreads();
  }

  // epilogue: lane holds column l32 and rows 8 * (r / 4) + 4 * half + r % 4 of each block
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = n0 + wn * 64 + j * 32 + l32;
      if (col >= g.N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
        if (row < g.M) epi_store(e, epi_steps(e, acc[i][j][r], row, col), row, col);
      }
    }
}

int w8gemm_launch(const float* x, int64_t ldx, const int8_t* b, const float* w_scale, int32_t w_f16, int64_t k_pad,
                  int64_t n_pad, int64_t M, int64_t N, int64_t K, const EpiDev& e, hipStream_t stream,
                  const mr_conv_geom* cg) {
  const int64_t x_elems = cg ? int64_t(cg->n) * cg->h * cg->w * cg->c : M * ldx;
  if (K % 4 != 0 || ldx % 4 != 0 || x_elems * 4 >= (int64_t(1) << 31) || k_pad * n_pad >= (int64_t(1) << 31))
    return MR_EUNSUPPORTED;
  W8GemmArgs g = {};
  g.x = x;
  g.b = b;
  g.ws = w_scale;
  g.ldx = static_cast<int32_t>(ldx);
  g.k_pad = static_cast<int32_t>(k_pad);
  g.n_pad = static_cast<int32_t>(n_pad);
  g.M = static_cast<int32_t>(M);
  g.N = static_cast<int32_t>(N);
  g.K = static_cast<int32_t>(K);
  g.w16 = w_f16;
  g.tiles_m = static_cast<int32_t>((M + W8T - 1) / W8T);
  g.x_bytes = static_cast<uint32_t>(x_elems * 4);
  if (cg) {
    g.H = cg->h; g.W = cg->w; g.C = cg->c; g.c_pad = cg->c_pad; g.OH = cg->oh; g.OW = cg->ow;
    g.KH = cg->kh; g.KW = cg->kw; g.SH = cg->sh; g.SW = cg->sw; g.PH = cg->ph; g.PW = cg->pw; g.DH = cg->dh; g.DW = cg->dw;
  }
  g.b_bytes = static_cast<uint32_t>(k_pad * n_pad);
  const int64_t tiles = int64_t(g.tiles_m) * ((N + W8T - 1) / W8T);
  MR_REQUIRE(tiles < (int64_t(1) << 31), "w8gemm: too many tiles");
  if (cg)
    hipLaunchKernelGGL(w8gemm_f32_kernel<true>, dim3(static_cast<unsigned>(tiles)), dim3(256), 0, stream, g, e);
  else
    hipLaunchKernelGGL(w8gemm_f32_kernel<false>, dim3(static_cast<unsigned>(tiles)), dim3(256), 0, stream, g, e);
  MR_LAUNCH_CHECK("w8gemm");
  return MR_OK;
}

}  // namespace mr

extern "C" int mr_w8_conv2d_f32(const float* x, const mr_conv_geom* cg, const int8_t* b, const float* w_scale,
                                int32_t w_f16, int64_t k_pad, int64_t n_pad, const mr_epilogue* epi, void* stream) {
  MR_REQUIRE(x && cg && b && w_scale, "mr_w8_conv2d_f32: NULL argument");
  const mr_conv_geom& G = *cg;
  MR_REQUIRE(G.n >= 0 && G.h > 0 && G.w > 0 && G.c > 0 && G.o > 0 && G.c % 4 == 0,
             "mr_w8_conv2d_f32: bad shape (the input's channel count must be a multiple of 4)");
  MR_REQUIRE(G.kh > 0 && G.kw > 0 && G.sh > 0 && G.sw > 0 && G.dh > 0 && G.dw > 0 && G.ph >= 0 && G.pw >= 0,
             "mr_w8_conv2d_f32: bad kernel/stride/padding/dilation");
  const int32_t oh = (G.h + 2 * G.ph - G.dh * (G.kh - 1) - 1) / G.sh + 1;
  const int32_t ow = (G.w + 2 * G.pw - G.dw * (G.kw - 1) - 1) / G.sw + 1;
  MR_REQUIRE(oh == G.oh && ow == G.ow && oh > 0 && ow > 0, "mr_w8_conv2d_f32: output %dx%d does not match (%dx%d)",
             G.oh, G.ow, oh, ow);
  MR_REQUIRE(G.c_pad >= G.c && G.c_pad % 4 == 0, "mr_w8_conv2d_f32: c_pad %d must be >= c and a multiple of 4",
             G.c_pad);
  MR_REQUIRE(k_pad >= int64_t(G.kh) * G.kw * G.c_pad && k_pad % 64 == 0,
             "mr_w8_conv2d_f32: k_pad %lld must cover kh*kw*c_pad and be a multiple of 64", (long long)k_pad);
  MR_REQUIRE(n_pad >= G.o && n_pad % 32 == 0, "mr_w8_conv2d_f32: n_pad %lld must be >= o and a multiple of 32",
             (long long)n_pad);
  MR_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(b) % 16 == 0,
             "mr_w8_conv2d_f32: operands must be 16-byte aligned");
  mr::EpiDev e;
  const int rc = mr::make_epi(epi, G.o, false, &e);
  if (rc != MR_OK) return rc;
  const int64_t M = int64_t(G.n) * oh * ow;
  if (M == 0) return MR_OK;
  MR_REQUIRE(M < (int64_t(1) << 31), "mr_w8_conv2d_f32: too many pixels");
  const int r = mr::w8gemm_launch(x, 0, b, w_scale, w_f16, k_pad, n_pad, M, G.o, k_pad, e,
                                  static_cast<hipStream_t>(stream), cg);
  if (r == MR_EUNSUPPORTED) mr::set_error("mr_w8_conv2d_f32: the input or the weights reach 2 GiB");
  return r;
}
