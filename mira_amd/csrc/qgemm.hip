// K2/K2c + K3: int8 x int8 -> int32 contraction on gfx950 MFMA
// (v_mfma_i32_32x32x32_i8) with the dequant / epilogue / requant fused into
// the store.  One kernel template serves the dense GEMM of qmatmul
// (mira/ops.py:616-620) and the implicit-GEMM convolution of qconv2d
// (mira/ops.py:630-634): only the loader of the activation tile differs.
//
// Tiling: a workgroup owns a BM x BN tile of the result and walks K in
// 64-byte steps.  Each step's A (activations, BM x 64) and B (weights,
// BN x 64) slices are fetched from global memory into registers while the
// previous slice is consumed from LDS (double-buffered LDS, one barrier per
// step).  Each wave computes a (BM/WM) x (BN/WN) sub-tile as 32x32 MFMA
// blocks.  Integer accumulation is exact and order-free, so A and B
// fragments only need the same byte order along K, which they get by
// construction (both read 16 contiguous K bytes per lane).
#include "mr_common.hpp"

namespace mr {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

enum AMode { A_DENSE = 0, A_CONV16 = 1, A_CONV4 = 2 };

struct GemmArgs {
  const int8_t* a;  // dense: [M, lda] int8; conv: NHWC int8 input
  int64_t lda;
  const int8_t* b;  // packed weights [n_pad, k_pad]
  int64_t k_pad;
  int64_t M;
  int32_t N;
  int32_t n_pad;
  int32_t k_tiles;
  int32_t tiles_m;
  int32_t tiles_n;
  // convolution geometry (A_CONV16 / A_CONV4)
  int32_t H, W, C_pad, OH, OW, KH, KW, SH, SW, PH, PW, DH, DW;
  int32_t row_bytes;  // A_CONV4: packed bytes per kernel row
  int32_t k_real;     // A_CONV16: KH*KW*C_pad (k beyond is padding)
};

constexpr int BK = 64;         // K bytes per pipeline step
constexpr int LDS_STRIDE = 80; // bytes per LDS row (64 data + 16 pad: conflict-free b128 reads)

// Dequantize, run the epilogue on, and store the 16 values of one 32x32 MFMA
// block that this lane holds: column `col`, rows rbase + 8*(r/4) + (r%4).
// The step loop runs at run time: the descriptor is a by-reference kernel
// argument, so indexing it dynamically reads the kernel-argument segment.
__device__ __forceinline__ void store_block(const EpiDev* __restrict__ e, const v16i& acc, int64_t rbase, int col,
                                            int64_t M, int N) {
  if (col >= N) return;
  const double scale = e->scale[col];
  int64_t rows[16];
  float y[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int64_t row = rbase + 8 * (r >> 2) + (r & 3);
    rows[r] = row < M ? row : M - 1;
    y[r] = dequant(acc[r], scale);
  }
  for (int s = 0; s < e->n_steps; ++s) {
    const EpiStepDev st = e->steps[s];
    if (st.fn == MR_EPI_RELU) {
#pragma unroll
      for (int v = 0; v < 16; ++v) y[v] = np_maximum(y[v], 0.0f);
      continue;
    }
    float o[16];
    if (st.mode == MR_BC_SCALAR) {
      const float c = st.ptr[0];
#pragma unroll
      for (int v = 0; v < 16; ++v) o[v] = c;
    } else if (st.mode == MR_BC_COL) {
      const float c = st.ptr[col];
#pragma unroll
      for (int v = 0; v < 16; ++v) o[v] = c;
    } else if (st.mode == MR_BC_ROW) {
#pragma unroll
      for (int v = 0; v < 16; ++v) o[v] = st.ptr[rows[v] * st.ld];
    } else {
#pragma unroll
      for (int v = 0; v < 16; ++v) o[v] = st.ptr[rows[v] * st.ld + col];
    }
    if (st.swapped) {
#pragma unroll
      for (int v = 0; v < 16; ++v) y[v] = epi_binary(st.fn, o[v], y[v]);
    } else {
#pragma unroll
      for (int v = 0; v < 16; ++v) y[v] = epi_binary(st.fn, y[v], o[v]);
    }
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int64_t row = rbase + 8 * (r >> 2) + (r & 3);
    if (row < M) {
      if (e->out_acc) e->out_acc[row * e->ldacc + col] = acc[r];
      epi_store(*e, y[r], row, col);
    }
  }
}

template <int BM, int BN, int WM, int WN, int AMODE>
__global__ void __launch_bounds__(WM* WN * 64) qgemm_kernel(const GemmArgs g, const EpiDev e) {
  constexpr int NT = WM * WN * 64;
  constexpr int TM = BM / WM;
  constexpr int TN = BN / WN;
  constexpr int FM = TM / 32;
  constexpr int FN = TN / 32;
  constexpr int A_PER_T = BM * 4 / NT;
  constexpr int B_PER_T = BN * 4 / NT;
  static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile must be a multiple of 32");
  static_assert(A_PER_T * NT == BM * 4 && B_PER_T * NT == BN * 4, "loader mapping");

  __shared__ __attribute__((aligned(16))) int8_t lds[2 * (BM + BN) * LDS_STRIDE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN;
  const int wn = wave % WN;

  // XCD-aware tile order: consecutive workgroup ids land on different XCDs
  // (round-robin over 8), so give each XCD a contiguous run of tiles; the
  // N-tiles of one M-tile then share that XCD's L2 for their A rows.
  const int total = g.tiles_m * g.tiles_n;
  int t = blockIdx.x;
  const int full = total & ~7;
  if (t < full) t = (t & 7) * (full >> 3) + (t >> 3);
  const int tile_m = t / g.tiles_n;
  const int tile_n = t - tile_m * g.tiles_n;
  const int64_t m0 = int64_t(tile_m) * BM;
  const int n0 = tile_n * BN;

  // ---- per-thread loader state
  const int kc = tid & 3;  // which 16-byte chunk of the 64-byte K step
  int64_t a_row_off[A_PER_T];  // dense: row byte offset; conv: image pixel base
  int32_t a_ih0[A_PER_T], a_iw0[A_PER_T];
  bool a_valid[A_PER_T];
#pragma unroll
  for (int i = 0; i < A_PER_T; ++i) {
    const int64_t m = m0 + (tid >> 2) + i * (NT >> 2);
    a_valid[i] = m < g.M;
    if (AMODE == A_DENSE) {
      a_row_off[i] = m * g.lda;
      a_ih0[i] = a_iw0[i] = 0;
    } else {
      const int64_t mm = a_valid[i] ? m : 0;
      const int64_t ohw = int64_t(g.OH) * g.OW;
      const int64_t img = mm / ohw;
      const int32_t rem = static_cast<int32_t>(mm - img * ohw);
      const int32_t oh = rem / g.OW;
      const int32_t ow = rem - oh * g.OW;
      a_row_off[i] = img * g.H * g.W;
      a_ih0[i] = oh * g.SH - g.PH;
      a_iw0[i] = ow * g.SW - g.PW;
    }
  }

  v4i ra[A_PER_T], rb[B_PER_T];

  auto load_global = [&](int kt) {
    const int32_t k = kt * BK + kc * 16;
#pragma unroll
    for (int i = 0; i < A_PER_T; ++i) {
      v4i v = {0, 0, 0, 0};
      if (AMODE == A_DENSE) {
        if (a_valid[i] && k < g.lda) v = *reinterpret_cast<const v4i*>(g.a + a_row_off[i] + k);
      } else if (AMODE == A_CONV16) {
        if (a_valid[i] && k < g.k_real) {
          const int32_t tap = k / g.C_pad;
          const int32_t c0 = k - tap * g.C_pad;
          const int32_t kh = tap / g.KW;
          const int32_t kw = tap - kh * g.KW;
          const int32_t ih = a_ih0[i] + kh * g.DH;
          const int32_t iw = a_iw0[i] + kw * g.DW;
          if (unsigned(ih) < unsigned(g.H) && unsigned(iw) < unsigned(g.W)) {
            const int64_t pix = a_row_off[i] + int64_t(ih) * g.W + iw;
            v = *reinterpret_cast<const v4i*>(g.a + pix * g.C_pad + c0);
          }
        }
      } else {  // A_CONV4: 4 taps of one kernel row, 4 channels (one dword) each
        const int32_t kh = k / g.row_bytes;
        const int32_t kw0 = (k - kh * g.row_bytes) >> 2;
        const int32_t ih = a_ih0[i] + kh * g.DH;
        if (a_valid[i] && kh < g.KH && unsigned(ih) < unsigned(g.H)) {
          const int32_t* rowp = reinterpret_cast<const int32_t*>(g.a) + (a_row_off[i] + int64_t(ih) * g.W);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int32_t kw = kw0 + j;
            const int32_t iw = a_iw0[i] + kw * g.DW;
            if (kw < g.KW && unsigned(iw) < unsigned(g.W)) v[j] = rowp[iw];
          }
        }
      }
      ra[i] = v;
    }
#pragma unroll
    for (int i = 0; i < B_PER_T; ++i) {
      const int n = n0 + (tid >> 2) + i * (NT >> 2);
      v4i v = {0, 0, 0, 0};
      if (n < g.n_pad) v = *reinterpret_cast<const v4i*>(g.b + int64_t(n) * g.k_pad + k);
      rb[i] = v;
    }
  };

  auto store_lds = [&](int buf) {
    int8_t* As = lds + buf * (BM + BN) * LDS_STRIDE;
    int8_t* Bs = As + BM * LDS_STRIDE;
#pragma unroll
    for (int i = 0; i < A_PER_T; ++i)
      *reinterpret_cast<v4i*>(As + ((tid >> 2) + i * (NT >> 2)) * LDS_STRIDE + kc * 16) = ra[i];
#pragma unroll
    for (int i = 0; i < B_PER_T; ++i)
      *reinterpret_cast<v4i*>(Bs + ((tid >> 2) + i * (NT >> 2)) * LDS_STRIDE + kc * 16) = rb[i];
  };

  v16i acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  load_global(0);
  store_lds(0);
  __syncthreads();

  const int frag_row = lane & 31;
  const int frag_k = (lane >> 5) * 16;
  for (int kt = 0; kt < g.k_tiles; ++kt) {
    const bool more = kt + 1 < g.k_tiles;
    if (more) load_global(kt + 1);
    const int8_t* As = lds + (kt & 1) * (BM + BN) * LDS_STRIDE;
    const int8_t* Bs = As + BM * LDS_STRIDE;
#pragma unroll
    for (int kk = 0; kk < BK; kk += 32) {
      v4i af[FM], bf[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[i] = *reinterpret_cast<const v4i*>(As + (wm * TM + i * 32 + frag_row) * LDS_STRIDE + kk + frag_k);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bf[j] = *reinterpret_cast<const v4i*>(Bs + (wn * TN + j * 32 + frag_row) * LDS_STRIDE + kk + frag_k);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if (more) store_lds((kt + 1) & 1);
    __syncthreads();
  }

  // ---- fused epilogue.  32x32 MFMA result layout: lane holds column
  // (lane & 31) and rows 8*(r/4) + 4*(lane/32) + (r%4), r = 0..15.
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int col = n0 + wn * TN + j * 32 + (lane & 31);
#pragma unroll
    for (int i = 0; i < FM; ++i)
      store_block(&e, acc[i][j], m0 + wm * TM + i * 32 + 4 * (lane >> 5), col, g.M, g.N);
  }
}

// ---------------------------------------------------------------- host dispatch

struct TileCfg {
  int bm, bn;
};

template <int AMODE>
static int launch(const GemmArgs& g0, const EpiDev& e, hipStream_t stream) {
  GemmArgs g = g0;
  // Pick the tile: wide N tiles when N allows, and enough workgroups to
  // cover the CUs (smaller M tiles for small problems).
  const int cus = device_cu_count();
  int bm, bn;
  if (g.N <= 32) {
    bm = 64; bn = 32;
  } else if (g.N <= 64) {
    bm = ((g.M + 255) / 256 >= cus) ? 256 : 128;
    bn = 64;
  } else {
    bn = 128;
    bm = ((g.M + 255) / 256) * ((g.N + 127) / 128) >= 2 * cus ? 256 : 128;
  }
  g.tiles_m = static_cast<int32_t>((g.M + bm - 1) / bm);
  g.tiles_n = (g.N + bn - 1) / bn;
  const int64_t blocks = int64_t(g.tiles_m) * g.tiles_n;
  MR_REQUIRE(blocks < (int64_t(1) << 31), "problem too large: %lld tiles", (long long)blocks);
  dim3 grid(static_cast<unsigned>(blocks));
  if (bm == 64 && bn == 32) {
    hipLaunchKernelGGL((qgemm_kernel<64, 32, 2, 1, AMODE>), grid, dim3(128), 0, stream, g, e);
  } else if (bm == 128 && bn == 64) {
    hipLaunchKernelGGL((qgemm_kernel<128, 64, 2, 1, AMODE>), grid, dim3(128), 0, stream, g, e);
  } else if (bm == 256 && bn == 64) {
    hipLaunchKernelGGL((qgemm_kernel<256, 64, 4, 1, AMODE>), grid, dim3(256), 0, stream, g, e);
  } else if (bm == 128 && bn == 128) {
    hipLaunchKernelGGL((qgemm_kernel<128, 128, 2, 2, AMODE>), grid, dim3(256), 0, stream, g, e);
  } else {
    hipLaunchKernelGGL((qgemm_kernel<256, 128, 2, 2, AMODE>), grid, dim3(256), 0, stream, g, e);
  }
  MR_LAUNCH_CHECK("qgemm");
  return MR_OK;
}

static bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

}  // namespace mr

extern "C" {

int mr_qmatmul(const int8_t* a, int64_t lda, const int8_t* b, int64_t k_pad, int64_t n_pad, int64_t M, int64_t N,
               int64_t K, const mr_epilogue* epi, void* stream) {
  MR_REQUIRE(a && b, "mr_qmatmul: NULL operand");
  MR_REQUIRE(M >= 0 && N > 0 && K > 0, "mr_qmatmul: bad sizes M=%lld N=%lld K=%lld", (long long)M, (long long)N,
             (long long)K);
  MR_REQUIRE(lda >= K && lda % 16 == 0, "mr_qmatmul: lda %lld must be >= K and a multiple of 16", (long long)lda);
  MR_REQUIRE(k_pad >= K && k_pad % 64 == 0, "mr_qmatmul: k_pad %lld must be >= K and a multiple of 64",
             (long long)k_pad);
  MR_REQUIRE(n_pad >= N && n_pad % 32 == 0, "mr_qmatmul: n_pad %lld must be >= N and a multiple of 32",
             (long long)n_pad);
  MR_REQUIRE(N < (int64_t(1) << 30) && k_pad < (int64_t(1) << 30), "mr_qmatmul: N or K too large");
  MR_REQUIRE(mr::aligned16(a) && mr::aligned16(b), "mr_qmatmul: operands must be 16-byte aligned");
  mr::EpiDev e;
  int rc = mr::make_epi(epi, N, true, &e);
  if (rc != MR_OK) return rc;
  if (M == 0) return MR_OK;
  mr::GemmArgs g = {};
  g.a = a;
  g.lda = lda;
  g.b = b;
  g.k_pad = k_pad;
  g.M = M;
  g.N = static_cast<int32_t>(N);
  g.n_pad = static_cast<int32_t>(n_pad);
  g.k_tiles = static_cast<int32_t>(k_pad / mr::BK);
  return mr::launch<mr::A_DENSE>(g, e, static_cast<hipStream_t>(stream));
}

int mr_qconv2d(const int8_t* x, const mr_conv_geom* cg, const int8_t* b, int64_t k_pad, int64_t n_pad,
               const mr_epilogue* epi, void* stream) {
  MR_REQUIRE(x && cg && b, "mr_qconv2d: NULL argument");
  const mr_conv_geom& G = *cg;
  MR_REQUIRE(G.n >= 0 && G.h > 0 && G.w > 0 && G.c > 0 && G.o > 0, "mr_qconv2d: bad shape");
  MR_REQUIRE(G.kh > 0 && G.kw > 0 && G.sh > 0 && G.sw > 0 && G.dh > 0 && G.dw > 0 && G.ph >= 0 && G.pw >= 0,
             "mr_qconv2d: bad kernel/stride/padding/dilation");
  const int32_t oh = (G.h + 2 * G.ph - G.dh * (G.kh - 1) - 1) / G.sh + 1;
  const int32_t ow = (G.w + 2 * G.pw - G.dw * (G.kw - 1) - 1) / G.sw + 1;
  MR_REQUIRE(oh == G.oh && ow == G.ow && oh > 0 && ow > 0, "mr_qconv2d: output %dx%d does not match geometry (%dx%d)",
             G.oh, G.ow, oh, ow);
  int mode;
  int32_t row_bytes = 0, k_real = 0;
  if (G.c_pad == 4) {
    MR_REQUIRE(G.c <= 4, "mr_qconv2d: c_pad 4 holds at most 4 channels");
    mode = mr::A_CONV4;
    row_bytes = 16 * ((G.kw + 3) / 4);
    k_real = G.kh * row_bytes;
  } else {
    MR_REQUIRE(G.c_pad % 16 == 0 && G.c_pad >= G.c, "mr_qconv2d: c_pad %d must be 4 or a multiple of 16 >= c",
               G.c_pad);
    mode = mr::A_CONV16;
    k_real = G.kh * G.kw * G.c_pad;
  }
  MR_REQUIRE(k_pad >= k_real && k_pad % 64 == 0, "mr_qconv2d: k_pad %lld must be >= %d and a multiple of 64",
             (long long)k_pad, k_real);
  MR_REQUIRE(n_pad >= G.o && n_pad % 32 == 0, "mr_qconv2d: n_pad %lld must be >= o and a multiple of 32",
             (long long)n_pad);
  MR_REQUIRE(int64_t(G.n) * G.h * G.w < (int64_t(1) << 31), "mr_qconv2d: input has too many pixels");
  MR_REQUIRE(mr::aligned16(x) && mr::aligned16(b), "mr_qconv2d: operands must be 16-byte aligned");
  mr::EpiDev e;
  const int rc = mr::make_epi(epi, G.o, true, &e);
  if (rc != MR_OK) return rc;
  const int64_t M = int64_t(G.n) * oh * ow;
  if (M == 0) return MR_OK;
  mr::GemmArgs g = {};
  g.a = x;
  g.lda = 0;
  g.b = b;
  g.k_pad = k_pad;
  g.M = M;
  g.N = G.o;
  g.n_pad = static_cast<int32_t>(n_pad);
  g.k_tiles = static_cast<int32_t>(k_pad / mr::BK);
  g.H = G.h;
  g.W = G.w;
  g.C_pad = G.c_pad;
  g.OH = oh;
  g.OW = ow;
  g.KH = G.kh;
  g.KW = G.kw;
  g.SH = G.sh;
  g.SW = G.sw;
  g.PH = G.ph;
  g.PW = G.pw;
  g.DH = G.dh;
  g.DW = G.dw;
  g.row_bytes = row_bytes;
  g.k_real = k_real;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return mode == mr::A_CONV4 ? mr::launch<mr::A_CONV4>(g, e, s) : mr::launch<mr::A_CONV16>(g, e, s);
}

}  // extern "C"
