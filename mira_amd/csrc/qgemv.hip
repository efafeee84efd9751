// Small-M int8 matmul (decode-shaped qmatmul, mira/ops.py:616-620): M <= 8
// activation rows against packed weights (K-step-major: 64-byte slice kt of
// row n at (kt * n_pad + n) * 64).  With so few rows the work is reading the
// weights once (N*K bytes: 16 MiB per 4096x4096 layer), so the kernels are
// coalesced weight streams rather than MFMA tiles, multiplying 16-byte weight
// chunks with the matching activation bytes by v_dot4 (4 exact int8
// multiply-adds into int32).  qgemv_ks_kernel (k_pad <= 4096) lays a wave's
// loads along the packed rows, 1 KB contiguous each; qgemv_kernel (longer K)
// gives a group of LPC lanes CPW output columns, each lane walking 16-byte
// chunks of those columns, and reduces with lane shuffles.  The dequant /
// epilogue / requant of each result element runs on one lane (mira/ops.py:618,
// 192-199, 602-603).
#include "mr_common.hpp"
#include "np_sum.hpp"

namespace mr {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int GEMV_CPW = 2;   // output columns per lane group
constexpr int GEMV_UNR = 4;   // 16-byte weight chunks per column a lane has in flight

struct GemvArgs {
  const int8_t* a;    // [M][lda] int8 activations
  int64_t lda;
  const int8_t* b;    // packed weights, [k_pad / 64][n_pad][64]
  int32_t k_pad, N, lpc;   // lpc: lanes per column group (power of two, <= 64)
  int32_t n_pad;
  int32_t M;
};

template <int MR>
__global__ void __launch_bounds__(256) qgemv_kernel(const GemvArgs g, const EpiDev e) {
  const int lane = threadIdx.x & 63;
  const int lpc = g.lpc;
  const int sub = lane & (lpc - 1);                        // lane within its group
  const int64_t group = (int64_t(blockIdx.x) * 256 + threadIdx.x) / lpc;
  const int n0 = static_cast<int>(group * GEMV_CPW);
  const int chunks = g.k_pad / 16;

  int acc[MR][GEMV_CPW];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int c = 0; c < GEMV_CPW; ++c) acc[m][c] = 0;

  if (n0 < g.N) {
    const int8_t* brow[GEMV_CPW];
#pragma unroll
    for (int c = 0; c < GEMV_CPW; ++c) brow[c] = g.b + int64_t(min(n0 + c, g.N - 1)) * 64;
    const int64_t kstep = int64_t(g.n_pad) * 64;   // bytes between K steps of one row
    // GEMV_UNR chunks per column in flight per lane: the weights are read once, so the
    // stream's rate is the bytes in flight over the memory latency
    for (int kb = sub; kb < chunks; kb += GEMV_UNR * lpc) {
      v4i w[GEMV_UNR][GEMV_CPW];
#pragma unroll
      for (int u = 0; u < GEMV_UNR; ++u) {
        const int k16 = min(kb + u * lpc, chunks - 1);   // past the end: reread the last chunk, unused
#pragma unroll
        for (int c = 0; c < GEMV_CPW; ++c)
          w[u][c] = *reinterpret_cast<const v4i*>(brow[c] + (k16 >> 2) * kstep + (k16 & 3) * 16);
      }
#pragma unroll
      for (int u = 0; u < GEMV_UNR; ++u) {
        const int k16 = kb + u * lpc;
        if (k16 >= chunks) break;
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          if (m >= g.M) break;
          // activation bytes past K read the zero-padded row stride or, beyond
          // lda, contribute against zero weights; lda >= K and the weights are
          // zero for k >= K, so only bytes < lda are ever nonzero products
          v4i x = {0, 0, 0, 0};
          if (k16 * 16 < g.lda) x = *reinterpret_cast<const v4i*>(g.a + m * g.lda + k16 * 16);
#pragma unroll
          for (int c = 0; c < GEMV_CPW; ++c)
#pragma unroll
            for (int q = 0; q < 4; ++q) acc[m][c] = __builtin_amdgcn_sdot4(x[q], w[u][c][q], acc[m][c], false);
        }
      }
    }
  }
  // reduce over the group's lanes (all lanes of a group end with the sums)
  for (int off = lpc >> 1; off > 0; off >>= 1)
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
      for (int c = 0; c < GEMV_CPW; ++c) acc[m][c] += __shfl_xor(acc[m][c], off, 64);

  // lane `sub` of the group finishes element (m, c) = (sub / CPW, sub % CPW)
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int c = 0; c < GEMV_CPW; ++c) {
      if (sub != m * GEMV_CPW + c || m >= g.M || n0 + c >= g.N) continue;
      const int n = n0 + c;
      const int32_t v = acc[m][c];
      if (e.out_acc) e.out_acc[int64_t(m) * e.ldacc + n] = v;
      epi_store(e, epi_steps(e, dequant(v, e.scale[n]), m, n), m, n);
    }
}

// The same product with the weight stream laid along the packed rows: a
// workgroup of KW waves owns COLS adjacent columns; the LPC = 64 / COLS lanes of
// a column read consecutive 16-byte chunks of its 64-byte K-step rows, SPL =
// LPC / 4 steps per wave-wide load, so one load is COLS runs of SPL * 64 bytes
// (the packed layout keeps a K step of consecutive columns contiguous: with 16
// columns one load is the 1 KB run of their rows), and wave w covers its share of
// the K steps.  Each column's lanes reduce by shuffles, the KW waves through LDS,
// and the first COLS * M threads finish one element each with the same epilogue.
// The sums are exact int32, so the order does not matter.  Taken for k_pad <= 4096
// (every load of a lane in flight at once): 5.2 -> 4.7 us on a 4096x4096 layer at
// M = 1, 16.7 -> 11.8 us at M = 8.  Fewer columns per workgroup spread a narrow
// layer over more CUs (4096 -> 1000 at M = 1: 63 workgroups of 16 columns, or 250
// of 4).  Longer K stays on qgemv_kernel, whose lanes share each activation load
// between two columns (at K = 16384 and M = 3 it is 1.5x faster than this one).
//
// The activation rows are staged in LDS, and their loads are issued before the
// weight stream's: the vector-memory counter completes in issue order, so a row
// load issued after the weights would wait for all of them, and one per K step
// made each lane's later steps serial L2 round trips.  F32IN: the rows arrive as
// f32 and each workgroup quantizes them into LDS (mr_quantize_rows's arithmetic,
// mira/ops.py:602-603) while its weights are in flight, so the separate quantize
// launch of a decode step's first layer disappears behind the weight stream.
constexpr int KS_MAXS = 8;    // wave-wide loads a lane has in flight at once
constexpr int KS_KMAX = 4096; // largest k_pad of this kernel (8 waves x 8 steps x 64 bytes)

constexpr int LN_KMAX = 1024; // longest row the layer-normalising prologue takes

// The f32 rows of PRE 1 and 2: x [M][ldx] (K = GemvArgs::lda valid columns), the int8
// scale xs; PRE 2 layer-normalises each row first (gain g, bias b, eps; f16: the normalised
// values rounded to f16 before the quantize)
struct RowIn {
  const float* x;
  int64_t ldx;
  float xs;
  const float* g;
  const float* b;
  float eps;
  int32_t f16;
};

// PRE 0: int8 rows (GemvArgs::a); 1: f32 rows quantized here (the F32IN prologue);
// 2: f32 rows layer-normalised and quantized here (mira/ops.py:356-360 with the layernorm
// kernel's arithmetic, one wave per row)
template <int MR, int KW, int COLS, int PRE>
__global__ void __launch_bounds__(KW * 64) qgemv_ks_kernel(const GemvArgs g, const EpiDev e, const RowIn rin) {
  constexpr bool F32IN = PRE != 0, LN = PRE == 2;
  constexpr int LPC = 64 / COLS;   // lanes per column
  constexpr int SPL = LPC / 4;     // K steps per wave-wide load
  constexpr int NT = KW * 64;      // threads
  static_assert(KW * KS_MAXS * 64 >= KS_KMAX, "one pass covers k_pad");
  static_assert(!LN || (MR <= KW && 2 * LN_KMAX <= 4 * NT), "one wave per row; gains and biases in one pass");
  __shared__ int red[KW][MR][COLS];
  __shared__ __attribute__((aligned(16))) int8_t xq[MR][KS_KMAX];
  __shared__ __attribute__((aligned(16))) float xf[LN ? MR : 1][LN ? LN_KMAX : 4];   // LN: the f32 rows
  __shared__ float gbl[LN ? 2 * LN_KMAX : 1];                                        // LN: gains, biases
  const float* x = rin.x;
  const int64_t ldx = rin.ldx;
  const float xs = rin.xs;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = blockIdx.x * COLS;
  const int col = lane / LPC, j = lane % LPC;
  const int ksteps = g.k_pad / 64;
  // each wave's share of the steps, a whole number of loads (SPL steps each)
  const int per_wave = ((ksteps + KW - 1) / KW + SPL - 1) / SPL * SPL;
  const int s_begin = wave * per_wave, s_end = min(s_begin + per_wave, ksteps);
  const int8_t* bcol = g.b + int64_t(n0 + col) * 64 + (j & 3) * 16;   // n0 + COLS <= n_pad
  const int64_t kstep = int64_t(g.n_pad) * 64;

  // the rows' loads: F32IN 4 f32 words per thread and load (16-byte loads where the
  // rows allow), else 16 int8 bytes (lda % 16 == 0 and a 16-byte aligned: a chunk
  // is all below lda or all past it); zeros past the rows' ends
  constexpr int XB = F32IN ? 4 : 16;                        // row elements per thread and load
  constexpr int NQ = (MR * (LN ? LN_KMAX : KS_KMAX) / XB + NT - 1) / NT;   // loads per thread at most
  const int per_row = g.k_pad / XB;
  float4 vf[F32IN ? NQ : 1];
  v4i vi[F32IN ? 1 : NQ];
#pragma unroll
  for (int u = 0; u < NQ; ++u) {
    const int i = threadIdx.x + u * NT;
    const int m = i / per_row, k0 = (i - m * per_row) * XB;
    if constexpr (F32IN) {
      const bool vec = reinterpret_cast<uintptr_t>(x) % 16 == 0 && ldx % 4 == 0;
      vf[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (m < g.M && k0 < g.lda) {
        const float* xr = x + m * ldx + k0;
        if (vec && k0 + 3 < g.lda) {
          vf[u] = *reinterpret_cast<const float4*>(xr);
        } else {
          vf[u].x = xr[0];
          if (k0 + 1 < g.lda) vf[u].y = xr[1];
          if (k0 + 2 < g.lda) vf[u].z = xr[2];
          if (k0 + 3 < g.lda) vf[u].w = xr[3];
        }
      }
    } else {
      vi[u] = v4i{0, 0, 0, 0};
      if (m < g.M && k0 < g.lda) vi[u] = *reinterpret_cast<const v4i*>(g.a + m * g.lda + k0);
    }
  }
  // LN: the gains and biases ([g | b], 2K floats), before the weights as well
  float gbv[LN ? 4 : 1];
  if constexpr (LN) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = threadIdx.x + u * NT;
      gbv[u] = i < g.lda ? rin.g[i] : i < 2 * g.lda ? rin.b[i - g.lda] : 0.0f;
    }
  }
  // then the weight stream, every load of a lane in flight at once
  v4i w[KS_MAXS];
#pragma unroll
  for (int i = 0; i < KS_MAXS; ++i) {
    const int s = min(s_begin + i * SPL + (j >> 2), ksteps - 1);   // past the share: re-read, unused
    w[i] = *reinterpret_cast<const v4i*>(bcol + s * kstep);
  }
  // the rows into LDS (quantized for F32IN) while the weights arrive
#pragma unroll
  for (int u = 0; u < NQ; ++u) {
    const int i = threadIdx.x + u * NT;
    if (i >= MR * per_row) break;
    const int m = i / per_row, k0 = (i - m * per_row) * XB;
    if (m >= g.M) break;
    if constexpr (LN) {
      *reinterpret_cast<float4*>(&xf[m][k0]) = vf[u];
    } else if constexpr (F32IN) {
      const float f[4] = {vf[u].x, vf[u].y, vf[u].z, vf[u].w};
      uint32_t packed = 0;
#pragma unroll
      for (int t = 0; t < 4; ++t)
        if (k0 + t < g.lda) packed |= uint32_t(uint8_t(quantize_one(f[t], xs))) << (8 * t);
      *reinterpret_cast<uint32_t*>(&xq[m][k0]) = packed;
    } else {
      *reinterpret_cast<v4i*>(&xq[m][k0]) = vi[u];
    }
  }
  if constexpr (LN) {
    // wave m normalises row m from LDS, as layernorm_kernel does, and quantizes it
#pragma unroll
    for (int u = 0; u < 4; ++u) gbl[threadIdx.x + u * NT < 2 * LN_KMAX ? threadIdx.x + u * NT : 0] = gbv[u];
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (wave < g.M) {
      const int d = g.lda;
      float mu, sd;
      layernorm_row_stats([&](int64_t i) { return xf[wave][i]; }, d, lane, rin.eps, mu, sd);
      for (int i = lane; i < d; i += 64) {
        float v = layernorm_value(xf[wave][i], mu, sd, gbl[i], gbl[d + i]);
        if (rin.f16) v = round_f16(v);
        xq[wave][i] = quantize_one(v, xs);
      }
    }
  }
  // every wave's LDS stores done before any wave reads: an LDS-only wait and the
  // barrier, so the weight loads stay in flight across it (__syncthreads would
  // wait for them); the memory clobber keeps the compiler from moving LDS
  // accesses across
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  int acc[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) acc[m] = 0;
#pragma unroll
  for (int i = 0; i < KS_MAXS; ++i) {
    const int s = s_begin + i * SPL + (j >> 2);
    if (s_begin + i * SPL >= s_end) break;
    if (s >= s_end) continue;
    const int k = s * 64 + (j & 3) * 16;
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      if (m >= g.M) break;
      const v4i xv = *reinterpret_cast<const v4i*>(&xq[m][k]);
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[m] = __builtin_amdgcn_sdot4(xv[q], w[i][q], acc[m], false);
    }
  }
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int off = 1; off < LPC; off <<= 1) acc[m] += __shfl_xor(acc[m], off, 64);
  if (j == 0) {
#pragma unroll
    for (int m = 0; m < MR; ++m) red[wave][m][col] = acc[m];
  }
  __syncthreads();
  const int t = threadIdx.x;
  if (t < MR * COLS) {
    const int m = t / COLS, c = t % COLS, n = n0 + c;
    if (m < g.M && n < g.N) {
      int32_t v = 0;
#pragma unroll
      for (int w = 0; w < KW; ++w) v += red[w][m][c];
      if (e.out_acc) e.out_acc[int64_t(m) * e.ldacc + n] = v;
      epi_store(e, epi_steps(e, dequant(v, e.scale[n]), m, n), m, n);
    }
  }
}

// Weight-only int8 (mira/quantize.py:45-68): y[M,N] = x[M,K] (f32) @ W, W the
// dequantized constant fl32(q[k][n] * scale[n]) (mira/ops.py:581-589), then
// the epilogue (mira/ops.py:217-219).  Same weight stream as qgemv_kernel
// (16-byte chunks of packed int8 columns, LPC lanes per column pair); each
// weight byte is dequantized into f32 exactly as the reference does, then
// multiply-added into f32 accumulators.  blockIdx.y picks a block of MR rows
// (the weights are streamed once per block: meant for decode shapes).  The summation order is not
// NumPy's BLAS order, so results agree to f32 rounding, not bit for bit.
template <int MR>
__global__ void __launch_bounds__(256) w8gemv_kernel(const float* __restrict__ x, const int64_t ldx,
                                                      const float* __restrict__ wscale, const int w_f16,
                                                      const GemvArgs g, const EpiDev e) {
  const int lane = threadIdx.x & 63;
  const int lpc = g.lpc;
  const int sub = lane & (lpc - 1);
  const int64_t group = (int64_t(blockIdx.x) * 256 + threadIdx.x) / lpc;
  const int n0 = static_cast<int>(group * GEMV_CPW);
  const int chunks = g.k_pad / 16;
  const bool x_vec = (ldx & 3) == 0;   // rows 16-byte aligned: float4 activation loads
  const int r0 = blockIdx.y * MR;      // first row of this block
  const int rows = min(MR, g.M - r0);

  float acc[MR][GEMV_CPW];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int c = 0; c < GEMV_CPW; ++c) acc[m][c] = 0.0f;

  if (n0 < g.N) {
    const int8_t* brow[GEMV_CPW];
    float s[GEMV_CPW];
#pragma unroll
    for (int c = 0; c < GEMV_CPW; ++c) {
      const int n = min(n0 + c, g.N - 1);
      brow[c] = g.b + int64_t(n) * 64;
      s[c] = wscale[n];
    }
    const int64_t kstep = int64_t(g.n_pad) * 64;
    for (int k16 = sub; k16 < chunks; k16 += lpc) {
      if (k16 * 16 >= g.lda) break;   // past K: zero weights and no activation columns
      v4i wq[GEMV_CPW];
#pragma unroll
      for (int c = 0; c < GEMV_CPW; ++c)
        wq[c] = *reinterpret_cast<const v4i*>(brow[c] + (k16 >> 2) * kstep + (k16 & 3) * 16);
      float w[GEMV_CPW][16];
#pragma unroll
      for (int c = 0; c < GEMV_CPW; ++c)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          w[c][i] = __fmul_rn(static_cast<float>(static_cast<int8_t>(wq[c][i >> 2] >> (8 * (i & 3)))), s[c]);
      if (w_f16) {   // f16 weights (a dequantize of dtype f16): the product rounded once more
#pragma unroll
        for (int c = 0; c < GEMV_CPW; ++c)
#pragma unroll
          for (int i = 0; i < 16; ++i) w[c][i] = round_f16(w[c][i]);
      }
      const int kv = min(16, static_cast<int>(g.lda) - k16 * 16);   // activation columns in this chunk
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        if (m >= rows) break;
        const float* xr = x + (r0 + m) * ldx + k16 * 16;
        float xv[16];
        if (kv == 16 && x_vec) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float4 t = *reinterpret_cast<const float4*>(xr + 4 * q);
            xv[4 * q] = t.x; xv[4 * q + 1] = t.y; xv[4 * q + 2] = t.z; xv[4 * q + 3] = t.w;
          }
        } else {
#pragma unroll
          for (int i = 0; i < 16; ++i) xv[i] = i < kv ? xr[i] : 0.0f;
        }
#pragma unroll
        for (int c = 0; c < GEMV_CPW; ++c)
#pragma unroll
          for (int i = 0; i < 16; ++i) acc[m][c] = __fmaf_rn(xv[i], w[c][i], acc[m][c]);
      }
    }
  }
  for (int off = lpc >> 1; off > 0; off >>= 1)
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
      for (int c = 0; c < GEMV_CPW; ++c) acc[m][c] += __shfl_xor(acc[m][c], off, 64);

#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int c = 0; c < GEMV_CPW; ++c) {
      if (sub != m * GEMV_CPW + c || m >= rows || n0 + c >= g.N) continue;
      const int n = n0 + c;
      epi_store(e, epi_steps(e, acc[m][c], r0 + m, n), r0 + m, n);
    }
}

// The weight-row stream for M <= 8, k_pad <= 4096: 16 columns per workgroup where
// that gives every CU one, else 8 or 4 (n0 + COLS <= n_pad: n_pad % 32 == 0).
template <int PRE, int MR>
static void ks_launch_m(const GemvArgs& g, const EpiDev& e, const RowIn& rin, hipStream_t stream) {
  const int64_t cus = device_cu_count();
  const int cols = (g.N + 15) / 16 >= cus ? 16 : (g.N + 7) / 8 >= cus ? 8 : 4;
  const dim3 grid(static_cast<unsigned>((g.N + cols - 1) / cols)), block(512);
  if (cols == 16)
    hipLaunchKernelGGL((qgemv_ks_kernel<MR, 8, 16, PRE>), grid, block, 0, stream, g, e, rin);
  else if (cols == 8)
    hipLaunchKernelGGL((qgemv_ks_kernel<MR, 8, 8, PRE>), grid, block, 0, stream, g, e, rin);
  else
    hipLaunchKernelGGL((qgemv_ks_kernel<MR, 8, 4, PRE>), grid, block, 0, stream, g, e, rin);
}

template <int PRE>
static void ks_launch(const GemvArgs& g, const EpiDev& e, const RowIn& rin, hipStream_t stream) {
  if (g.M == 1)
    ks_launch_m<PRE, 1>(g, e, rin, stream);
  else if (g.M == 2)
    ks_launch_m<PRE, 2>(g, e, rin, stream);
  else if (g.M <= 4)
    ks_launch_m<PRE, 4>(g, e, rin, stream);
  else
    ks_launch_m<PRE, 8>(g, e, rin, stream);
}

// M <= 8 rows: returns MR_EUNSUPPORTED for larger M (the caller uses the tiled kernel).
int gemv_launch(const int8_t* a, int64_t lda, const int8_t* b, int64_t k_pad, int64_t n_pad, int64_t M,
                int64_t N, const EpiDev& e, hipStream_t stream) {
  if (M > 8) return MR_EUNSUPPORTED;
  GemvArgs g = {};
  g.a = a;
  g.lda = lda;
  g.b = b;
  g.k_pad = static_cast<int32_t>(k_pad);
  g.n_pad = static_cast<int32_t>(n_pad);
  g.N = static_cast<int32_t>(N);
  g.M = static_cast<int32_t>(M);
  if (k_pad <= KS_KMAX) {
    ks_launch<0>(g, e, RowIn{}, stream);
    MR_LAUNCH_CHECK("qgemv");
    return MR_OK;
  }
  // lanes per column group: enough 16-byte chunks per lane to keep loads in
  // flight, and at least M * CPW lanes to finish the results
  int lpc = 64;
  while (lpc > 4 && k_pad / 16 < 4 * lpc) lpc >>= 1;
  while (lpc < M * GEMV_CPW) lpc <<= 1;
  g.lpc = lpc;
  const int64_t groups = (N + GEMV_CPW - 1) / GEMV_CPW;
  const int64_t blocks = (groups * lpc + 255) / 256;
  MR_REQUIRE(blocks < (int64_t(1) << 31), "qgemv: too many columns");
  const dim3 grid(static_cast<unsigned>(blocks));
  if (M == 1)
    hipLaunchKernelGGL(qgemv_kernel<1>, grid, dim3(256), 0, stream, g, e);
  else if (M == 2)
    hipLaunchKernelGGL(qgemv_kernel<2>, grid, dim3(256), 0, stream, g, e);
  else if (M <= 4)
    hipLaunchKernelGGL(qgemv_kernel<4>, grid, dim3(256), 0, stream, g, e);
  else
    hipLaunchKernelGGL(qgemv_kernel<8>, grid, dim3(256), 0, stream, g, e);
  MR_LAUNCH_CHECK("qgemv");
  return MR_OK;
}

}  // namespace mr

extern "C" int mr_qmatmul_f32in(const float* x, int64_t ldx, float x_scale, const int8_t* b, int64_t k_pad,
                                int64_t n_pad, int64_t M, int64_t N, int64_t K, const mr_epilogue* epi,
                                void* stream) {
  MR_REQUIRE(x && b, "mr_qmatmul_f32in: NULL operand");
  MR_REQUIRE(M >= 0 && N > 0 && K > 0, "mr_qmatmul_f32in: bad sizes M=%lld N=%lld K=%lld", (long long)M,
             (long long)N, (long long)K);
  MR_REQUIRE(ldx >= K && x_scale > 0.0f, "mr_qmatmul_f32in: ldx %lld < K %lld or x_scale %g <= 0", (long long)ldx,
             (long long)K, (double)x_scale);
  MR_REQUIRE(k_pad >= K && k_pad % 64 == 0, "mr_qmatmul_f32in: k_pad %lld must be >= K and a multiple of 64",
             (long long)k_pad);
  MR_REQUIRE(n_pad >= N && n_pad % 32 == 0 && N < (int64_t(1) << 30),
             "mr_qmatmul_f32in: n_pad %lld must be >= N and a multiple of 32", (long long)n_pad);
  MR_REQUIRE(reinterpret_cast<uintptr_t>(b) % 16 == 0, "mr_qmatmul_f32in: weights must be 16-byte aligned");
  if (M > 8 || k_pad > mr::KS_KMAX) {
    mr::set_error("mr_qmatmul_f32in: M=%lld rows, k_pad %lld: the fused quantize takes M <= 8 and k_pad <= %d",
                  (long long)M, (long long)k_pad, mr::KS_KMAX);
    return MR_EUNSUPPORTED;
  }
  mr::EpiDev e;
  const int rc = mr::make_epi(epi, N, true, &e, true);
  if (rc != MR_OK) return rc;
  if (M == 0) return MR_OK;
  mr::GemvArgs g = {};
  g.lda = K;   // columns of x
  g.b = b;
  g.k_pad = static_cast<int32_t>(k_pad);
  g.n_pad = static_cast<int32_t>(n_pad);
  g.N = static_cast<int32_t>(N);
  g.M = static_cast<int32_t>(M);
  mr::RowIn rin = {};
  rin.x = x;
  rin.ldx = ldx;
  rin.xs = x_scale;
  mr::ks_launch<1>(g, e, rin, static_cast<hipStream_t>(stream));
  MR_LAUNCH_CHECK("qgemv_f32in");
  return MR_OK;
}

extern "C" int mr_qmatmul_lnin(const float* x, int64_t ldx, const float* gamma, const float* beta, float eps,
                               int32_t round_f16, float x_scale, const int8_t* b, int64_t k_pad, int64_t n_pad,
                               int64_t M, int64_t N, int64_t K, const mr_epilogue* epi, void* stream) {
  MR_REQUIRE(x && gamma && beta && b, "mr_qmatmul_lnin: NULL operand");
  MR_REQUIRE(M >= 0 && N > 0 && K > 0, "mr_qmatmul_lnin: bad sizes M=%lld N=%lld K=%lld", (long long)M,
             (long long)N, (long long)K);
  MR_REQUIRE(ldx >= K && x_scale > 0.0f, "mr_qmatmul_lnin: ldx %lld < K %lld or x_scale %g <= 0", (long long)ldx,
             (long long)K, (double)x_scale);
  MR_REQUIRE(k_pad >= K && k_pad % 64 == 0, "mr_qmatmul_lnin: k_pad %lld must be >= K and a multiple of 64",
             (long long)k_pad);
  MR_REQUIRE(n_pad >= N && n_pad % 32 == 0 && N < (int64_t(1) << 30),
             "mr_qmatmul_lnin: n_pad %lld must be >= N and a multiple of 32", (long long)n_pad);
  MR_REQUIRE(reinterpret_cast<uintptr_t>(b) % 16 == 0, "mr_qmatmul_lnin: weights must be 16-byte aligned");
  if (M > 8 || K > mr::LN_KMAX || k_pad > mr::LN_KMAX) {
    mr::set_error("mr_qmatmul_lnin: M=%lld rows, K=%lld: the fused layer normalisation takes M <= 8 and "
                  "k_pad <= %d", (long long)M, (long long)K, mr::LN_KMAX);
    return MR_EUNSUPPORTED;
  }
  mr::EpiDev e;
  const int rc = mr::make_epi(epi, N, true, &e, true);
  if (rc != MR_OK) return rc;
  if (M == 0) return MR_OK;
  mr::GemvArgs g = {};
  g.lda = K;   // columns of x: the normalised length
  g.b = b;
  g.k_pad = static_cast<int32_t>(k_pad);
  g.n_pad = static_cast<int32_t>(n_pad);
  g.N = static_cast<int32_t>(N);
  g.M = static_cast<int32_t>(M);
  mr::RowIn rin = {};
  rin.x = x;
  rin.ldx = ldx;
  rin.xs = x_scale;
  rin.g = gamma;
  rin.b = beta;
  rin.eps = eps;
  rin.f16 = round_f16;
  mr::ks_launch<2>(g, e, rin, static_cast<hipStream_t>(stream));
  MR_LAUNCH_CHECK("qgemv_lnin");
  return MR_OK;
}

extern "C" int mr_w8_matmul_f32(const float* x, int64_t ldx, const int8_t* b, const float* w_scale, int32_t w_f16,
                                int64_t k_pad, int64_t n_pad, int64_t M, int64_t N, int64_t K,
                                const mr_epilogue* epi, void* stream) {
  MR_REQUIRE(x && b && w_scale, "mr_w8_matmul_f32: NULL operand");
  MR_REQUIRE(M >= 0 && N > 0 && K > 0, "mr_w8_matmul_f32: M=%lld, N=%lld, K=%lld", (long long)M, (long long)N,
             (long long)K);
  MR_REQUIRE(ldx >= K, "mr_w8_matmul_f32: ldx %lld < K %lld", (long long)ldx, (long long)K);
  MR_REQUIRE(k_pad >= K && k_pad % 64 == 0, "mr_w8_matmul_f32: k_pad %lld must be >= K and a multiple of 64",
             (long long)k_pad);
  MR_REQUIRE(n_pad >= N && n_pad % 32 == 0, "mr_w8_matmul_f32: n_pad %lld must be >= N and a multiple of 32",
             (long long)n_pad);
  MR_REQUIRE(N < (int64_t(1) << 30) && k_pad < (int64_t(1) << 30), "mr_w8_matmul_f32: problem too large");
  MR_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(b) % 16 == 0,
             "mr_w8_matmul_f32: operands must be 16-byte aligned");
  mr::EpiDev e;
  const int rc = mr::make_epi(epi, N, false, &e);
  if (rc != MR_OK) return rc;
  if (M == 0) return MR_OK;
  // more than 16 rows: tiles on f32 MFMAs (the weights cross HBM once per 128 rows)
  if (M > 16) {
    const int rt = mr::w8gemm_launch(x, ldx, b, w_scale, w_f16, k_pad, n_pad, M, N, K, e, static_cast<hipStream_t>(stream));
    if (rt != MR_EUNSUPPORTED) return rt;
  }
  MR_REQUIRE(M <= 8 * 65535, "mr_w8_matmul_f32: M=%lld rows need K and ldx multiples of 4 (tiled kernel)",
             (long long)M);
  mr::GemvArgs g = {};
  g.b = b;
  g.lda = K;   // activation columns (the kernel stops at K)
  g.k_pad = static_cast<int32_t>(k_pad);
  g.n_pad = static_cast<int32_t>(n_pad);
  g.N = static_cast<int32_t>(N);
  g.M = static_cast<int32_t>(M);
  const int mr_rows = static_cast<int>(M < 8 ? M : 8);   // rows per block
  int lpc = 64;
  while (lpc > 4 && k_pad / 16 < 4 * lpc) lpc >>= 1;
  while (lpc < mr_rows * mr::GEMV_CPW) lpc <<= 1;
  g.lpc = lpc;
  const int64_t groups = (N + mr::GEMV_CPW - 1) / mr::GEMV_CPW;
  const int mr_blk = mr_rows == 1 ? 1 : mr_rows == 2 ? 2 : mr_rows <= 4 ? 4 : 8;
  const dim3 grid(static_cast<unsigned>((groups * lpc + 255) / 256), static_cast<unsigned>((M + mr_blk - 1) / mr_blk));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (mr_blk == 1)
    hipLaunchKernelGGL(mr::w8gemv_kernel<1>, grid, dim3(256), 0, s, x, ldx, w_scale, w_f16, g, e);
  else if (mr_blk == 2)
    hipLaunchKernelGGL(mr::w8gemv_kernel<2>, grid, dim3(256), 0, s, x, ldx, w_scale, w_f16, g, e);
  else if (mr_blk == 4)
    hipLaunchKernelGGL(mr::w8gemv_kernel<4>, grid, dim3(256), 0, s, x, ldx, w_scale, w_f16, g, e);
  else
    hipLaunchKernelGGL(mr::w8gemv_kernel<8>, grid, dim3(256), 0, s, x, ldx, w_scale, w_f16, g, e);
  MR_LAUNCH_CHECK("w8gemv");
  return MR_OK;
}
