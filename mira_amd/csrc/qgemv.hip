// Small-M int8 matmul (decode-shaped qmatmul, mira/ops.py:616-620): M <= 8
// activation rows against packed weights (K-step-major: 64-byte slice kt of
// row n at (kt * n_pad + n) * 64).  With so few rows
// the work is reading the weights once (N*K bytes: 16 MiB per 4096x4096
// layer), so the kernel is a coalesced weight stream rather than MFMA tiles:
// a group of LPC lanes owns CPW output columns, each lane walks 16-byte
// chunks of those weight rows (a group reads LPC*16 contiguous bytes per
// row per load), multiplies them with the matching activation bytes by
// v_dot4 (4 exact int8 multiply-adds into int32), and the group reduces its
// partial sums with lane shuffles.  The dequant / epilogue / requant of each
// result element then runs on one lane (mira/ops.py:618, 192-199, 602-603).
#include "mr_common.hpp"

namespace mr {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int GEMV_CPW = 2;   // output columns per lane group

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
    for (int k16 = sub; k16 < chunks; k16 += lpc) {
      v4i w[GEMV_CPW];
#pragma unroll
      for (int c = 0; c < GEMV_CPW; ++c)
        w[c] = *reinterpret_cast<const v4i*>(brow[c] + (k16 >> 2) * kstep + (k16 & 3) * 16);
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
          for (int q = 0; q < 4; ++q) acc[m][c] = __builtin_amdgcn_sdot4(x[q], w[c][q], acc[m][c], false);
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
