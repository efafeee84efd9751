// The float ops of a transformer decode step around its W8A8 projections
// (examples/gpt_text.mira's `generate` body): layer normalisation, the f32
// attention matmuls, softmax, and the transposes and concatenations that
// reshape the key/value cache.  All operate on C-order (row-major) tensors.
//
// layernorm, transpose and concat reproduce mira/ops.py bit for bit: layernorm
// is NumPy's pairwise f32 sums and single IEEE operations.  softmax and the f32
// batched matmul do not: exp (libm) and BLAS's summation order cannot be
// matched, so the rocm target runs them only when asked for approximate f32
// ops, and their results agree with NumPy's to f32 rounding.
#include "mr_common.hpp"
#include "np_sum.hpp"

namespace mr {

// ---------------------------------------------------------------- layernorm

// mira/ops.py:356-360 on [rows, d]: mu = mean(x), var = mean((x - mu)^2),
// y = (x - mu) / sqrt(var + eps) * g + b, rounded to f16 when out_f16, and the
// optional int8 copy clip(rint(y / xs), +-127) of the next q-op's input.
// NumPy's mean is an add-reduce seeded with +0 over the pairwise f32 sum, then
// the division of that f32 sum by the count in double precision, rounded back
// to f32; eps is added in f32; the square root and the division are IEEE.  The
// squared deviations are recomputed inside the sum, so no workspace is needed.
// One wave per row: rows of at most 128 elements split the pairwise
// accumulators over lanes, longer rows run the pairwise recursion on lane 0.
__global__ void __launch_bounds__(64) layernorm_kernel(const float* __restrict__ x, int32_t d,
                                                       const float* __restrict__ g, const float* __restrict__ b,
                                                       float eps, int out_f16, float* __restrict__ y,
                                                       int8_t* __restrict__ yq, int64_t ldq, float xs) {
  const int64_t r = blockIdx.x;
  const int lane = threadIdx.x;
  const float* xr = x + r * d;
  float mu, sd;
  layernorm_row_stats([=](int64_t i) { return xr[i]; }, d, lane, eps, mu, sd);
  for (int i = lane; i < d; i += 64) {
    float v = layernorm_value(xr[i], mu, sd, g[i], b[i]);
    if (out_f16) v = round_f16(v);
    if (y) y[r * d + i] = v;
    if (yq) yq[r * ldq + i] = quantize_one(v, xs);
  }
}

// ---------------------------------------------------------------- softmax (approximate)

// mira/ops.py:308-311 over the last axis of [rows, n]: e = exp(x - max), e / sum(e).
// One wave per row; the maximum is exact, exp and the sum's order are not NumPy's.
__global__ void __launch_bounds__(256) softmax_kernel(const float* __restrict__ x, int64_t rows, int32_t n,
                                                     int out_f16, float* __restrict__ y) {
  const int64_t r = blockIdx.x * int64_t(blockDim.x / 64) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;
  const float* xr = x + r * n;
  float* yr = y + r * n;
  float m = -__builtin_inff();
  for (int i = lane; i < n; i += 64) m = np_maximum(m, xr[i]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = np_maximum(m, __shfl_xor(m, o));
  float s = 0.0f;
  for (int i = lane; i < n; i += 64) {
    const float e = expf(__fsub_rn(xr[i], m));
    yr[i] = e;
    s = __fadd_rn(s, e);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s = __fadd_rn(s, __shfl_xor(s, o));
  for (int i = lane; i < n; i += 64) {
    const float v = __fdiv_rn(yr[i], s);
    yr[i] = out_f16 ? round_f16(v) : v;
  }
}

// ---------------------------------------------------------------- batched f32 matmul (approximate)

// mira/ops.py:217-219 for float operands: c[bt] = a[bt] @ w[bt] with the batch
// index bt broadcast onto each operand through its own batch strides (sa, sw;
// 0 for a broadcast dimension), then the epilogue on the [batches * M, N] result
// (C order).  Each operand is a strided view: a[bt][m][k] sits at
// a + oa(bt) + m * sam + k * sak and w[bt][k][n] at w + ow(bt) + k * swk + n * swn,
// so transposed operands are read in place.  f32 multiply-adds in k order per
// partial sum: the result is not NumPy/BLAS's to the last bit.
struct BmmArgs {
  const float* a;
  const float* w;
  int64_t batches, M, N, K;
  int32_t nb;                 // batch dimensions (<= 4)
  int64_t bdim[4];            // batch extents, outermost first
  int64_t sa[4], sw[4];       // element strides of each batch dimension in a and w
  int64_t sam, sak, swk, swn; // element strides of a's M and K axes and of w's K and N axes
};

__device__ inline void bmm_offsets(const BmmArgs& p, int64_t bt, int64_t& oa, int64_t& ow) {
  oa = 0;
  ow = 0;
  for (int i = p.nb - 1; i >= 0; --i) {
    const int64_t q = bt % p.bdim[i];
    bt /= p.bdim[i];
    oa += q * p.sa[i];
    ow += q * p.sw[i];
  }
}

// One wave per (output row, block of NB = 2^nb_log2 columns): lane = kg * NB + j
// computes column j of the block over k = kg, kg + KG, ... (KG = 64 / NB k-groups),
// and log2(KG) butterfly steps add the k-groups.  The host picks NB so that
// consecutive lanes read consecutive floats of w: along n when w's n axis is
// contiguous, along k when its k axis is (the scores of attention read the key
// cache that way).  Columns past N and lanes past K contribute nothing.
__global__ void __launch_bounds__(256) bmm_f32_kernel(const BmmArgs p, const EpiDev e, int nb_log2,
                                                      int64_t jobs) {
  const int lane = threadIdx.x & 63;
  const int NB = 1 << nb_log2;
  const int KG = 64 >> nb_log2;
  const int j = lane & (NB - 1);
  const int kg = lane >> nb_log2;
  const int64_t nblocks = (p.N + NB - 1) / NB;
  for (int64_t job = blockIdx.x * int64_t(blockDim.x / 64) + (threadIdx.x >> 6); job < jobs;
       job += int64_t(gridDim.x) * (blockDim.x / 64)) {
    const int64_t row = job / nblocks;
    const int64_t n = (job - row * nblocks) * NB + j;
    const bool valid = n < p.N;
    const int64_t m = row % p.M;
    int64_t oa, ow;
    bmm_offsets(p, row / p.M, oa, ow);
    const float* ar = p.a + oa + m * p.sam;
    const float* wc = p.w + ow + (valid ? n : 0) * p.swn;
    float acc = 0.0f;
    if (valid) {
      // eight loads in flight before their multiply-adds, which stay in k order
      int64_t k = kg;
      for (; k + 7 * KG < p.K; k += 8 * KG) {
        float av[8], wv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          av[u] = ar[(k + u * KG) * p.sak];
          wv[u] = wc[(k + u * KG) * p.swk];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) acc = fmaf(av[u], wv[u], acc);
      }
      for (; k < p.K; k += KG) acc = fmaf(ar[k * p.sak], wc[k * p.swk], acc);
    }
    for (int o = NB; o < 64; o <<= 1) acc = __fadd_rn(acc, __shfl_xor(acc, o));
    if (kg == 0 && valid) {
      const float y = epi_steps(e, acc, row, n);
      if (e.out_f32) e.out_f32[row * e.ldo + n] = y;
      if (e.out_i8) e.out_i8[row * e.ldq + n] = quantize_rcp(y, e.out_rxs);
    }
  }
}

// ---------------------------------------------------------------- transpose / concat

// mira/ops.py:375: y = ascontiguousarray(transpose(x, perm)) for rank <= 4
// (shapes padded with leading 1s to rank 4; perm over the padded axes).
struct PermArgs {
  int64_t oshape[4];    // output extents
  int64_t istride[4];   // input element stride of the axis each output axis reads
};

__global__ void __launch_bounds__(256) transpose4_kernel(const float* __restrict__ x, const PermArgs p,
                                                         float* __restrict__ y) {
  const int64_t total = p.oshape[0] * p.oshape[1] * p.oshape[2] * p.oshape[3];
  for (int64_t t = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; t < total; t += int64_t(gridDim.x) * blockDim.x) {
    int64_t rest = t, off = 0;
#pragma unroll
    for (int i = 3; i >= 0; --i) {
      off += (rest % p.oshape[i]) * p.istride[i];
      rest /= p.oshape[i];
    }
    y[t] = x[off];
  }
}

// One operand of mira/ops.py:402 concatenate: x viewed as [outer, inner] rows
// lands in y's [outer, ld] rows at column offset `at`.
__global__ void __launch_bounds__(256) copy_rows_kernel(const float* __restrict__ x, int64_t outer, int64_t inner,
                                                        float* __restrict__ y, int64_t ld, int64_t at) {
  const int64_t total = outer * inner;
  for (int64_t t = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; t < total; t += int64_t(gridDim.x) * blockDim.x) {
    const int64_t r = t / inner;
    y[r * ld + at + (t - r * inner)] = x[t];
  }
}

// ---------------------------------------------------------------- fused decode attention (approximate)

// One attention of a decode step, the ops MIRA's program spells out one by one (matmul of the
// query with the transposed keys, the scale and the mask, softmax over the keys, matmul with the
// values; examples/gpt_text.mira, mira/ops.py:217-219, 310-313): the keys and values are a
// cache of T rows joined by the step's own row (slot T), read in place.  Approximate like the
// ops it replaces: expf and f32 multiply-adds in key order, within f32 rounding of NumPy.
struct AttnArgs {
  const float* q;            // [B, H*HD] rows (row stride ldq)
  int64_t ldq;
  const float* kc;           // caches [B, T, c_ld]: row j of sequence b at b * c_bs + j * c_ld
  const float* vc;
  int64_t c_ld, c_bs;
  const float* kn;           // the step's key / value rows [B, ...] (row strides ldkn, ldvn)
  const float* vn;
  int64_t ldkn, ldvn;
  const float* mask;         // [T + 1], the same for every sequence and head
  float scale;
  int32_t B, H, T;
  float* out;                // [B, H*HD] (row stride ldo), optional
  int64_t ldo;
  int8_t* out_i8;            // its int8 copy clip(rint(y / xs)), optional
  int64_t ldq8;
  float xs;
};

// One wave per (sequence, head); lane l takes keys l, l + 64, ...: their scores stay in
// registers (JMAX * 64 keys at most), the max and the sum of exponentials are butterflies,
// and each lane's share of the context product is summed over the lanes at the end.
template <int HD, int JMAX>
__global__ void __launch_bounds__(256) attention_decode_kernel(const AttnArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t job = blockIdx.x * int64_t(blockDim.x / 64) + (threadIdx.x >> 6);
  if (job >= int64_t(a.B) * a.H) return;
  const int64_t b = job / a.H;
  const int h = static_cast<int>(job - b * a.H);
  float qv[HD];
#pragma unroll
  for (int d = 0; d < HD; d += 4) {
    const float4 v = *reinterpret_cast<const float4*>(a.q + b * a.ldq + h * HD + d);
    qv[d] = v.x; qv[d + 1] = v.y; qv[d + 2] = v.z; qv[d + 3] = v.w;
  }
  const int nj = a.T + 1;
  float sc[JMAX];
  float m = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < JMAX; ++i) {
    const int j = lane + 64 * i;
    sc[i] = -__builtin_inff();
    if (j < nj) {
      const float* kr = j < a.T ? a.kc + b * a.c_bs + int64_t(j) * a.c_ld + h * HD : a.kn + b * a.ldkn + h * HD;
      float acc = 0.0f;
#pragma unroll
      for (int d = 0; d < HD; d += 4) {
        const float4 k = *reinterpret_cast<const float4*>(kr + d);
        acc = fmaf(qv[d], k.x, acc);
        acc = fmaf(qv[d + 1], k.y, acc);
        acc = fmaf(qv[d + 2], k.z, acc);
        acc = fmaf(qv[d + 3], k.w, acc);
      }
      sc[i] = __fadd_rn(__fmul_rn(acc, a.scale), a.mask[j]);
      m = np_maximum(m, sc[i]);
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = np_maximum(m, __shfl_xor(m, o));
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < JMAX; ++i) {
    const int j = lane + 64 * i;
    if (j < nj) {
      sc[i] = expf(__fsub_rn(sc[i], m));
      sum = __fadd_rn(sum, sc[i]);
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) sum = __fadd_rn(sum, __shfl_xor(sum, o));
  float ov[HD];
#pragma unroll
  for (int d = 0; d < HD; ++d) ov[d] = 0.0f;
#pragma unroll
  for (int i = 0; i < JMAX; ++i) {
    const int j = lane + 64 * i;
    if (j < nj) {
      const float pj = __fdiv_rn(sc[i], sum);
      const float* vr = j < a.T ? a.vc + b * a.c_bs + int64_t(j) * a.c_ld + h * HD : a.vn + b * a.ldvn + h * HD;
#pragma unroll
      for (int d = 0; d < HD; d += 4) {
        const float4 v = *reinterpret_cast<const float4*>(vr + d);
        ov[d] = fmaf(pj, v.x, ov[d]);
        ov[d + 1] = fmaf(pj, v.y, ov[d + 1]);
        ov[d + 2] = fmaf(pj, v.z, ov[d + 2]);
        ov[d + 3] = fmaf(pj, v.w, ov[d + 3]);
      }
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1)
#pragma unroll
    for (int d = 0; d < HD; ++d) ov[d] = __fadd_rn(ov[d], __shfl_xor(ov[d], o));
  if (lane != 0) return;
  if (a.out) {
#pragma unroll
    for (int d = 0; d < HD; d += 4)
      *reinterpret_cast<float4*>(a.out + b * a.ldo + h * HD + d) = make_float4(ov[d], ov[d + 1], ov[d + 2], ov[d + 3]);
  }
  if (a.out_i8) {
#pragma unroll
    for (int d = 0; d < HD; d += 4) {
      uint32_t w = 0;
#pragma unroll
      for (int c = 0; c < 4; ++c) w |= uint32_t(uint8_t(quantize_one(ov[d + c], a.xs))) << (8 * c);
      *reinterpret_cast<uint32_t*>(a.out_i8 + b * a.ldq8 + h * HD + d) = w;
    }
  }
}

// ---------------------------------------------------------------- the greedy decode loop's own state

// Start of a decode step at position t = *t_io (examples/gpt_text.mira:66-81, the body of
// `generate`'s loop): the input row of each sequence, emb[token t] + pos[t] (one f32 add, as
// NumPy adds the two gathered rows), and the step's mask over the T cache rows and the step's
// own row (0 for rows already written and for its own row, `neg` for the rest).  The position
// is latched into *t_cur for the step's end (decode_commit_kernel advances *t_io).  Token ids
// are clamped into [0, V) and t into [0, T) so no read leaves its table; the host keeps both
// in range.
__global__ void __launch_bounds__(256) decode_embed_kernel(const int32_t* __restrict__ tokens, int64_t ld_tok,
                                                           const int32_t* __restrict__ t_io, int32_t* t_cur,
                                                           const float* __restrict__ emb, int32_t V,
                                                           const float* __restrict__ pos, int32_t T, int32_t D,
                                                           float* __restrict__ h, int64_t B, float* __restrict__ mask,
                                                           float neg) {
  const int t = min(max(t_io[0], 0), T - 1);
  const int64_t row = blockIdx.x;
  if (row < B) {
    const int tok = min(max(tokens[row * ld_tok + t], 0), V - 1);
    for (int d = threadIdx.x; d < D; d += blockDim.x)
      h[row * D + d] = __fadd_rn(emb[int64_t(tok) * D + d], pos[int64_t(t) * D + d]);
    return;
  }
  for (int j = threadIdx.x; j <= T; j += blockDim.x) mask[j] = (j < t || j == T) ? 0.0f : neg;
  if (threadIdx.x == 0) t_cur[0] = t;
}

struct CommitArgs {
  int32_t n;                  // key/value rows to store (<= MR_DECODE_MAX_CACHES)
  const float* row[MR_DECODE_MAX_CACHES];
  int64_t ld_row[MR_DECODE_MAX_CACHES];
  float* cache[MR_DECODE_MAX_CACHES];
  int64_t c_ld, c_bs;         // cache row stride and per-sequence stride (elements)
  int32_t D;                  // elements per row
};

// NumPy's argmax order: a NaN beats every number and the first NaN wins; among numbers the
// larger wins, and the smaller index on a tie.
__device__ inline bool argmax_better(float v, int i, float bv, int bi) {
  const bool vn = v != v, bn = bv != bv;
  if (vn || bn) return vn && (!bn || i < bi);
  return v > bv || (v == bv && i < bi);
}

// End of the step at position t = *t_cur: each sequence's key/value rows go to cache row t,
// the next token is the argmax of its logits once the prompt is consumed (t + 1 >= prompt_len,
// else the prompt's own token stays), and *t_io advances to t + 1.  One block per sequence.
__global__ void __launch_bounds__(64) decode_commit_kernel(const float* __restrict__ logits, int64_t ldl, int32_t V,
                                                           const CommitArgs c, int32_t* tokens, int64_t ld_tok,
                                                           int32_t* t_io, const int32_t* __restrict__ t_cur,
                                                           int32_t prompt_len, int32_t T) {
  const int64_t b = blockIdx.x;
  const int t = min(max(t_cur[0], 0), T - 2);
  const int lane = threadIdx.x;
  float bv = -__builtin_inff();
  int bi = 0x7fffffff;
  for (int i = lane; i < V; i += 64) {
    const float v = logits[b * ldl + i];
    if (argmax_better(v, i, bv, bi)) { bv = v; bi = i; }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    if (argmax_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  for (int k = 0; k < c.n; ++k)
    for (int d = lane; d < c.D; d += 64) c.cache[k][b * c.c_bs + int64_t(t) * c.c_ld + d] = c.row[k][b * c.ld_row[k] + d];
  if (lane == 0) {
    if (t + 1 >= prompt_len) tokens[b * ld_tok + t + 1] = bi;
    if (b == 0) t_io[0] = t + 1;
  }
}

static unsigned grid_1d(int64_t total, int block) {
  int64_t g = (total + block - 1) / block;
  const int64_t cap = int64_t(device_cu_count()) * 32;
  return static_cast<unsigned>(g < 1 ? 1 : (g > cap ? cap : g));
}

}  // namespace mr

extern "C" {

int mr_layernorm_f32(const float* x, int64_t rows, int32_t d, const float* gamma, const float* beta, float eps,
                     int32_t out_f16, float* y, int8_t* yq, int64_t ldq, float xs, void* stream) {
  MR_REQUIRE(x && gamma && beta, "mr_layernorm_f32: NULL operand");
  MR_REQUIRE(y || yq, "mr_layernorm_f32: no output");
  MR_REQUIRE(rows >= 0 && d > 0, "mr_layernorm_f32: bad shape [%lld, %d]", (long long)rows, d);
  if (yq) MR_REQUIRE(ldq >= d && xs > 0.0f, "mr_layernorm_f32: int8 output needs ldq >= d and xs > 0");
  if (rows == 0) return MR_OK;
  MR_REQUIRE(rows < (int64_t(1) << 31), "mr_layernorm_f32: too many rows");
  hipLaunchKernelGGL(mr::layernorm_kernel, dim3(static_cast<unsigned>(rows)), dim3(64), 0,
                     static_cast<hipStream_t>(stream), x, d, gamma, beta, eps, out_f16, y, yq, ldq, xs);
  MR_LAUNCH_CHECK("layernorm");
  return MR_OK;
}

int mr_softmax_f32(const float* x, int64_t rows, int32_t n, int32_t out_f16, float* y, void* stream) {
  MR_REQUIRE(x && y, "mr_softmax_f32: NULL pointer");
  MR_REQUIRE(rows >= 0 && n > 0, "mr_softmax_f32: bad shape");
  if (rows == 0) return MR_OK;
  const int64_t blocks = (rows + 3) / 4;
  MR_REQUIRE(blocks < (int64_t(1) << 31), "mr_softmax_f32: too many rows");
  hipLaunchKernelGGL(mr::softmax_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, rows, n, out_f16, y);
  MR_LAUNCH_CHECK("softmax");
  return MR_OK;
}

int mr_bmm_f32(const float* a, const float* w, int32_t nb, const int64_t* bdim, const int64_t* sa, const int64_t* sw,
               const int64_t* mk_strides, int64_t M, int64_t N, int64_t K, const mr_epilogue* epi, void* stream) {
  MR_REQUIRE(a && w && mk_strides, "mr_bmm_f32: NULL operand");
  MR_REQUIRE(nb >= 0 && nb <= 4 && (nb == 0 || (bdim && sa && sw)), "mr_bmm_f32: 0..4 batch dimensions");
  MR_REQUIRE(M > 0 && N > 0 && K > 0, "mr_bmm_f32: bad sizes");
  mr::BmmArgs p = {};
  p.a = a;
  p.w = w;
  p.M = M;
  p.N = N;
  p.K = K;
  p.nb = nb;
  p.sam = mk_strides[0];
  p.sak = mk_strides[1];
  p.swk = mk_strides[2];
  p.swn = mk_strides[3];
  MR_REQUIRE(p.sam >= 0 && p.sak >= 0 && p.swk >= 0 && p.swn >= 0, "mr_bmm_f32: negative stride");
  p.batches = 1;
  for (int i = 0; i < nb; ++i) {
    MR_REQUIRE(bdim[i] > 0 && sa[i] >= 0 && sw[i] >= 0, "mr_bmm_f32: bad batch dimension %d", i);
    p.bdim[i] = bdim[i];
    p.sa[i] = sa[i];
    p.sw[i] = sw[i];
    p.batches *= bdim[i];
  }
  mr::EpiDev e;
  const int rc = mr::make_epi(epi, N, false, &e);
  if (rc != MR_OK) return rc;
  MR_REQUIRE(!e.out_acc, "mr_bmm_f32: no int32 accumulators");
  // lanes along k when w's k axis is the contiguous one and long enough to give every
  // lane work, else along n
  auto log2_ceil = [](int64_t v) { int l = 0; while ((int64_t(1) << l) < v && l < 6) ++l; return l; };
  const bool along_k = p.swk == 1 && p.swn != 1 && K >= 64;
  int nb_log2 = along_k ? 6 - log2_ceil(K) : log2_ceil(N);
  // along n with too few rows to fill the GPU (a decode step's [1, K] x [K, N]), each lane's
  // serial k loop is the latency: narrow the column block until a lane walks at most 8 k
  // (one batch of loads in flight), down to 4 columns per wave
  if (!along_k) {
    const int64_t rows = p.batches * M;
    while (nb_log2 > 2 && rows * ((N + (int64_t(1) << nb_log2) - 1) >> nb_log2) < 1024 &&
           (K << nb_log2) > 64 * 8)
      --nb_log2;
  }
  const int64_t jobs = p.batches * M * ((N + (int64_t(1) << nb_log2) - 1) >> nb_log2);
  hipLaunchKernelGGL(mr::bmm_f32_kernel, dim3(mr::grid_1d(jobs * 64, 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), p, e, nb_log2, jobs);
  MR_LAUNCH_CHECK("bmm_f32");
  return MR_OK;
}

int mr_transpose_f32(const float* x, int32_t rank, const int64_t* shape, const int32_t* perm, float* y, void* stream) {
  MR_REQUIRE(x && y && shape && perm, "mr_transpose_f32: NULL argument");
  MR_REQUIRE(rank >= 1 && rank <= 4, "mr_transpose_f32: rank %d not in 1..4", rank);
  MR_REQUIRE(x != y, "mr_transpose_f32: in place is not supported");
  int64_t s4[4], st4[4];
  const int pad = 4 - rank;
  for (int i = 0; i < 4; ++i) s4[i] = i < pad ? 1 : shape[i - pad];
  st4[3] = 1;
  for (int i = 2; i >= 0; --i) st4[i] = st4[i + 1] * s4[i + 1];
  mr::PermArgs p = {};
  bool seen[4] = {false, false, false, false};
  for (int i = 0; i < 4; ++i) {
    const int src = i < pad ? i : pad + perm[i - pad];
    MR_REQUIRE(src >= 0 && src < 4 && !seen[src] && (i < pad) == (src < pad), "mr_transpose_f32: bad perm");
    seen[src] = true;
    p.oshape[i] = s4[src];
    p.istride[i] = st4[src];
  }
  const int64_t total = s4[0] * s4[1] * s4[2] * s4[3];
  if (total == 0) return MR_OK;
  hipLaunchKernelGGL(mr::transpose4_kernel, dim3(mr::grid_1d(total, 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, p, y);
  MR_LAUNCH_CHECK("transpose");
  return MR_OK;
}

int mr_copy_rows_f32(const float* x, int64_t outer, int64_t inner, float* y, int64_t ld, int64_t at, void* stream) {
  MR_REQUIRE(outer >= 0 && inner >= 0 && at >= 0 && at + inner <= ld, "mr_copy_rows_f32: bad extents");
  if (outer * inner == 0) return MR_OK;      // an empty operand (its pointer may be NULL)
  MR_REQUIRE(x && y, "mr_copy_rows_f32: NULL pointer");
  hipLaunchKernelGGL(mr::copy_rows_kernel, dim3(mr::grid_1d(outer * inner, 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, outer, inner, y, ld, at);
  MR_LAUNCH_CHECK("copy_rows");
  return MR_OK;
}

int mr_attention_decode_f32(const float* q, int64_t ldq, const float* k_cache, const float* v_cache, int64_t c_ld,
                            int64_t c_bs, const float* k_new, int64_t ld_kn, const float* v_new, int64_t ld_vn,
                            const float* mask,
                            float scale, int64_t B, int32_t H, int32_t hd, int32_t T, float* out, int64_t ldo,
                            int8_t* out_i8, int64_t ldq8, float xs, void* stream) {
  MR_REQUIRE(q && k_new && v_new && mask && (T == 0 || (k_cache && v_cache)), "mr_attention_decode_f32: NULL operand");
  MR_REQUIRE(out || out_i8, "mr_attention_decode_f32: no output");
  MR_REQUIRE(hd == 16 || hd == 32 || hd == 64, "mr_attention_decode_f32: head width %d not in {16, 32, 64}", hd);
  MR_REQUIRE(B >= 0 && H > 0 && T >= 0 && T + 1 <= 1024, "mr_attention_decode_f32: needs T + 1 <= 1024 keys");
  const int64_t w = int64_t(H) * hd;
  MR_REQUIRE(ldq >= w && ld_kn >= w && ld_vn >= w && c_ld >= w && c_bs >= int64_t(T) * c_ld,
             "mr_attention_decode_f32: bad strides");
  MR_REQUIRE(ldq % 4 == 0 && ld_kn % 4 == 0 && ld_vn % 4 == 0 && c_ld % 4 == 0 && c_bs % 4 == 0,
             "mr_attention_decode_f32: row strides "
             "must be multiples of 4 floats");
  auto al16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  MR_REQUIRE(al16(q) && al16(k_new) && al16(v_new) && (T == 0 || (al16(k_cache) && al16(v_cache))),
             "mr_attention_decode_f32: operands must be 16-byte aligned");
  if (out) MR_REQUIRE(ldo >= w && ldo % 4 == 0 && al16(out), "mr_attention_decode_f32: bad f32 output");
  if (out_i8) MR_REQUIRE(ldq8 >= w && ldq8 % 4 == 0 && reinterpret_cast<uintptr_t>(out_i8) % 4 == 0 && xs > 0.0f,
                         "mr_attention_decode_f32: bad int8 output");
  if (B == 0) return MR_OK;
  mr::AttnArgs a = {q, ldq, k_cache, v_cache, c_ld, c_bs, k_new, v_new, ld_kn, ld_vn, mask, scale,
                    static_cast<int32_t>(B), H, T, out, ldo, out_i8, ldq8, xs};
  MR_REQUIRE(B * H < (int64_t(1) << 31) && B < (int64_t(1) << 31), "mr_attention_decode_f32: too many heads");
  const dim3 grid(static_cast<unsigned>((B * H + 3) / 4)), block(256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int jmax = (T + 1 + 63) / 64;
#define MR_ATTN(HDV, JM) hipLaunchKernelGGL((mr::attention_decode_kernel<HDV, JM>), grid, block, 0, s, a)
  if (hd == 16) { if (jmax <= 5) MR_ATTN(16, 5); else MR_ATTN(16, 16); }
  else if (hd == 32) { if (jmax <= 5) MR_ATTN(32, 5); else MR_ATTN(32, 16); }
  else { if (jmax <= 5) MR_ATTN(64, 5); else MR_ATTN(64, 16); }
#undef MR_ATTN
  MR_LAUNCH_CHECK("attention_decode");
  return MR_OK;
}

int mr_decode_embed(const int32_t* tokens, int64_t ld_tok, const int32_t* t_io, int32_t* t_cur, const float* emb,
                    int32_t V, const float* pos, int32_t T, int32_t D, float* h, int64_t B, float* mask, float neg,
                    void* stream) {
  MR_REQUIRE(tokens && t_io && t_cur && emb && pos && h && mask, "mr_decode_embed: NULL argument");
  MR_REQUIRE(V > 0 && T > 0 && D > 0 && B >= 0 && ld_tok >= T, "mr_decode_embed: bad sizes");
  MR_REQUIRE(B < (int64_t(1) << 31), "mr_decode_embed: too many sequences");
  hipLaunchKernelGGL(mr::decode_embed_kernel, dim3(static_cast<unsigned>(B + 1)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), tokens, ld_tok, t_io, t_cur, emb, V, pos, T, D, h, B, mask, neg);
  MR_LAUNCH_CHECK("decode_embed");
  return MR_OK;
}

int mr_decode_commit(const float* logits, int64_t ldl, int32_t V, int32_t n_caches, const float* const* rows,
                     const int64_t* ld_rows, float* const* caches, int64_t c_ld, int64_t c_bs, int32_t D,
                     int32_t* tokens, int64_t ld_tok, int32_t* t_io, const int32_t* t_cur, int32_t prompt_len,
                     int32_t T, int64_t B, void* stream) {
  MR_REQUIRE(logits && tokens && t_io && t_cur, "mr_decode_commit: NULL argument");
  MR_REQUIRE(V > 0 && ldl >= V && T >= 2 && ld_tok >= T && B >= 0 && D >= 0, "mr_decode_commit: bad sizes");
  MR_REQUIRE(n_caches >= 0 && n_caches <= MR_DECODE_MAX_CACHES && (n_caches == 0 || (rows && ld_rows && caches)),
             "mr_decode_commit: 0..%d cache rows", MR_DECODE_MAX_CACHES);
  MR_REQUIRE(c_ld >= D && c_bs >= (int64_t(T) - 1) * c_ld + D, "mr_decode_commit: bad cache strides");
  MR_REQUIRE(B < (int64_t(1) << 31), "mr_decode_commit: too many sequences");
  mr::CommitArgs c = {};
  c.n = n_caches;
  for (int k = 0; k < n_caches; ++k) {
    MR_REQUIRE(rows[k] && caches[k] && ld_rows[k] >= D, "mr_decode_commit: bad cache row %d", k);
    c.row[k] = rows[k];
    c.ld_row[k] = ld_rows[k];
    c.cache[k] = caches[k];
  }
  c.c_ld = c_ld;
  c.c_bs = c_bs;
  c.D = D;
  if (B == 0) return MR_OK;
  hipLaunchKernelGGL(mr::decode_commit_kernel, dim3(static_cast<unsigned>(B)), dim3(64), 0,
                     static_cast<hipStream_t>(stream), logits, ldl, V, c, tokens, ld_tok, t_io, t_cur, prompt_len, T);
  MR_LAUNCH_CHECK("decode_commit");
  return MR_OK;
}

}  // extern "C"
