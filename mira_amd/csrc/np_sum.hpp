// NumPy's float32 pairwise summation, shared by every kernel that reproduces
// an f32 add-reduce (np.sum / np.mean along an axis).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mr {

// NumPy's float32 pairwise summation (numpy/_core/src/umath/loops_utils.h.src,
// @TYPE@_pairwise_sum, PW_BLOCKSIZE 128) of the n values elem(0..n), where
// elem(i) loads (or computes) the i-th summand.  A block of fewer than 8 values
// is summed in order from -0.0; a block of 8..128 values runs 8 interleaved
// accumulators, combines them as ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)) and adds
// the n % 8 trailing values in order.
template <class Elem>
__device__ inline float pairwise_block_of(Elem elem, int64_t off, int64_t n) {
  if (n < 8) {
    float res = -0.0f;
    for (int64_t i = 0; i < n; ++i) res = __fadd_rn(res, elem(off + i));
    return res;
  }
  float r[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = elem(off + j);
  int64_t i = 8;
  for (; i < n - (n % 8); i += 8) {
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = __fadd_rn(r[j], elem(off + i + j));
  }
  float res = __fadd_rn(__fadd_rn(__fadd_rn(r[0], r[1]), __fadd_rn(r[2], r[3])),
                        __fadd_rn(__fadd_rn(r[4], r[5]), __fadd_rn(r[6], r[7])));
  for (; i < n; ++i) res = __fadd_rn(res, elem(off + i));
  return res;
}

// Above 128 values NumPy splits at n/2 rounded down to a multiple of 8 and
// adds the two halves' sums.  The recursion runs with an explicit stack; its
// depth is about log2(n / 128) + 1, so 40 levels cover n < 2^46.
template <class Elem>
__device__ inline float pairwise_sum_of(Elem elem, int64_t n) {
  if (n <= 128) return pairwise_block_of(elem, 0, n);
  int64_t off[40], cnt[40];
  float left[40];
  int state[40];
  int sp = 0;
  off[0] = 0;
  cnt[0] = n;
  state[0] = 0;
  float ret = 0.0f;
  while (true) {
    if (cnt[sp] <= 128) {
      ret = pairwise_block_of(elem, off[sp], cnt[sp]);
      --sp;
      // unwind: finished children return into their parents
      while (sp >= 0) {
        if (state[sp] == 0) {
          left[sp] = ret;
          state[sp] = 1;
          int64_t n2 = cnt[sp] / 2;
          n2 -= n2 % 8;
          off[sp + 1] = off[sp] + n2;
          cnt[sp + 1] = cnt[sp] - n2;
          state[sp + 1] = 0;
          ++sp;
          break;
        }
        ret = __fadd_rn(left[sp], ret);
        --sp;
      }
      if (sp < 0) return ret;
      continue;
    }
    int64_t n2 = cnt[sp] / 2;
    n2 -= n2 % 8;
    state[sp] = 0;
    off[sp + 1] = off[sp];
    cnt[sp + 1] = n2;
    state[sp + 1] = 0;
    ++sp;
  }
}

// The pairwise sum of n values spaced `stride` apart in memory.
__device__ inline float pairwise_sum(const float* a, int64_t n, int64_t stride) {
  return pairwise_sum_of([=](int64_t i) { return a[i * stride]; }, n);
}

// The same sum computed by one 64-lane wave, for n <= 128 (a single block):
// lane j < 8 runs accumulator r[j] over elem(j), elem(j + 8), ... in order, the
// combine tree is three butterfly steps (additions commute exactly, so lane 0
// ends with ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7))), and lane 0 adds the tail.
// Every lane of the wave calls it; every lane gets the result.
template <class Elem>
__device__ inline float wave_pairwise_block(Elem elem, int n, int lane) {
  float res;
  if (n < 8) {
    res = -0.0f;
    if (lane == 0)
      for (int i = 0; i < n; ++i) res = __fadd_rn(res, elem(i));
  } else {
    const int body = n - n % 8;
    float r = 0.0f;
    if (lane < 8) {
      r = elem(lane);
      for (int i = lane + 8; i < body; i += 8) r = __fadd_rn(r, elem(i));
    }
    r = __fadd_rn(r, __shfl_xor(r, 1));
    r = __fadd_rn(r, __shfl_xor(r, 2));
    r = __fadd_rn(r, __shfl_xor(r, 4));
    res = r;
    if (lane == 0)
      for (int i = body; i < n; ++i) res = __fadd_rn(res, elem(i));
  }
  return __shfl(res, 0);
}

// ---------------------------------------------------------------- layer normalisation of one row

// Correctly rounded f32 square root (NumPy's np.sqrt), whatever the compiler lowers sqrtf to
// (clang's __fsqrt_rn is the hardware approximation, within 1 ulp).  Rounding to nearest
// picks s when the true root lies between the midpoints m- and m+ to s's neighbours; a
// midpoint has at most 25 significant bits, so m*m is exact in double and the comparison
// with v is exact (never equal: m*m has more bits than a float).  A faithful first guess
// is off by at most one ulp, so one correction suffices.
__device__ inline float sqrt_rn(float v) {
  float s = sqrtf(v);
  if (!(v > 0.0f) || !(v < __builtin_inff())) return s;     // +-0, negative, NaN, inf: exact cases
  const float dn = nextafterf(s, 0.0f), up = nextafterf(s, __builtin_inff());
  const double x = static_cast<double>(v);
  const double lo = 0.5 * (static_cast<double>(s) + static_cast<double>(dn));
  const double hi = 0.5 * (static_cast<double>(s) + static_cast<double>(up));
  if (__dmul_rn(lo, lo) > x) return dn;
  if (__dmul_rn(hi, hi) < x) return up;
  return s;
}

__device__ inline float mean_of_sum(float s, int d) {
  return static_cast<float>(__ddiv_rn(static_cast<double>(__fadd_rn(0.0f, s)), static_cast<double>(d)));
}

// mira/ops.py:356-360 for one row of d elements (read through elem) by one 64-lane wave:
// mu = mean(x), sd = sqrt(mean((x - mu)^2) + eps).  NumPy's mean is an add-reduce seeded
// with +0 over the pairwise f32 sum, then the division of that f32 sum by the count in
// double precision, rounded back to f32; eps is added in f32; the square root is IEEE.
// Rows of at most 128 elements split the pairwise accumulators over the lanes, longer rows
// run the pairwise recursion on lane 0.  Every lane ends with mu and sd.
template <class Elem>
__device__ inline void layernorm_row_stats(Elem elem, int d, int lane, float eps, float& mu, float& sd) {
  if (d <= 128) {
    mu = mean_of_sum(wave_pairwise_block(elem, d, lane), d);
  } else {
    float s = 0.0f;
    if (lane == 0) s = pairwise_sum_of(elem, d);
    mu = mean_of_sum(__shfl(s, 0), d);
  }
  const float m = mu;
  auto sq = [=](int64_t i) {
    const float t = __fsub_rn(elem(i), m);
    return __fmul_rn(t, t);
  };
  float var;
  if (d <= 128) {
    var = mean_of_sum(wave_pairwise_block(sq, d, lane), d);
  } else {
    float s = 0.0f;
    if (lane == 0) s = pairwise_sum_of(sq, d);
    var = mean_of_sum(__shfl(s, 0), d);
  }
  sd = sqrt_rn(__fadd_rn(var, eps));
}

// (x - mu) / sd * g + b, each operation rounded once (before any f16 rounding of the result)
__device__ inline float layernorm_value(float x, float mu, float sd, float g, float b) {
  return __fadd_rn(__fmul_rn(__fdiv_rn(__fsub_rn(x, mu), sd), g), b);
}

}  // namespace mr
