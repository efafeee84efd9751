// Shared host/device helpers for libmira_rocm.so (gfx950).
//
// Numerics follow NumPy's float32 semantics as used by MIRA's golden model:
// every epilogue step is one correctly rounded IEEE-754 single operation
// (the library is built with -ffp-contract=off so nothing is fused), the
// activation quantizer divides (never multiplies by a reciprocal) and rounds
// half to even, and dequantization multiplies in double precision.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdarg>
#include <cstdio>

#include "../../include/mira_rocm.h"

namespace mr {

// ---------------------------------------------------------------- host errors

void set_error(const char* fmt, ...);
int device_cu_count();

}  // namespace mr

#define MR_REQUIRE(cond, ...)            \
  do {                                   \
    if (!(cond)) {                       \
      mr::set_error(__VA_ARGS__);        \
      return MR_EINVAL;                  \
    }                                    \
  } while (0)

#define MR_HIP_CHECK(call)                                                      \
  do {                                                                          \
    hipError_t e_ = (call);                                                     \
    if (e_ != hipSuccess) {                                                     \
      mr::set_error("%s failed: %s", #call, hipGetErrorString(e_));             \
      return MR_EHIP;                                                           \
    }                                                                           \
  } while (0)

// Launch-error check after a kernel launch.
#define MR_LAUNCH_CHECK(name)                                                   \
  do {                                                                          \
    hipError_t e_ = hipGetLastError();                                          \
    if (e_ != hipSuccess) {                                                     \
      mr::set_error("%s launch failed: %s", name, hipGetErrorString(e_));       \
      return MR_EHIP;                                                           \
    }                                                                           \
  } while (0)

namespace mr {

// ---------------------------------------------------------------- device numerics

// mira/ops.py:602-603: clip(round(f32(x) / f32(scale)), -127, 127).
// IEEE division (the build keeps -fhip-fp32-correctly-rounded-divide-sqrt),
// rintf is round-half-to-even (v_rndne_f32).  NaN input is outside the
// reference's defined behaviour (NumPy casts NaN to int64 as INT64_MIN); it
// maps to -127 here.
__device__ __forceinline__ int8_t quantize_one(float x, float xs) {
  float t = rintf(__fdiv_rn(x, xs));
  t = fminf(fmaxf(t, -127.0f), 127.0f);
  return static_cast<int8_t>(static_cast<int>(t));
}

// NumPy float32 maximum/minimum on x86: NaN in either operand propagates, and
// on equality (including +0 vs -0) the second operand is returned.
__device__ __forceinline__ float np_maximum(float a, float b) {
  if (a != a) return a;
  if (b != b) return b;
  return a > b ? a : b;
}
__device__ __forceinline__ float np_minimum(float a, float b) {
  if (a != a) return a;
  if (b != b) return b;
  return a < b ? a : b;
}

// One epilogue step (mira/ops.py:192-199): fn(acc, other), or fn(other, acc)
// when swapped.
__device__ __forceinline__ float epi_binary(int fn, float a, float b) {
  switch (fn) {
    case MR_EPI_ADD: return __fadd_rn(a, b);
    case MR_EPI_SUB: return __fsub_rn(a, b);
    case MR_EPI_MUL: return __fmul_rn(a, b);
    case MR_EPI_DIV: return __fdiv_rn(a, b);
    case MR_EPI_MAX: return np_maximum(a, b);
    case MR_EPI_MIN: return np_minimum(a, b);
    default: return a;
  }
}

// Device copy of mr_epilogue (passed by value as a kernel argument).
struct EpiStepDev {
  int32_t fn;
  int32_t swapped;
  int32_t mode;
  int32_t reserved;
  const float* ptr;
  int64_t ld;
};

struct EpiDev {
  int32_t n_steps;
  int32_t has_scale;
  EpiStepDev steps[MR_MAX_EPI];
  const double* scale;
  float* out_f32;
  int64_t ldo;
  int8_t* out_i8;
  int64_t ldq;
  float out_xs;
  int32_t reserved;
  int32_t* out_acc;
  int64_t ldacc;
};

// Apply the f32 epilogue steps to NV values of one column `col` at rows
// row[v] (callers clamp rows past the end to a valid row and skip their
// stores).  The step loop is unrolled with static indices so the descriptor
// stays in the kernel-argument segment (a dynamic index would copy it to
// scratch); the value loop is innermost so each step's branch is uniform.
template <int NV>
__device__ __forceinline__ void epi_steps_col(const EpiDev& e, float (&y)[NV], const int64_t (&row)[NV],
                                              int64_t col) {
#pragma unroll
  for (int s = 0; s < MR_MAX_EPI; ++s) {
    if (s >= e.n_steps) break;
    const int fn = e.steps[s].fn;
    const int mode = e.steps[s].mode;
    const float* p = e.steps[s].ptr;
    const int64_t ld = e.steps[s].ld;
    if (fn == MR_EPI_RELU) {
#pragma unroll
      for (int v = 0; v < NV; ++v) y[v] = np_maximum(y[v], 0.0f);
      continue;
    }
    float o[NV];
    if (mode == MR_BC_SCALAR) {
      const float c = p[0];
#pragma unroll
      for (int v = 0; v < NV; ++v) o[v] = c;
    } else if (mode == MR_BC_COL) {
      const float c = p[col];
#pragma unroll
      for (int v = 0; v < NV; ++v) o[v] = c;
    } else if (mode == MR_BC_ROW) {
#pragma unroll
      for (int v = 0; v < NV; ++v) o[v] = p[row[v] * ld];
    } else {
#pragma unroll
      for (int v = 0; v < NV; ++v) o[v] = p[row[v] * ld + col];
    }
    if (e.steps[s].swapped) {
#pragma unroll
      for (int v = 0; v < NV; ++v) y[v] = epi_binary(fn, o[v], y[v]);
    } else {
#pragma unroll
      for (int v = 0; v < NV; ++v) y[v] = epi_binary(fn, y[v], o[v]);
    }
  }
}

// Single-element form for the elementwise kernels.
__device__ __forceinline__ float epi_steps(const EpiDev& e, float y, int64_t row, int64_t col) {
  float v[1] = {y};
  const int64_t r[1] = {row};
  epi_steps_col<1>(e, v, r, col);
  return v[0];
}

// Write the outputs for one finished result element.
__device__ __forceinline__ void epi_store(const EpiDev& e, float y, int64_t row, int64_t col) {
  if (e.out_f32) e.out_f32[row * e.ldo + col] = y;
  if (e.out_i8) e.out_i8[row * e.ldq + col] = quantize_one(y, e.out_xs);
}

// Dequantize one int32 accumulator (mira/ops.py:618 / :633):
// f32(f64(acc) * (f64(x_scale) * f64(w_scale[col]))); the combined scale is
// precomputed on the host in double precision.
__device__ __forceinline__ float dequant(int32_t acc, double scale) {
  return static_cast<float>(__dmul_rn(static_cast<double>(acc), scale));
}

// ---------------------------------------------------------------- host-side epilogue validation

int make_epi(const mr_epilogue* epi, int64_t cols, bool need_scale, EpiDev* out);

}  // namespace mr
