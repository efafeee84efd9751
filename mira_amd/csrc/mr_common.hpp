// Shared host/device helpers for libmira_rocm.so (gfx950).
//
// Numerics follow NumPy's float32 semantics as used by MIRA's golden model:
// every epilogue step is one correctly rounded IEEE-754 single operation
// (the library is built with -ffp-contract=off so nothing is fused), the
// activation quantizer rounds the correctly rounded float32 quotient half to
// even (computed either by IEEE division or by the provably equivalent
// double-precision reciprocal multiply below, never by a float32 reciprocal),
// and dequantization multiplies in double precision.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstdint>
#include <cstdarg>
#include <cstdio>

#include "../../include/mira_rocm.h"

namespace mr {

// ---------------------------------------------------------------- host errors

void set_error(const char* fmt, ...);
int device_cu_count();

// Largest contraction length whose int32 accumulator cannot overflow:
// K * 127 * 127 <= 2^31 - 1 (both operands are clipped to [-127, 127]).
constexpr int64_t MAX_EXACT_K = 133144;

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

// The same quantizer with the division replaced by a double-precision
// multiply with rxs = fl64(1 / xs): for float32 y and xs the exact quotient
// is never within 2^-49 (relative) of a float32 rounding midpoint, and
// fl64(fl64(y) * rxs) is within 2^-51 of it, so rounding it to float32 gives
// exactly fl32(y / xs).  Checked against IEEE division in the test suite.
__device__ __forceinline__ int8_t quantize_rcp(float y, double rxs) {
  float t = rintf(static_cast<float>(__dmul_rn(static_cast<double>(y), rxs)));
  t = fminf(fmaxf(t, -127.0f), 127.0f);
  return static_cast<int8_t>(static_cast<int>(t));
}

// NumPy float32 maximum/minimum on x86: NaN in either operand propagates
// (the first one if both are NaN), and on equality (including +0 vs -0) the
// second operand is returned.  Written as selects so no lane branches.
__device__ __forceinline__ float np_maximum(float a, float b) {
  float r = a > b ? a : b;
  r = b != b ? b : r;
  return a != a ? a : r;
}
__device__ __forceinline__ float np_minimum(float a, float b) {
  float r = a < b ? a : b;
  r = b != b ? b : r;
  return a != a ? a : r;
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

// The unary steps with a libm call (mira/ops.py:94-103), each operation in
// NumPy's order: gelu = (0.5 * x) * (1 + tanh(c * (x + 0.044715 * x^3))),
// sigmoid = 1 / (1 + exp(-x)), tanh.  expf/tanhf and x*x*x for NumPy's powf
// differ from NumPy's results in the last bits, so these steps are approximate.
__device__ __noinline__ float epi_unary_approx(int fn, float x) {
  switch (fn) {
    case MR_EPI_GELU: {
      const float x3 = __fmul_rn(__fmul_rn(x, x), x);
      const float u = __fmul_rn(0.7978845608028654f, __fadd_rn(x, __fmul_rn(0.044715f, x3)));
      return __fmul_rn(__fmul_rn(0.5f, x), __fadd_rn(1.0f, tanhf(u)));
    }
    case MR_EPI_SIGMOID: return __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-x)));
    case MR_EPI_TANH: return tanhf(x);
    default: return x;
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
  int32_t f16;     // round results to f16 after the steps (MR_EPI_OUT_F16)
  int32_t out_h16; // out_f32 holds IEEE halves (MR_EPI_OUT_H16; implies f16)
  int32_t full_h16;  // MR_BC_FULL operands hold IEEE halves (MR_EPI_FULL_H16)
  int32_t* out_acc;
  int64_t ldacc;
  double out_rxs;  // fl64(1 / out_xs), computed on the host
  // Fixed form recognised on the host (make_epi): the steps are, in this order
  // and each optional, mul(per-column) -> add(per-column) -> add(full) ->
  // maximum(scalar) or relu -> minimum(scalar), none swapped.  Every
  // bias/residual/ReLU/ReLU6 epilogue has this form, with or without a
  // per-channel BatchNorm multiply in front; kernels then run it without the
  // general step interpreter.
  int32_t fixed;
  int32_t f_mul, f_col, f_full, f_lo, f_hi;
  int32_t nt_f32;  // f32 results stored with the non-temporal hint (set by the launcher: results of 256 MiB
                  // or more, and fixed-form results with a residual of 96 MiB or more; qgemm.hip stream_f32)
  const float* mul_ptr;
  const float* col_ptr;
  const float* full_ptr;
  int64_t full_ld;
  const float* lo_ptr;  // NULL with f_lo set: relu (maximum with +0)
  const float* hi_ptr;
};

// Element i of an array of IEEE halves that an f32 pointer stands for (an f16 value
// stored as a half: the conversion back is exact).
__device__ __forceinline__ float half_at(const float* p, int64_t i) {
  return __half2float(reinterpret_cast<const __half*>(p)[i]);
}

// The half in the low 16 bits of b, as a float (exact).
__device__ __forceinline__ float half_bits(uint32_t b) {
  return __half2float(__ushort_as_half(static_cast<unsigned short>(b & 0xffffu)));
}

// Two f16 values (floats already rounded to f16, so the conversions are exact) as halves,
// a in the low 16 bits.
__device__ __forceinline__ uint32_t pack_halves(float a, float b) {
  return uint32_t(__half_as_ushort(__float2half_rn(a))) | (uint32_t(__half_as_ushort(__float2half_rn(b))) << 16);
}

// NumPy's maximum(y, b) / minimum(y, b) for a bound b that is the same for the
// whole wave: an unordered compare and a select.  !(y <= b) holds for y > b
// and for NaN y, so a NaN y propagates and equality returns b, as NumPy does;
// a NaN bound is returned as is (it replaces y first, and !(NaN <= NaN)).
// Every step is a vector instruction: folding b_nan into the compare's
// condition instead puts a scalar OR between the compare and the select of
// each element.
__device__ __forceinline__ float max_bound(float y, float b, bool b_nan) {
  const float v = b_nan ? b : y;
  return !(v <= b) ? v : b;
}
__device__ __forceinline__ float min_bound(float y, float b, bool b_nan) {
  const float v = b_nan ? b : y;
  return !(v >= b) ? v : b;
}

// The general step interpreter (mira/ops.py:192-199) for one element at
// (row, col): a rolled loop, so its code stays small; the descriptor is a
// by-reference kernel argument and is read from the kernel-argument segment.
__device__ __forceinline__ float epi_generic(const EpiDev& e, float y, int64_t row, int64_t col) {
#pragma unroll 1
  for (int s = 0; s < e.n_steps; ++s) {
    const int fn = e.steps[s].fn;
    if (fn == MR_EPI_RELU) {
      y = np_maximum(y, 0.0f);
      continue;
    }
    if (fn >= MR_EPI_GELU) {
      y = epi_unary_approx(fn, y);
      continue;
    }
    const float* p = e.steps[s].ptr;
    const int mode = e.steps[s].mode;
    float o;
    if (mode == MR_BC_SCALAR) o = p[0];
    else if (mode == MR_BC_COL) o = p[col];
    else if (mode == MR_BC_ROW) o = p[row * e.steps[s].ld];
    else if (e.full_h16) o = half_at(p, row * e.steps[s].ld + col);
    else o = p[row * e.steps[s].ld + col];
    y = e.steps[s].swapped ? epi_binary(fn, o, y) : epi_binary(fn, y, o);
  }
  return y;
}

// The fixed form (see EpiDev): mul(col)? add(col)? add(full)? maximum(lo)? minimum(hi)?
__device__ __forceinline__ float epi_fixed(const EpiDev& e, float y, int64_t row, int64_t col) {
  if (e.f_mul) y = __fmul_rn(y, e.mul_ptr[col]);
  if (e.f_col) y = __fadd_rn(y, e.col_ptr[col]);
  if (e.f_full) y = __fadd_rn(y, e.full_h16 ? half_at(e.full_ptr, row * e.full_ld + col) : e.full_ptr[row * e.full_ld + col]);
  if (e.f_lo) y = np_maximum(y, e.lo_ptr ? e.lo_ptr[0] : 0.0f);
  if (e.f_hi) y = np_minimum(y, e.hi_ptr[0]);
  return y;
}

// NumPy's astype(float16) of an f32 value, back in f32: round to nearest even
// (overflow to inf, f16 subnormals kept), for ops whose result dtype is f16
// (mira/ops.py:620, 634 and every other op's final .astype).  Idempotent.
__device__ __forceinline__ float round_f16(float y) { return __half2float(__float2half_rn(y)); }

__device__ __forceinline__ float epi_steps(const EpiDev& e, float y, int64_t row, int64_t col) {
  y = e.fixed ? epi_fixed(e, y, row, col) : epi_generic(e, y, row, col);
  return e.f16 ? round_f16(y) : y;
}

// Write the outputs for one finished result element.  H16 = false leaves out the store
// of an f16 result as a half (for callers whose epilogues never have one).
template <bool H16 = true>
__device__ __forceinline__ void epi_store(const EpiDev& e, float y, int64_t row, int64_t col) {
  if (e.f16) y = round_f16(y);
  if (e.out_f32) {
    if (H16 && e.out_h16)
      reinterpret_cast<__half*>(e.out_f32)[row * e.ldo + col] = __float2half_rn(y);
    else
      e.out_f32[row * e.ldo + col] = y;
  }
  if (e.out_i8) e.out_i8[row * e.ldq + col] = quantize_rcp(y, e.out_rxs);
}

// Dequantize one int32 accumulator (mira/ops.py:618 / :633):
// f32(f64(acc) * (f64(x_scale) * f64(w_scale[col]))); the combined scale is
// precomputed on the host in double precision.
__device__ __forceinline__ float dequant(int32_t acc, double scale) {
  return static_cast<float>(__dmul_rn(static_cast<double>(acc), scale));
}

// Workgroup barrier without a memory fence: what it orders is established by a wait
// before it (a counted vmcnt wait for LDS DMA, or operands already consumed).  The
// signal fences keep the compiler from moving memory accesses across it.
__device__ __forceinline__ void block_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Barrier after LDS stores that other waves read next.  s_barrier does not
// wait for the wave's own outstanding LDS operations, so the stores are first
// drained (lgkmcnt 0; vmcnt and expcnt untouched): without this a wave can
// read a row another wave has issued but not yet written.
__device__ __forceinline__ void lds_store_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);   // vmcnt 63, expcnt 7, lgkmcnt 0
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Word 3 of a raw buffer resource (32-bit elements) on gfx9: loads past num_records
// return 0 and stores past it are dropped, which the kernels use for bounds.
constexpr int BUF_DWORD3 = 0x00020000;

// ---------------------------------------------------------------- host-side epilogue validation

// allow_h16: the caller's kernels implement MR_EPI_OUT_H16 / MR_EPI_FULL_H16; need_output =
// false for an intermediate result that a fused kernel consumes without storing it
int make_epi(const mr_epilogue* epi, int64_t cols, bool need_scale, EpiDev* out, bool allow_h16 = false,
             bool need_output = true);

// Decode-shaped qmatmul (M <= 8 rows): weight-streaming kernel; MR_EUNSUPPORTED for larger M.
int gemv_launch(const int8_t* a, int64_t lda, const int8_t* b, int64_t k_pad, int64_t n_pad, int64_t M, int64_t N,
                const EpiDev& e, hipStream_t stream);

// Weight-only int8 matmul of many rows on f32 MFMAs (w8gemm.hip); MR_EUNSUPPORTED when K
// or ldx is not a multiple of 4 or an operand reaches 2 GiB.
// With a conv geometry, the implicit-GEMM convolution of an NHWC f32 image (C % 4 == 0).
int w8gemm_launch(const float* x, int64_t ldx, const int8_t* b, const float* w_scale, int32_t w_f16, int64_t k_pad,
                  int64_t n_pad, int64_t M, int64_t N, int64_t K, const EpiDev& e, hipStream_t stream,
                  const mr_conv_geom* cg = nullptr);

// Epilogue forms a kernel is compiled for: EF_GENERIC runs the step
// interpreter, EF_FIXED the fixed form (see EpiDev) with its flags read at run
// time, and EF_SPEC | SF_* the fixed form with its steps and outputs known at
// compile time: a tile whose columns are all in range (any tile when N % 4 == 0) then runs its rows as
// straight-line code (all LDS reads, then all operand loads, then the math and
// the stores), so the rows' latencies overlap.
constexpr int EF_GENERIC = 0, EF_FIXED = 1, EF_SPEC = 0x100;
constexpr int SF_COL = 1, SF_FULL = 2, SF_LO = 4, SF_HI = 8, SF_F32 = 16, SF_I8 = 32;
constexpr int SF_MUL = 64;   // no compiled form has it: a leading mul runs the EF_FIXED path
constexpr int SF_F16 = 128;  // results rounded to f16 (compiled for the ResNet-style forms only)
// an f16 graph's residual read as halves (EpiDev full_h16) / its f32 result stored as halves
// (out_h16); EF_SPEC is 0x100, so these sit above it
constexpr int SF_H16R = 512, SF_H16O = 1024;
// the forms with compiled kernels: bias+ReLU -> int8; bias+residual+ReLU -> f32
// and/or int8; bias -> f32 (ResNet blocks, downsample and fc layers, MLPs)
constexpr int SPEC_RELU_I8 = SF_COL | SF_LO | SF_I8;
constexpr int SPEC_RES_F32_I8 = SF_COL | SF_FULL | SF_LO | SF_F32 | SF_I8;
constexpr int SPEC_RES_I8 = SF_COL | SF_FULL | SF_LO | SF_I8;
constexpr int SPEC_RES_F32 = SF_COL | SF_FULL | SF_LO | SF_F32;
constexpr int SPEC_BIAS_F32 = SF_COL | SF_F32;
// the fused stem's usual form: bias + ReLU, pooled, to f32 and int8
constexpr int SPEC_RELU_F32_I8 = SF_COL | SF_LO | SF_F32 | SF_I8;
// MobileNet-style blocks: 1x1 expansion + ReLU6 -> f32 (read by the depthwise
// conv); linear projection -> f32 + int8, with or without the residual add, or
// int8 only when no later residual reads the block's output
constexpr int SPEC_RELU6_F32 = SF_COL | SF_LO | SF_HI | SF_F32;
constexpr int SPEC_BIAS_F32_I8 = SF_COL | SF_F32 | SF_I8;
constexpr int SPEC_BIAS_RES_F32_I8 = SF_COL | SF_FULL | SF_F32 | SF_I8;
constexpr int SPEC_BIAS_I8 = SF_COL | SF_I8;
constexpr int SPEC_BIAS_RES_I8 = SF_COL | SF_FULL | SF_I8;

// The compile-time form of an epilogue, or -1 when it has none: the fixed
// form without an int32 accumulator output, every output and operand row
// 16-byte (f32) / 4-byte (int8) aligned.
inline int spec_form(const EpiDev& e) {
  if (!e.fixed || e.out_acc) return -1;
  auto al = [](const void* p, int64_t ld, int bytes) {
    return reinterpret_cast<uintptr_t>(p) % bytes == 0 && ld % 4 == 0;
  };
  int f = 0;
  if (e.f16) f |= SF_F16;
  if (e.f_mul) f |= SF_MUL;
  if (e.f_col) f |= SF_COL;
  if (e.f_full) {
    if (!al(e.full_ptr, e.full_ld, e.full_h16 ? 8 : 16)) return -1;
    f |= SF_FULL | (e.full_h16 ? SF_H16R : 0);
  }
  if (e.f_lo) f |= SF_LO;
  if (e.f_hi) f |= SF_HI;
  if (e.out_f32) {
    if (!al(e.out_f32, e.ldo, e.out_h16 ? 8 : 16)) return -1;
    f |= SF_F32 | (e.out_h16 ? SF_H16O : 0);
  }
  if (e.out_i8) {
    if (!al(e.out_i8, e.ldq, 4)) return -1;
    f |= SF_I8;
  }
  return f;
}

}  // namespace mr
