// K1: the activation quantizer of mira/ops.py:602-603 (f32 -> int8),
// bandwidth-bound: 4 bytes read and 1 byte written per element.
#include "mr_common.hpp"

namespace mr {

// Row-major [rows, cols] f32 (row stride ldx) -> [rows, ldq] int8, zero pad.
// One thread writes 4 consecutive output bytes (one dword store).
__global__ void __launch_bounds__(256) quantize_rows_kernel(const float* __restrict__ x, int64_t rows,
                                                            int64_t cols, int64_t ldx, int8_t* __restrict__ q,
                                                            int64_t ldq, float xs) {
  const int64_t groups = ldq >> 2;
  const int64_t total = rows * groups;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = t / groups;
    const int64_t c0 = (t - r * groups) << 2;
    const float* xr = x + r * ldx;
    uint32_t packed = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t c = c0 + j;
      const int8_t v = c < cols ? quantize_one(xr[c], xs) : int8_t(0);
      packed |= uint32_t(uint8_t(v)) << (8 * j);
    }
    *reinterpret_cast<uint32_t*>(q + r * ldq + c0) = packed;
  }
}

// NCHW f32 -> NHWC int8 with c_pad channels.  Thread t handles one pixel and
// one group of 4 channels; pixels are fastest so the f32 reads coalesce and
// for c_pad == 4 the dword stores do too.  F16: quantize the f16 rounding of
// each value (an f32 -> f16 cast fused in front).
template <bool F16>
__global__ void __launch_bounds__(256) quantize_nchw_nhwc_kernel(const float* __restrict__ x, int n, int c,
                                                                 int hw, int8_t* __restrict__ q, int c_pad,
                                                                 float xs) {
  const int groups = c_pad >> 2;
  const int64_t total = (int64_t)n * groups * hw;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t p = t % hw;
    const int64_t rest = t / hw;
    const int g = static_cast<int>(rest % groups);
    const int64_t img = rest / groups;
    uint32_t packed = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int ch = g * 4 + j;
      float f = ch < c ? x[(img * c + ch) * hw + p] : 0.0f;
      if constexpr (F16) f = round_f16(f);
      const int8_t v = ch < c ? quantize_one(f, xs) : int8_t(0);
      packed |= uint32_t(uint8_t(v)) << (8 * j);
    }
    *reinterpret_cast<uint32_t*>(q + (img * hw + p) * c_pad + g * 4) = packed;
  }
}

// Same result, four consecutive pixels per thread (hw % 4 == 0): one 16-byte
// load per channel plane, the quotient through the double-precision
// reciprocal of the scale (equal to the IEEE quotient, see quantize_rcp),
// and one 16-byte store of four 4-channel pixels when c_pad == 4.  The grid's
// y index is (image, channel group), so no thread divides.
template <bool F16>
__global__ void __launch_bounds__(256) quantize_nchw_nhwc4_kernel(const float* __restrict__ x, int c, int hw,
                                                                  int8_t* __restrict__ q, int c_pad, double rxs) {
  const int groups = c_pad >> 2;
  const int img = blockIdx.y / groups;
  const int g = blockIdx.y - img * groups;
  const int p = 4 * (blockIdx.x * 256 + threadIdx.x);
  if (p >= hw) return;
  uint32_t packed[4] = {0, 0, 0, 0};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int ch = g * 4 + j;
    if (ch >= c) break;
    const float4 v = *reinterpret_cast<const float4*>(x + (int64_t(img) * c + ch) * hw + p);
    float f[4] = {v.x, v.y, v.z, v.w};
    if constexpr (F16) {
#pragma unroll
      for (int k = 0; k < 4; ++k) f[k] = round_f16(f[k]);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) packed[k] |= uint32_t(uint8_t(quantize_rcp(f[k], rxs))) << (8 * j);
  }
  int8_t* dst = q + (int64_t(img) * hw + p) * c_pad + g * 4;
  if (c_pad == 4) {
    *reinterpret_cast<uint4*>(dst) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) *reinterpret_cast<uint32_t*>(dst + k * c_pad) = packed[k];
  }
}

static int grid_for(int64_t total, int block) {
  int64_t g = (total + block - 1) / block;
  const int64_t cap = int64_t(device_cu_count()) * 64;
  if (g > cap) g = cap;
  if (g < 1) g = 1;
  return static_cast<int>(g);
}

template <bool F16>
static int quantize_nchw_nhwc(const char* who, const float* x, int32_t n, int32_t c, int32_t h, int32_t w, int8_t* q,
                              int32_t c_pad, float xs, void* stream) {
  MR_REQUIRE(x && q, "%s: NULL pointer", who);
  MR_REQUIRE(n >= 0 && c > 0 && h > 0 && w > 0, "%s: bad shape", who);
  MR_REQUIRE(c_pad >= c && c_pad % 4 == 0, "%s: c_pad %d must be >= c %d and a multiple of 4", who, c_pad, c);
  MR_REQUIRE(reinterpret_cast<uintptr_t>(q) % 4 == 0, "%s: q must be 4-byte aligned", who);
  MR_REQUIRE(xs > 0.0f, "%s: scale must be positive", who);
  if (n == 0) return MR_OK;
  const int64_t hw = int64_t(h) * w;
  if (hw % 4 == 0 && int64_t(n) * (c_pad / 4) < 65536 && hw < (int64_t(1) << 30) &&
      reinterpret_cast<uintptr_t>(x) % 16 == 0 && (c_pad != 4 || reinterpret_cast<uintptr_t>(q) % 16 == 0)) {
    const dim3 grid(static_cast<unsigned>((hw / 4 + 255) / 256), static_cast<unsigned>(n * (c_pad / 4)));
    hipLaunchKernelGGL(quantize_nchw_nhwc4_kernel<F16>, grid, dim3(256), 0, static_cast<hipStream_t>(stream), x, c,
                       static_cast<int>(hw), q, c_pad, 1.0 / static_cast<double>(xs));
    MR_LAUNCH_CHECK("quantize_nchw_nhwc");
    return MR_OK;
  }
  const int64_t total = int64_t(n) * (c_pad / 4) * h * w;
  hipLaunchKernelGGL(quantize_nchw_nhwc_kernel<F16>, dim3(grid_for(total, 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, n, c, h * w, q, c_pad, xs);
  MR_LAUNCH_CHECK("quantize_nchw_nhwc");
  return MR_OK;
}

}  // namespace mr

extern "C" {

int mr_quantize_rows(const float* x, int64_t rows, int64_t cols, int64_t ldx, int8_t* q, int64_t ldq, float xs,
                     void* stream) {
  MR_REQUIRE(x && q, "mr_quantize_rows: NULL pointer");
  MR_REQUIRE(rows >= 0 && cols >= 0, "mr_quantize_rows: negative size");
  MR_REQUIRE(ldx >= cols, "mr_quantize_rows: ldx %lld < cols %lld", (long long)ldx, (long long)cols);
  MR_REQUIRE(ldq >= cols && ldq % 4 == 0, "mr_quantize_rows: ldq %lld must be >= cols and a multiple of 4",
             (long long)ldq);
  MR_REQUIRE(reinterpret_cast<uintptr_t>(q) % 4 == 0, "mr_quantize_rows: q must be 4-byte aligned");
  MR_REQUIRE(xs > 0.0f, "mr_quantize_rows: scale must be positive");
  if (rows == 0 || ldq == 0) return MR_OK;
  const int64_t total = rows * (ldq / 4);
  hipLaunchKernelGGL(mr::quantize_rows_kernel, dim3(mr::grid_for(total, 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, rows, cols, ldx, q, ldq, xs);
  MR_LAUNCH_CHECK("quantize_rows");
  return MR_OK;
}

int mr_quantize_nchw_nhwc(const float* x, int32_t n, int32_t c, int32_t h, int32_t w, int8_t* q, int32_t c_pad,
                          float xs, void* stream) {
  return mr::quantize_nchw_nhwc<false>("mr_quantize_nchw_nhwc", x, n, c, h, w, q, c_pad, xs, stream);
}

int mr_quantize_f16_nchw_nhwc(const float* x, int32_t n, int32_t c, int32_t h, int32_t w, int8_t* q, int32_t c_pad,
                              float xs, void* stream) {
  return mr::quantize_nchw_nhwc<true>("mr_quantize_f16_nchw_nhwc", x, n, c, h, w, q, c_pad, xs, stream);
}

}  // extern "C"
