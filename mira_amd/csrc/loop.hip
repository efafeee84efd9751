// Kernels for the integer and data-movement ops of device loops: while / if sub-graphs
// that the rocm target runs entirely on the GPU (a token buffer, a step counter, cache rows
// written at a runtime position).  Every value is 4 bytes per element on the device: f32,
// f16 values held as f32, and i32 values held as their own bits in the same buffers, so the
// data-movement kernels copy words and only the arithmetic reads them as integers.
// Positions read from device memory (gather indices, dynamic-slice starts) are clamped
// into range inside the kernels, so no input can address outside a buffer.
#include "mr_common.hpp"

#include <climits>

namespace mr {

// workgroups of a grid-stride launch over `total` elements: one per `block`, at most 64 per CU
static int grid_1d(int64_t total, int block) {
  int64_t g = (total + block - 1) / block;
  const int64_t cap = int64_t(device_cu_count()) * 64;
  if (g > cap) g = cap;
  if (g < 1) g = 1;
  return static_cast<int>(g);
}

namespace {

struct Shape4 {
  int64_t n[4];
  int64_t sa[4];
  int64_t sb[4];
  int64_t sc[4];
};

__device__ __forceinline__ void offsets(const Shape4& sh, int64_t i, int64_t& ia, int64_t& ib, int64_t& ic) {
  int64_t r = i;
  ia = ib = ic = 0;
#pragma unroll
  for (int d = 3; d >= 0; --d) {
    const int64_t c = r % sh.n[d];
    r /= sh.n[d];
    ia += c * sh.sa[d];
    ib += c * sh.sb[d];
    ic += c * sh.sc[d];
  }
}

// NumPy int32 arithmetic (mira/ops.py:163-169 with integers kept exact): add / sub / mul
// wrap around, comparisons give 1 / 0
__device__ __forceinline__ int32_t ew_i32(int fn, int32_t a, int32_t b) {
  const uint32_t ua = static_cast<uint32_t>(a), ub = static_cast<uint32_t>(b);
  switch (fn) {
    case MR_EPI_ADD: return static_cast<int32_t>(ua + ub);
    case MR_EPI_SUB: return static_cast<int32_t>(ua - ub);
    case MR_EPI_MUL: return static_cast<int32_t>(ua * ub);
    case MR_EPI_MAX: return a > b ? a : b;
    case MR_EPI_MIN: return a < b ? a : b;
    case MR_EPI_RELU: return a > 0 ? a : 0;
    case MR_EW_GREATER: return a > b ? 1 : 0;
    case MR_EW_GREATER_EQUAL: return a >= b ? 1 : 0;
    case MR_EW_EQUAL: return a == b ? 1 : 0;
    case MR_EW_NEG: return static_cast<int32_t>(0u - ua);
    case MR_EW_ABS: return a < 0 ? static_cast<int32_t>(0u - ua) : a;
    default: return a;
  }
}

__global__ void __launch_bounds__(256) elementwise_i32_kernel(int fn, const int32_t* __restrict__ a,
                                                              const int32_t* __restrict__ b, int32_t* __restrict__ y,
                                                              const Shape4 sh, int64_t total) {
  const int64_t stride = int64_t(gridDim.x) * 256;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < total; i += stride) {
    int64_t ia, ib, ic;
    offsets(sh, i, ia, ib, ic);
    y[i] = ew_i32(fn, a[ia], b ? b[ib] : 0);
  }
}

// astype between f32, f16 (held as f32) and i32 (mira/ops.py:405-406): integers to floats
// round to nearest (to f16 directly, one rounding); floats to integers truncate toward zero,
// and NaN, infinities and values outside int32 give INT_MIN, as NumPy's conversion does on x86
__global__ void __launch_bounds__(256) cast_kernel(const uint32_t* __restrict__ x, int64_t n, int from, int to,
                                                   uint32_t* __restrict__ y) {
  const int64_t stride = int64_t(gridDim.x) * 256;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride) {
    const uint32_t w = x[i];
    if (from == MR_DT_I32) {
      const int32_t v = static_cast<int32_t>(w);
      const float f = to == MR_DT_F16 ? __half2float(__int2half_rn(v)) : __int2float_rn(v);
      y[i] = __float_as_uint(f);
    } else {
      const float f = __uint_as_float(w);
      int32_t v = INT_MIN;
      if (f == f && f < 2147483648.0f && f >= -2147483648.0f) v = static_cast<int32_t>(f);
      y[i] = static_cast<uint32_t>(v);
    }
  }
}

// y[i, :] = table[idx[i], :] (mira/ops.py:479-484, axis 0): a negative index counts from the
// end as in NumPy's take; one still out of range (NumPy raises) is clamped into the table
__global__ void __launch_bounds__(256) gather_rows_kernel(const uint32_t* __restrict__ table, int64_t rows,
                                                          int64_t row, const int32_t* __restrict__ idx,
                                                          int64_t n_idx, uint32_t* __restrict__ y) {
  const int64_t total = n_idx * row, stride = int64_t(gridDim.x) * 256;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < total; i += stride) {
    const int64_t k = i / row;
    int64_t r = idx[k];
    if (r < 0) r += rows;
    r = r < 0 ? 0 : (r >= rows ? rows - 1 : r);
    y[i] = table[r * row + (i - k * row)];
  }
}

// the start of a runtime window, clamped so it stays inside each axis (mira/ops.py:538-539);
// axes before the value's rank are leading 1s with start 0
__device__ __forceinline__ void clamped_starts(const int32_t* start, int rank, const int64_t* shape,
                                               const int64_t* size, int64_t* st) {
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    int64_t s = d < 4 - rank ? 0 : start[d - (4 - rank)];
    const int64_t hi = shape[d] - size[d];
    st[d] = s < 0 ? 0 : (s > hi ? hi : s);
  }
}

struct Window {
  int64_t shape[4];   // the whole value
  int64_t size[4];    // the window
};

// y = x[start : start + size] (mira/ops.py:551-554)
__global__ void __launch_bounds__(256) dynamic_slice_kernel(const uint32_t* __restrict__ x, const Window w,
                                                            const int32_t* __restrict__ start, int rank,
                                                            uint32_t* __restrict__ y, int64_t total) {
  int64_t st[4];
  clamped_starts(start, rank, w.shape, w.size, st);
  const int64_t stride = int64_t(gridDim.x) * 256;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < total; i += stride) {
    int64_t r = i, src = 0, mul = 1;
#pragma unroll
    for (int d = 3; d >= 0; --d) {
      const int64_t c = r % w.size[d];
      r /= w.size[d];
      src += (c + st[d]) * mul;
      mul *= w.shape[d];
    }
    y[i] = x[src];
  }
}

// y = x with x[start : start + size] replaced by upd (mira/ops.py:567-572), in one pass
__global__ void __launch_bounds__(256) dynamic_update_kernel(const uint32_t* __restrict__ x, const Window w,
                                                             const uint32_t* __restrict__ upd,
                                                             const int32_t* __restrict__ start, int rank,
                                                             uint32_t* __restrict__ y, int64_t total) {
  int64_t st[4];
  clamped_starts(start, rank, w.shape, w.size, st);
  const int64_t stride = int64_t(gridDim.x) * 256;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < total; i += stride) {
    int64_t r = i, u = 0, mul = 1;
    bool inside = true;
#pragma unroll
    for (int d = 3; d >= 0; --d) {
      const int64_t c = r % w.shape[d] - st[d];
      r /= w.shape[d];
      inside = inside && c >= 0 && c < w.size[d];
      u += c * mul;
      mul *= w.size[d];
    }
    y[i] = inside ? upd[u] : x[i];
  }
}

// index of the first maximum of each row (mira/ops.py:527-528): NumPy's argmax, where the
// first NaN wins; one wave per row
__global__ void __launch_bounds__(256) argmax_kernel(const float* __restrict__ x, int64_t rows, int64_t n,
                                                     int32_t* __restrict__ y) {
  const int lane = threadIdx.x & 63;
  const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float* xr = x + row * n;
  float best = -INFINITY;
  int at = -1;
  bool nan = false;
  for (int j = lane; j < n; j += 64) {
    const float v = xr[j];
    if (nan) continue;
    if (v != v) {
      nan = true;
      at = j;
    } else if (at < 0 || v > best) {
      best = v;
      at = j;
    }
  }
  // combine lanes: a NaN beats any number (the earliest NaN), else the larger value, ties to
  // the earlier index
  for (int off = 32; off > 0; off >>= 1) {
    const float ob = __shfl_xor(best, off, 64);
    const int oa = __shfl_xor(at, off, 64);
    const bool on = __shfl_xor(static_cast<int>(nan), off, 64) != 0;
    bool take;
    if (oa < 0) take = false;
    else if (at < 0) take = true;
    else if (nan != on) take = on;
    else if (nan) take = oa < at;
    else take = ob > best || (ob == best && oa < at);
    if (take) {
      best = ob;
      at = oa;
      nan = on;
    }
  }
  if (lane == 0) y[row] = at < 0 ? 0 : at;
}

// y = where(cond != 0, a, b) (mira/ops.py:432-433), all three broadcast by strides; an f32
// condition is true when non-zero or NaN, an i32 one when non-zero
__global__ void __launch_bounds__(256) where_kernel(const uint32_t* __restrict__ c, int c_int,
                                                    const uint32_t* __restrict__ a, const uint32_t* __restrict__ b,
                                                    uint32_t* __restrict__ y, const Shape4 sh, int64_t total) {
  const int64_t stride = int64_t(gridDim.x) * 256;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < total; i += stride) {
    int64_t ia, ib, ic;
    offsets(sh, i, ia, ib, ic);
    const uint32_t w = c[ic];
    const bool t = c_int ? w != 0u : __uint_as_float(w) != 0.0f;
    y[i] = t ? a[ia] : b[ib];
  }
}

}  // namespace

}  // namespace mr

extern "C" {

int mr_elementwise_i32(int32_t fn, const int32_t* a, const int64_t* a_stride, const int32_t* b,
                       const int64_t* b_stride, int32_t* y, const int64_t* shape, void* stream) {
  const bool unary = fn == MR_EPI_RELU || fn == MR_EW_NEG || fn == MR_EW_ABS;
  const bool binary = fn == MR_EPI_ADD || fn == MR_EPI_SUB || fn == MR_EPI_MUL || fn == MR_EPI_MAX ||
                      fn == MR_EPI_MIN || fn == MR_EW_GREATER || fn == MR_EW_GREATER_EQUAL || fn == MR_EW_EQUAL;
  MR_REQUIRE(unary || binary, "mr_elementwise_i32: unsupported function %d", fn);
  MR_REQUIRE(a && a_stride && y && shape, "mr_elementwise_i32: NULL argument");
  MR_REQUIRE(!binary || (b && b_stride), "mr_elementwise_i32: a binary function needs b and its strides");
  mr::Shape4 sh = {};
  int64_t total = 1;
  for (int d = 0; d < 4; ++d) {
    MR_REQUIRE(shape[d] >= 0 && a_stride[d] >= 0 && (!binary || b_stride[d] >= 0), "mr_elementwise_i32: bad shape");
    sh.n[d] = shape[d];
    sh.sa[d] = a_stride[d];
    sh.sb[d] = binary ? b_stride[d] : 0;
    total *= shape[d];
  }
  if (total == 0) return MR_OK;
  hipLaunchKernelGGL(mr::elementwise_i32_kernel, dim3(mr::grid_1d(total, 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), fn, a, binary ? b : nullptr, y, sh, total);
  MR_LAUNCH_CHECK("elementwise_i32");
  return MR_OK;
}

int mr_cast_32(const void* x, int64_t n, int32_t from, int32_t to, void* y, void* stream) {
  MR_REQUIRE(x && y && n >= 0, "mr_cast_32: bad arguments");
  const bool ok = (from == MR_DT_I32 && (to == MR_DT_F32 || to == MR_DT_F16)) ||
                  ((from == MR_DT_F32 || from == MR_DT_F16) && to == MR_DT_I32);
  MR_REQUIRE(ok, "mr_cast_32: unsupported cast %d -> %d", from, to);
  if (n == 0) return MR_OK;
  hipLaunchKernelGGL(mr::cast_kernel, dim3(mr::grid_1d(n, 256)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint32_t*>(x), n, from, to, static_cast<uint32_t*>(y));
  MR_LAUNCH_CHECK("cast_32");
  return MR_OK;
}

int mr_gather_rows_32(const void* table, int64_t rows, int64_t row_elems, const int32_t* idx, int64_t n_idx,
                      void* y, void* stream) {
  MR_REQUIRE(table && idx && y, "mr_gather_rows_32: NULL argument");
  MR_REQUIRE(rows > 0 && row_elems > 0 && n_idx >= 0, "mr_gather_rows_32: bad shape");
  if (n_idx == 0) return MR_OK;
  hipLaunchKernelGGL(mr::gather_rows_kernel, dim3(mr::grid_1d(n_idx * row_elems, 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint32_t*>(table), rows, row_elems, idx,
                     n_idx, static_cast<uint32_t*>(y));
  MR_LAUNCH_CHECK("gather_rows_32");
  return MR_OK;
}

static int window(const int64_t* shape, const int64_t* size, int32_t rank, mr::Window* w, int64_t* total,
                  const char* who) {
  MR_REQUIRE(shape && size && rank >= 1 && rank <= 4, "%s: bad rank", who);
  int64_t t = 1;
  for (int d = 0; d < 4; ++d) {
    MR_REQUIRE(shape[d] >= 1 && size[d] >= 0 && size[d] <= shape[d], "%s: window does not fit", who);
    MR_REQUIRE(d >= 4 - rank || (shape[d] == 1 && size[d] == 1), "%s: axes before the rank must be 1", who);
    w->shape[d] = shape[d];
    w->size[d] = size[d];
    t *= size[d];
  }
  *total = t;
  return MR_OK;
}

int mr_dynamic_slice_32(const void* x, const int64_t* shape, const int32_t* start, int32_t rank,
                        const int64_t* size, void* y, void* stream) {
  MR_REQUIRE(x && start && y, "mr_dynamic_slice_32: NULL argument");
  mr::Window w = {};
  int64_t total = 0;
  const int rc = window(shape, size, rank, &w, &total, "mr_dynamic_slice_32");
  if (rc != MR_OK) return rc;
  if (total == 0) return MR_OK;
  hipLaunchKernelGGL(mr::dynamic_slice_kernel, dim3(mr::grid_1d(total, 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint32_t*>(x), w, start, rank,
                     static_cast<uint32_t*>(y), total);
  MR_LAUNCH_CHECK("dynamic_slice_32");
  return MR_OK;
}

int mr_dynamic_update_slice_32(const void* x, const int64_t* shape, const void* upd, const int64_t* size,
                               const int32_t* start, int32_t rank, void* y, void* stream) {
  MR_REQUIRE(x && upd && start && y && x != y, "mr_dynamic_update_slice_32: bad pointers");
  mr::Window w = {};
  int64_t window_total = 0;
  const int rc = window(shape, size, rank, &w, &window_total, "mr_dynamic_update_slice_32");
  if (rc != MR_OK) return rc;
  const int64_t total = shape[0] * shape[1] * shape[2] * shape[3];
  hipLaunchKernelGGL(mr::dynamic_update_kernel, dim3(mr::grid_1d(total, 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint32_t*>(x), w,
                     static_cast<const uint32_t*>(upd), start, rank, static_cast<uint32_t*>(y), total);
  MR_LAUNCH_CHECK("dynamic_update_slice_32");
  return MR_OK;
}

int mr_argmax_f32(const float* x, int64_t rows, int64_t n, int32_t* y, void* stream) {
  MR_REQUIRE(x && y && rows >= 0 && n >= 1 && n < (int64_t(1) << 31), "mr_argmax_f32: bad arguments");
  if (rows == 0) return MR_OK;
  const int64_t blocks = (rows + 3) / 4;
  MR_REQUIRE(blocks < (int64_t(1) << 31), "mr_argmax_f32: too many rows");
  hipLaunchKernelGGL(mr::argmax_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, rows, n, y);
  MR_LAUNCH_CHECK("argmax");
  return MR_OK;
}

int mr_where_32(const void* cond, int32_t cond_int, const int64_t* c_stride, const void* a, const int64_t* a_stride,
                const void* b, const int64_t* b_stride, void* y, const int64_t* shape, void* stream) {
  MR_REQUIRE(cond && c_stride && a && a_stride && b && b_stride && y && shape, "mr_where_32: NULL argument");
  mr::Shape4 sh = {};
  int64_t total = 1;
  for (int d = 0; d < 4; ++d) {
    MR_REQUIRE(shape[d] >= 0 && c_stride[d] >= 0 && a_stride[d] >= 0 && b_stride[d] >= 0, "mr_where_32: bad shape");
    sh.n[d] = shape[d];
    sh.sa[d] = a_stride[d];
    sh.sb[d] = b_stride[d];
    sh.sc[d] = c_stride[d];
    total *= shape[d];
  }
  if (total == 0) return MR_OK;
  hipLaunchKernelGGL(mr::where_kernel, dim3(mr::grid_1d(total, 256)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint32_t*>(cond), cond_int, static_cast<const uint32_t*>(a),
                     static_cast<const uint32_t*>(b), static_cast<uint32_t*>(y), sh, total);
  MR_LAUNCH_CHECK("where_32");
  return MR_OK;
}

}  // extern "C"
