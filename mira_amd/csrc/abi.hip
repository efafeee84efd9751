// Library-level entry points: version, errors, device set-up, and the host
// side validation of epilogue descriptors shared by every fused kernel.
#include <cstring>
#include <string>

#include "mr_common.hpp"

namespace mr {

static thread_local char g_error[1024] = "";
static int g_cu_count = 0;

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

int device_cu_count() { return g_cu_count > 0 ? g_cu_count : 256; }

int make_epi(const mr_epilogue* epi, int64_t cols, bool need_scale, EpiDev* out, bool allow_h16, bool need_output) {
  MR_REQUIRE(epi != nullptr, "epilogue descriptor is NULL");
  MR_REQUIRE(epi->n_steps >= 0 && epi->n_steps <= MR_MAX_EPI, "epilogue has %d steps (max %d)",
             epi->n_steps, MR_MAX_EPI);
  if (need_scale) {
    MR_REQUIRE(epi->scale != nullptr, "epilogue needs a per-column dequant scale");
  } else {
    MR_REQUIRE(epi->scale == nullptr, "this kernel has no int32 accumulator to dequantize");
  }
  MR_REQUIRE(!need_output || epi->out_f32 || epi->out_i8 || epi->out_acc, "epilogue writes no output");
  MR_REQUIRE((epi->flags & ~(MR_EPI_OUT_F16 | MR_EPI_OUT_H16 | MR_EPI_FULL_H16)) == 0, "unknown epilogue flags 0x%x",
             epi->flags);
  if ((epi->flags & (MR_EPI_OUT_H16 | MR_EPI_FULL_H16)) && !allow_h16) {
    set_error("this kernel does not take f16 values stored as halves (epilogue flags 0x%x)", epi->flags);
    return MR_EUNSUPPORTED;
  }
  if (epi->out_f32) MR_REQUIRE(epi->ldo >= cols, "ldo %lld < cols %lld", (long long)epi->ldo, (long long)cols);
  if (epi->out_i8) {
    MR_REQUIRE(epi->ldq >= cols, "ldq %lld < cols %lld", (long long)epi->ldq, (long long)cols);
    MR_REQUIRE(epi->out_xs > 0.0f, "requant scale must be positive, got %g", (double)epi->out_xs);
  }
  if (epi->out_acc) {
    MR_REQUIRE(need_scale, "int32 accumulators exist only for int8 contractions");
    MR_REQUIRE(epi->ldacc >= cols, "ldacc < cols");
  }
  std::memset(out, 0, sizeof(*out));
  out->n_steps = epi->n_steps;
  out->has_scale = epi->scale != nullptr;
  for (int s = 0; s < epi->n_steps; ++s) {
    const mr_epi_step& st = epi->steps[s];
    MR_REQUIRE(st.fn >= MR_EPI_ADD && st.fn <= MR_EPI_TANH, "epilogue step %d: unknown fn %d", s, st.fn);
    const bool unary = st.fn == MR_EPI_RELU || st.fn >= MR_EPI_GELU;
    if (!unary) {
      MR_REQUIRE(st.ptr != nullptr, "epilogue step %d: operand pointer is NULL", s);
      MR_REQUIRE(st.mode >= MR_BC_SCALAR && st.mode <= MR_BC_FULL, "epilogue step %d: bad mode %d", s,
                 st.mode);
      if (st.mode == MR_BC_FULL) MR_REQUIRE(st.ld >= cols, "epilogue step %d: ld < cols", s);
    }
    out->steps[s].fn = st.fn;
    out->steps[s].swapped = st.swapped;
    out->steps[s].mode = st.mode;
    out->steps[s].ptr = st.ptr;
    out->steps[s].ld = st.ld;
  }
  out->scale = epi->scale;
  out->out_f32 = epi->out_f32;
  out->ldo = epi->ldo;
  out->out_i8 = epi->out_i8;
  out->ldq = epi->ldq;
  out->out_xs = epi->out_xs;
  out->out_h16 = (epi->flags & MR_EPI_OUT_H16) != 0;
  out->full_h16 = (epi->flags & MR_EPI_FULL_H16) != 0;
  out->f16 = (epi->flags & (MR_EPI_OUT_F16 | MR_EPI_OUT_H16)) != 0;
  out->out_acc = epi->out_acc;
  out->ldacc = epi->ldacc;
  out->out_rxs = epi->out_i8 ? 1.0 / static_cast<double>(epi->out_xs) : 0.0;
  // recognise the fixed form  mul(col)? add(col)? add(full)? max(scalar)|relu? min(scalar)?
  int stage = 0;
  bool fixed = true;
  for (int s = 0; s < epi->n_steps && fixed; ++s) {
    const mr_epi_step& st = epi->steps[s];
    if (st.fn == MR_EPI_RELU) {
      if (stage > 3) fixed = false;
      out->f_lo = 1;
      out->lo_ptr = nullptr;
      stage = 4;
      continue;
    }
    if (st.swapped) {
      fixed = false;
    } else if (st.fn == MR_EPI_MUL && st.mode == MR_BC_COL && stage < 1) {
      out->f_mul = 1;
      out->mul_ptr = st.ptr;
      stage = 1;
    } else if (st.fn == MR_EPI_ADD && st.mode == MR_BC_COL && stage < 2) {
      out->f_col = 1;
      out->col_ptr = st.ptr;
      stage = 2;
    } else if (st.fn == MR_EPI_ADD && st.mode == MR_BC_FULL && stage < 3) {
      out->f_full = 1;
      out->full_ptr = st.ptr;
      out->full_ld = st.ld;
      stage = 3;
    } else if (st.fn == MR_EPI_MAX && st.mode == MR_BC_SCALAR && stage < 4) {
      out->f_lo = 1;
      out->lo_ptr = st.ptr;
      stage = 4;
    } else if (st.fn == MR_EPI_MIN && st.mode == MR_BC_SCALAR && stage < 5) {
      out->f_hi = 1;
      out->hi_ptr = st.ptr;
      stage = 5;
    } else {
      fixed = false;
    }
  }
  out->fixed = fixed;
  if (!fixed) out->f_mul = out->f_col = out->f_full = out->f_lo = out->f_hi = 0;
  return MR_OK;
}

}  // namespace mr

extern "C" {

int mr_abi_version(void) { return MR_ABI_VERSION; }

const char* mr_last_error(void) { return mr::g_error; }

int64_t mr_sizeof(const char* name) {
  if (!name) return -1;
  if (!std::strcmp(name, "mr_epi_step")) return sizeof(mr_epi_step);
  if (!std::strcmp(name, "mr_epilogue")) return sizeof(mr_epilogue);
  if (!std::strcmp(name, "mr_conv_geom")) return sizeof(mr_conv_geom);
  return -1;
}

int mr_init(int device) {
  int count = 0;
  MR_HIP_CHECK(hipGetDeviceCount(&count));
  MR_REQUIRE(device >= 0 && device < count, "device %d out of range (%d devices)", device, count);
  MR_HIP_CHECK(hipSetDevice(device));
  hipDeviceProp_t prop;
  MR_HIP_CHECK(hipGetDeviceProperties(&prop, device));
  mr::g_cu_count = prop.multiProcessorCount;
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    mr::set_error("device %d is %s; this library is built for gfx950 only", device, prop.gcnArchName);
    return MR_EUNSUPPORTED;
  }
  return MR_OK;
}

}  // extern "C"
