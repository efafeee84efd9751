// K2/K2c + K3: int8 x int8 -> int32 contraction on gfx950 MFMA
// (v_mfma_i32_32x32x32_i8) with the dequant / epilogue / requant fused into
// the store.  One kernel template serves the dense GEMM of qmatmul
// (mira/ops.py:616-620) and the implicit-GEMM convolution of qconv2d
// (mira/ops.py:630-634): only the address generation of the activation
// (A) tile differs.
//
// Pipeline.  A workgroup owns a BM x BN tile of the result and walks K in
// 64-byte steps.  Each step's A slice (BM x 64 bytes) and B slice (weights,
// BN x 64 bytes, contiguous: weights are stored K-step-major,
// [k_pad / 64][n_pad][64]) travel global -> LDS by direct-to-LDS loads (no
// VGPR staging), STAGES-1 steps ahead of the MFMAs, through a ring of STAGES
// LDS buffers.  The weights and the dense / 64-channel activation loaders use
// buffer loads: a lane's offset is fixed for a tap (or for the whole loop) and
// the step's advance is a scalar offset, so a step costs almost no vector
// instructions; padding taps and rows/columns past the end carry an offset
// past the buffer's range and read zeros.  The other activation loaders read
// such chunks from a 256-byte zero page.  One s_barrier per step; the only
// wait is a counted vmcnt for the step about to be consumed, so the LDS copy
// is always complete and no lane needs a masked write.
//
// LDS layout.  Each row of a slice is 64 bytes = four 16-byte chunks; chunk c
// of row r sits at position c ^ ((r >> 2) & 3).  gfx950's LDS serves 256 bytes
// (64 banks) per clock, i.e. 16 lanes of a ds_read_b128; 16 consecutive rows of
// one chunk then land on 16 distinct 16-byte bank groups.
//
// MFMA fragments.  Integer accumulation is exact and order-free, so the A and
// B fragments only need the same byte order along K: both read 16 contiguous
// K bytes per lane.  Result layout of the 32x32 block: lane holds column
// (lane & 31) and rows 8*(r/4) + 4*(lane/32) + (r%4), r = 0..15.
#include "mr_common.hpp"

#include <algorithm>
#include <type_traits>

namespace mr {

typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

// Source of every padding or out-of-range chunk (zero-initialised at load time).
__device__ __attribute__((aligned(256))) int8_t g_zero_page[256];

enum AMode {
  A_DENSE = 0,   // row-major [M, lda] int8
  A_CONV64 = 1,  // NHWC, c_pad % 64 == 0: a 64-byte K step is one tap, one channel block
  A_CONV16 = 2,  // NHWC, c_pad % 16 == 0: K steps may span taps
  A_CONV4 = 3,   // NHWC, c_pad == 4: each 16-byte chunk is 4 taps of one kernel row
  A_PATCH = 4    // NHWC, c_pad % 64 == 0, stride 1, dilation 1: A fragments read from a
                 // per-tile input patch (tile rows plus the kernel's halo) held in LDS
};

// A_PATCH: LDS bytes reserved for one tile's input patch (ResNet layer 1: 6 x 58
// pixels x 5 slots = 27 840 bytes), and the tile height.  With the 256x64 tile's
// 12 KB ring, four workgroups fill a CU's 160 KB.
constexpr int PATCH_MAX = 28672;
// tile rows (pixels) of the A_PATCH configurations: N <= 64 and N <= 128
constexpr int PATCH_BM64 = 256, PATCH_BM128 = 128;
static int patch_bm(int n) { return n <= 64 ? PATCH_BM64 : PATCH_BM128; }

struct GemmArgs {
  const int8_t* a;  // dense: [M, lda]; conv: NHWC input
  int64_t lda;
  const int8_t* b;  // packed weights [n_pad, k_pad]
  int64_t k_pad;
  int64_t M;
  int32_t N;
  int32_t n_pad;
  int32_t k_tiles;
  int32_t tiles_m;
  int32_t tiles_n;
  // convolution geometry
  int32_t H, W, C_pad, OH, OW, KH, KW, SH, SW, PH, PW, DH, DW;
  int32_t row_bytes;  // A_CONV4: packed bytes per kernel row
  int32_t k_real;     // A_CONV16: KH*KW*C_pad
  int32_t cb_per_tap; // A_CONV64 / A_PATCH: C_pad / 64
  // A_PATCH: a tile is `tr` output rows of one image (tr * OW <= BM pixels);
  // its patch is pr x pc input pixels (rows oh0-PH .. oh0-PH+pr-1, columns -PW .. pc-PW-1)
  int32_t tr, rg_per_img, pr, pc, patch_slots;
  // A_PATCH divisions by launch constants: n / (C_pad / 16 + 1) == umulhi(n, ps_magic),
  // n / pc == umulhi(n, pc_magic), n / OW == umulhi(n, ow_magic) with
  // magic = ceil(2^32 / d), exact for the n the kernel divides (n * d < 2^32,
  // checked on the host)
  uint32_t ps_magic, pc_magic, ow_magic;
  // dense / 64-channel conv loaders: bytes of A and of the packed weights, the ranges of
  // their buffer resources (each < 2^31: offsets are 32-bit)
  uint32_t a_bytes, b_bytes;
};

// A buffer-load offset past every resource's range: the load returns zeros.  The range
// check compares the lane's offset (not the scalar offset) with the resource's size, so
// a lane with this offset reads zeros whatever scalar offset the step adds.
constexpr uint32_t OOB_OFF = 0x80000000u;

// ceil(2^32 / d) for d >= 2: n / d == __umulhi(n, magic) whenever n * d < 2^32.  With
// magic = (2^32 + e) / d, 0 <= e < d, n * magic / 2^32 = n / d + n * e / (d * 2^32), and
// n * e < 2^32 keeps the added term under 1/d, the least distance from n / d up to the
// next integer, so the floor is unchanged.
static uint32_t div_magic(uint32_t d) { return static_cast<uint32_t>(((uint64_t(1) << 32) + d - 1) / d); }

constexpr int BK = 64;


template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

__device__ __forceinline__ void dma16(const void* src, int8_t* lds_dst) {
  __builtin_amdgcn_global_load_lds(src, (lds_void*)lds_dst, 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void* src, int8_t* lds_dst) {
  __builtin_amdgcn_global_load_lds(src, (lds_void*)lds_dst, 4, 0, 0);
}
// 16 bytes per lane from a buffer resource at (lane offset + scalar offset) into LDS; the
// 64 lanes' chunks land contiguously at lds_dst (the LDS address is a wave-uniform M0)
__device__ __forceinline__ void dma16_buf(__amdgpu_buffer_rsrc_t r, int8_t* lds_dst, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)lds_dst, 16, voff, soff, 0, 0);
}

// Per-thread constants of the 4 result columns col0 .. col0+3 a thread owns
// in the epilogue: dequant scales and, for the fixed form, the per-column
// operand and the scalar bounds.
struct EpiCols4 {
  double scale[4];
  float mulv[4];
  float colv[4];
  float lo, hi;
  bool lo_nan, hi_nan;
  bool vec;  // four valid columns and every access 16-byte (f32) / 4-byte (int8) aligned
};


// clip(rint(y / xs), -127, 127) with the division done as a multiplication by
// the double-precision reciprocal (equal to the IEEE quotient; see
// quantize_rcp) and the clip as a median.
__device__ __forceinline__ int quantize_med3(float y, double rxs) {
  const float t = rintf(static_cast<float>(__dmul_rn(static_cast<double>(y), rxs)));
  return static_cast<int>(__builtin_amdgcn_fmed3f(t, -127.0f, 127.0f));
}

// The same quantizer for four results, packed little-endian into one word.  The
// quotient is clamped first (rounding commutes with a clamp to integer bounds) and
// then rounded by adding 1.5 * 2^23: every sum lies in [2^23, 2^24), where the
// spacing of floats is 1, so the addition rounds to the nearest integer with ties
// to even (as rintf) and leaves q + 2^22 in the low mantissa bits; the low byte of
// the bit pattern is q's two's-complement byte.  v_med3_f32 maps a NaN to -127, as
// quantize_med3 does.  Three byte permutes gather the four low bytes.
__device__ __forceinline__ uint32_t quantize4_med3(const float (&y)[4], double rxs) {
  uint32_t b[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const float t = __builtin_amdgcn_fmed3f(static_cast<float>(__dmul_rn(static_cast<double>(y[c]), rxs)),
                                            -127.0f, 127.0f);
    b[c] = __float_as_uint(__fadd_rn(t, 12582912.0f));
  }
  const uint32_t lo = __builtin_amdgcn_perm(b[1], b[0], 0x0c0c0400u);   // bytes 0, 1: b0, b1
  const uint32_t hi = __builtin_amdgcn_perm(b[3], b[2], 0x0c0c0400u);   // bytes 0, 1: b2, b3
  return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

__device__ __forceinline__ void load_cols4(const EpiDev& e, int col0, int N, EpiCols4& c) {
  bool vec = col0 + 3 < N && (e.ldo % 4 == 0) && (e.ldq % 4 == 0) && (e.ldacc % 4 == 0) &&
             (reinterpret_cast<uintptr_t>(e.out_f32) % (e.out_h16 ? 8 : 16) == 0) &&
             (reinterpret_cast<uintptr_t>(e.out_i8) % 4 == 0) && (reinterpret_cast<uintptr_t>(e.out_acc) % 16 == 0);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    c.scale[k] = col0 + k < N ? e.scale[col0 + k] : 0.0;
    c.mulv[k] = (e.f_mul && col0 + k < N) ? e.mul_ptr[col0 + k] : 0.0f;
    c.colv[k] = (e.f_col && col0 + k < N) ? e.col_ptr[col0 + k] : 0.0f;
  }
  c.lo = e.f_lo && e.lo_ptr ? e.lo_ptr[0] : 0.0f;
  c.hi = e.f_hi ? e.hi_ptr[0] : 0.0f;
  c.lo_nan = c.lo != c.lo;
  c.hi_nan = c.hi != c.hi;
  if (e.f_full)
    vec = vec && (e.full_ld % 4 == 0) && (reinterpret_cast<uintptr_t>(e.full_ptr) % (e.full_h16 ? 8 : 16) == 0);
  c.vec = vec;
}

// Dequantize, apply the epilogue to, and store result row `row`, columns
// col0 .. col0+3 (mira/ops.py:616-620 / 630-634, then 192-199).
// H16: the f16-as-halves paths are compiled in (read at run time from EpiDev); the
// compiled forms without halves leave them out, which keeps their fall-back rows inside
// the register budget.
template <bool FIXED, bool H16 = true>
__device__ __forceinline__ void store_row4(const EpiDev& e, const EpiCols4& c, const v4i& acc, int64_t row, int col0,
                                          int N) {
  float y[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) y[k] = dequant(acc[k], c.scale[k]);
  if constexpr (FIXED) {
    if (e.f_mul) {
#pragma unroll
      for (int k = 0; k < 4; ++k) y[k] = __fmul_rn(y[k], c.mulv[k]);
    }
    if (e.f_col) {
#pragma unroll
      for (int k = 0; k < 4; ++k) y[k] = __fadd_rn(y[k], c.colv[k]);
    }
    if (e.f_full) {
      float o[4];
      if (H16 && e.full_h16) {
        const __half* p = reinterpret_cast<const __half*>(e.full_ptr) + row * e.full_ld + col0;
        if (c.vec) {
          const uint2 v = *reinterpret_cast<const uint2*>(p);
          o[0] = half_bits(v.x); o[1] = half_bits(v.x >> 16); o[2] = half_bits(v.y); o[3] = half_bits(v.y >> 16);
        } else {
#pragma unroll
          for (int k = 0; k < 4; ++k) o[k] = col0 + k < N ? __half2float(p[k]) : 0.0f;
        }
      } else {
        const float* p = e.full_ptr + row * e.full_ld + col0;
        if (c.vec) {
          const float4 v = *reinterpret_cast<const float4*>(p);
          o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
        } else {
#pragma unroll
          for (int k = 0; k < 4; ++k) o[k] = col0 + k < N ? p[k] : 0.0f;
        }
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) y[k] = __fadd_rn(y[k], o[k]);
    }
    if (e.f_lo) {
#pragma unroll
      for (int k = 0; k < 4; ++k) y[k] = max_bound(y[k], c.lo, c.lo_nan);
    }
    if (e.f_hi) {
#pragma unroll
      for (int k = 0; k < 4; ++k) y[k] = min_bound(y[k], c.hi, c.hi_nan);
    }
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (col0 + k < N) y[k] = epi_generic(e, y[k], row, col0 + k);
  }
  if (e.f16) {
#pragma unroll
    for (int k = 0; k < 4; ++k) y[k] = round_f16(y[k]);
  }
  if (c.vec) {
    if (e.out_acc) *reinterpret_cast<v4i*>(e.out_acc + row * e.ldacc + col0) = acc;
    if (e.out_f32) {
      if (H16 && e.out_h16)
        *reinterpret_cast<uint2*>(reinterpret_cast<__half*>(e.out_f32) + row * e.ldo + col0) =
            make_uint2(pack_halves(y[0], y[1]), pack_halves(y[2], y[3]));
      else
        *reinterpret_cast<float4*>(e.out_f32 + row * e.ldo + col0) = make_float4(y[0], y[1], y[2], y[3]);
    }
    if (e.out_i8) {
      uint32_t packed = 0;
#pragma unroll
      for (int k = 0; k < 4; ++k) packed |= uint32_t(quantize_med3(y[k], e.out_rxs) & 0xff) << (8 * k);
      *reinterpret_cast<uint32_t*>(e.out_i8 + row * e.ldq + col0) = packed;
    }
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (col0 + k >= N) break;
      if (e.out_acc) e.out_acc[row * e.ldacc + col0 + k] = acc[k];
      epi_store<H16>(e, y[k], row, col0 + k);
    }
  }
}

// KB: K bytes per ring stage, 64 or 128 (two 64-byte K steps: each A and B
// row then moves as one 128-byte run, a whole cache line; dense and
// c_pad % 128 == 0 conv loaders only).
//
// The 64-column patch tiles (ResNet layer 1) are held to 128 VGPRs, 4 waves per
// SIMD: their residual epilogues stream 0.5 GB per launch, and the fourth
// workgroup per CU hides more of that latency than the registers it costs.  So
// are the 128x256 tiles with 64-byte stages (8 waves, 72 KB of LDS): two
// workgroups then share a CU, which the residual epilogues (140 VGPRs
// otherwise) left to one -- ResNet-18 B=256 layer-3 residual conv 77 -> 55 us.
template <int BM, int BN, int WM, int WN, int STAGES, int AMODE, int EF, int KB = 64>
__global__ void __launch_bounds__(WM* WN * 64)
    __attribute__((amdgpu_waves_per_eu((AMODE == A_PATCH && BN == 64) || (BM == 128 && BN == 256 && KB == 64) ? 4 : 1)))
    qgemm_kernel(const GemmArgs g, const EpiDev e) {
  constexpr int NW = WM * WN;
  constexpr int TM = BM / WM;
  constexpr int TN = BN / WN;
  constexpr int FM = TM / 32;
  constexpr int FN = TN / 32;
  constexpr int NB = FM * FN;
  constexpr bool PATCH = AMODE == A_PATCH;
  static_assert(KB == 64 || (KB == 128 && (AMODE == A_DENSE || AMODE == A_CONV64)), "128-byte stages");
  constexpr int CPR = KB / 16;                                // 16-byte chunks per LDS row
  constexpr int NKK = KB / 32;                                // 32-byte MFMA K steps per stage
  constexpr int A_ROWS_PER_OP = AMODE == A_CONV4 ? 4 : 64 / CPR;   // rows one wave-wide DMA covers
  constexpr int A_OPS = PATCH ? 0 : BM / A_ROWS_PER_OP / NW;   // A DMAs per wave per K step
  constexpr int A_OPS1 = A_OPS > 0 ? A_OPS : 1;
  constexpr int B_OPS = BN / (64 / CPR) / NW;
  constexpr int OPS = A_OPS + B_OPS;
  constexpr int A_STAGE = PATCH ? 0 : BM * KB;                  // A bytes in one ring stage
  constexpr int STAGE_BYTES = A_STAGE + BN * KB;
  constexpr int PATCH_OPS = PATCH ? PATCH_MAX / 16 / (NW * 64) : 0;   // patch DMAs per wave
  constexpr int RING_BYTES = STAGES * STAGE_BYTES;
  // the epilogue stages the int32 tile one 32-row block row per wave at a time
  constexpr int EP_ROWS = WM * 32;
  constexpr int EP_LD = BN + 4;                     // int32 row stride (16-byte pad)
  constexpr int EP_BYTES = EP_ROWS * EP_LD * 4;
  constexpr int LDS_BYTES = RING_BYTES + (PATCH ? PATCH_MAX : 0) > EP_BYTES ? RING_BYTES + (PATCH ? PATCH_MAX : 0)
                                                                            : EP_BYTES;
  static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile must be a multiple of 32");
  static_assert(PATCH || (A_OPS * A_ROWS_PER_OP * NW == BM), "loader mapping");
  static_assert(B_OPS * (64 / CPR) * NW == BN, "loader mapping");
  static_assert(!PATCH || PATCH_OPS * 16 * NW * 64 == PATCH_MAX, "patch loader mapping");
  // STAGES == 1: a single 64-byte K step (launched only for k_tiles == 1), no ring, so the
  // workgroup holds only its epilogue staging and many more fit on a CU
  static_assert((STAGES == 1 && KB == 64 && !PATCH) || (STAGES >= 3 && (STAGES - 2) * OPS < 64),
                "stages / vmcnt range");

  __shared__ __attribute__((aligned(1024))) int8_t lds[LDS_BYTES];
  int8_t* const patch = lds + RING_BYTES;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform: per-wave offsets stay scalar
  const int wm = wave / WN;
  const int wn = wave - wm * WN;

  // XCD-aware tile order: workgroup ids are dealt round-robin to the 8 XCDs,
  // so give each XCD a contiguous run of tiles; the N-tiles of one M-tile
  // then share that XCD's L2 for their A rows.
  const int total = g.tiles_m * g.tiles_n;
  int t = blockIdx.x;
  const int full = total & ~7;
  if (t < full) t = (t & 7) * (full >> 3) + (t >> 3);
  // grouped order: runs of GROUP_M M-tiles walked column by column, so the
  // tiles running together on an XCD share both A and B panels in its L2
  constexpr int GROUP_M = 8;
  const int gm_span = GROUP_M * g.tiles_n;
  const int group = t / gm_span;
  const int first_m = group * GROUP_M;
  const int gsize = min(g.tiles_m - first_m, GROUP_M);
  const int tin = t - group * gm_span;
  const int tile_m = first_m + tin % gsize;
  const int tile_n = tin / gsize;
  const int64_t m0 = int64_t(tile_m) * BM;
  const int n0 = tile_n * BN;
  // result rows of the tile: mbase + 0 .. mbase + mvalid - 1
  int64_t mbase = m0;
  int mvalid = static_cast<int>(min(int64_t(BM), g.M - m0));
  int p_img = 0, p_oh0 = 0;
  if constexpr (PATCH) {
    p_img = tile_m / g.rg_per_img;
    p_oh0 = (tile_m - p_img * g.rg_per_img) * g.tr;
    mbase = (int64_t(p_img) * g.OH + p_oh0) * g.OW;
    mvalid = min(g.tr, g.OH - p_oh0) * g.OW;
  }

  // 16-byte chunk c of LDS row r sits at position c ^ row_swz(r)
  auto row_swz = [](int r) __attribute__((always_inline)) { return KB == 64 ? (r >> 2) & 3 : (r >> 1) & 7; };

  // ---- A loader state, one entry per DMA this lane takes part in.
  // Dense and 64-channel conv loaders read through buffer resources: per step a lane's
  // offset is fixed (dense: plus the step's K offset; conv: refreshed once per tap) and the
  // rest of the step's offset is a scalar, so a step costs almost no vector instructions.
  constexpr bool BUF_A = AMODE == A_DENSE || AMODE == A_CONV64;
  const __amdgpu_buffer_rsrc_t rsrc_a =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(g.a), 0, BUF_A ? g.a_bytes : 0, BUF_DWORD3);
  const __amdgpu_buffer_rsrc_t rsrc_b =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(g.b), 0, g.b_bytes, BUF_DWORD3);
  uint32_t a_vo[A_OPS1];    // dense: offset of the lane's chunk at K = 0; conv64: at the current tap
  int32_t a_px[A_OPS1];     // conv64: offset of the lane's chunk at tap (0, 0) (negative above/left of the image)
  uint32_t a_tm[A_OPS1];    // conv64: bit kh * KW + kw set where that tap reads inside the image
  int64_t a_base[A_OPS1];   // conv16 / conv4: image pixel base
  int32_t a_ih0[A_OPS1], a_iw0[A_OPS1], a_k[A_OPS1];
  bool a_ok[A_OPS1];
#pragma unroll
  for (int j = 0; j < A_OPS; ++j) {
    const int slot = (wave * A_OPS + j) * 64 + lane;
    int row, koff;
    if constexpr (AMODE == A_CONV4) {
      row = slot >> 4;
      const int p = (slot >> 2) & 3;
      koff = ((p ^ ((row >> 2) & 3)) << 4) + ((slot & 3) << 2);
    } else {
      row = slot / CPR;
      koff = ((slot % CPR) ^ row_swz(row)) << 4;
    }
    a_k[j] = koff;
    const int64_t m = m0 + row;
    a_ok[j] = m < g.M;
    a_vo[j] = OOB_OFF;
    a_px[j] = 0;
    a_tm[j] = 0;
    if constexpr (AMODE == A_DENSE) {
      if (a_ok[j]) a_vo[j] = static_cast<uint32_t>(m * g.lda + koff);
      a_base[j] = 0;
      a_ih0[j] = a_iw0[j] = 0;
    } else {
      const int32_t mm = a_ok[j] ? static_cast<int32_t>(m) : 0;
      const int32_t ohw = g.OH * g.OW;
      const int32_t img = mm / ohw;
      const int32_t rem = mm - img * ohw;
      const int32_t oh = rem / g.OW;
      const int32_t ow = rem - oh * g.OW;
      a_base[j] = int64_t(img) * g.H * g.W;
      a_ih0[j] = oh * g.SH - g.PH;
      a_iw0[j] = ow * g.SW - g.PW;
      if constexpr (AMODE == A_CONV64) {
        a_px[j] = ((img * g.H + a_ih0[j]) * g.W + a_iw0[j]) * g.C_pad + koff;
        uint32_t tm = 0;
        if (a_ok[j]) {
          for (int i = 0, t = 0; i < g.KH; ++i) {
            const bool rok = unsigned(a_ih0[j] + i * g.DH) < unsigned(g.H);
            for (int jj = 0; jj < g.KW; ++jj, ++t)
              if (rok && unsigned(a_iw0[j] + jj * g.DW) < unsigned(g.W)) tm |= 1u << t;
          }
        }
        a_tm[j] = tm;
      }
    }
  }
  // ---- B loader state (weights K-step-major: 64-byte slice kt of row n at (kt * n_pad + n) * 64).
  // Rows past n_pad read zeros at every step.
  uint32_t b_vo[B_OPS];
#pragma unroll
  for (int j = 0; j < B_OPS; ++j) {
    const int slot = (wave * B_OPS + j) * 64 + lane;
    const int row = slot / CPR;
    const int koff = ((slot % CPR) ^ row_swz(row)) << 4;
    const int n = n0 + row;
    b_vo[j] = n < g.n_pad ? static_cast<uint32_t>(((koff >> 6) * g.n_pad + n) * 64 + (koff & 63)) : OOB_OFF;
  }

  // load cursor of A_CONV64: (kernel row, kernel column, 64-channel block) of the next
  // step, its tap index and the tap's offset in the input
  int l_kh = 0, l_kw = 0, l_cb = 0, l_t = 0, l_off = 0;

  auto issue = [&](int kt, int stage) {
    int8_t* As = lds + stage * STAGE_BYTES;
    int8_t* Bs = As + A_STAGE;
    if constexpr (AMODE == A_CONV64) {
      if (l_cb == 0) {   // a new tap: the lanes whose row reads outside the image for it read zeros
#pragma unroll
        for (int j = 0; j < A_OPS; ++j)
          a_vo[j] = (a_tm[j] >> l_t) & 1 ? static_cast<uint32_t>(a_px[j] + l_off) : OOB_OFF;
      }
    }
#pragma unroll
    for (int j = 0; j < A_OPS; ++j) {
      int8_t* dst = As + (wave * A_OPS + j) * (A_ROWS_PER_OP * KB);
      if constexpr (AMODE == A_DENSE) {
        dma16_buf(rsrc_a, dst, a_vo[j] + static_cast<uint32_t>(kt * KB), 0);
      } else if constexpr (AMODE == A_CONV64) {
        dma16_buf(rsrc_a, dst, a_vo[j], static_cast<uint32_t>(l_cb * 64));
      } else if constexpr (AMODE == A_CONV16) {
        const void* src = g_zero_page;
        const int32_t k = kt * BK + a_k[j];
        if (a_ok[j] && k < g.k_real) {
          const int32_t tap = k / g.C_pad;
          const int32_t c0 = k - tap * g.C_pad;
          const int32_t kh = tap / g.KW;
          const int32_t kw = tap - kh * g.KW;
          const int32_t ih = a_ih0[j] + kh * g.DH;
          const int32_t iw = a_iw0[j] + kw * g.DW;
          if (unsigned(ih) < unsigned(g.H) && unsigned(iw) < unsigned(g.W))
            src = g.a + (a_base[j] + int64_t(ih) * g.W + iw) * g.C_pad + c0;
        }
        dma16(src, dst);
      } else {  // A_CONV4: one dword = one tap (4 channels) of kernel row kh
        const void* src = g_zero_page;
        const int32_t k = kt * BK + a_k[j];
        const int32_t kh = k / g.row_bytes;
        const int32_t kw = (k - kh * g.row_bytes) >> 2;
        const int32_t ih = a_ih0[j] + kh * g.DH;
        const int32_t iw = a_iw0[j] + kw * g.DW;
        if (a_ok[j] && kh < g.KH && kw < g.KW && unsigned(ih) < unsigned(g.H) && unsigned(iw) < unsigned(g.W))
          src = g.a + (a_base[j] + int64_t(ih) * g.W + iw) * 4;
        dma4(src, dst);
      }
    }
    const uint32_t b_soff = static_cast<uint32_t>(kt * (KB / 64) * g.n_pad * 64);
#pragma unroll
    for (int j = 0; j < B_OPS; ++j) dma16_buf(rsrc_b, Bs + (wave * B_OPS + j) * 1024, b_vo[j], b_soff);
    if constexpr (AMODE == A_CONV64) {
      l_cb += KB / 64;
      if (l_cb == g.cb_per_tap) {
        l_cb = 0;
        ++l_t;
        if (++l_kw == g.KW) {
          l_kw = 0;
          ++l_kh;
        }
        l_off = (l_kh * g.DH * g.W + l_kw * g.DW) * g.C_pad;
      }
    }
  };

  v16i acc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[b][r] = 0;

  // A_PATCH: 16-byte chunk j of patch pixel P (P = r * pc + c) sits at slot
  // P * S + j, S = C_pad / 16 + 1 in {5, 9, 17}: each pixel is followed by one
  // unused slot, so 16 consecutive pixels' chunk j lie an odd number S of
  // 16-byte groups apart and fall on 16 distinct bank groups.  A fragment's
  // address is then a per-lane constant plus a per-step uniform offset.
  const int pS = (g.C_pad >> 4) + 1;
  if constexpr (PATCH) {
#pragma unroll
    for (int j = 0; j < PATCH_OPS; ++j) {
      const int slot = (wave * PATCH_OPS + j) * 64 + lane;
      const void* src = g_zero_page;
      if (slot < g.patch_slots) {
        const int P = static_cast<int>(__umulhi(static_cast<uint32_t>(slot), g.ps_magic));
        const int chunk = slot - P * pS;            // pS - 1: the padding slot
        const int r = static_cast<int>(__umulhi(static_cast<uint32_t>(P), g.pc_magic));
        const int ih = p_oh0 - g.PH + r;
        const int iw = P - r * g.pc - g.PW;
        if (chunk < pS - 1 && unsigned(ih) < unsigned(g.H) && unsigned(iw) < unsigned(g.W))
          src = g.a + ((int64_t(p_img) * g.H + ih) * g.W + iw) * g.C_pad + chunk * 16;
      }
      dma16(src, patch + (wave * PATCH_OPS + j) * 1024);
    }
  }

  const int KT = g.k_tiles / (KB / 64);   // ring stages
#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < KT) issue(s, s);

  // Fragments of one 32-byte half (kk) of a K step: lane (row r, half h) holds
  // bytes 16h .. 16h+15 of the half for row r of each 32-row block.
  const int frag_row = lane & 31;
  const int swz = row_swz(frag_row);
  // A_PATCH: LDS byte address of each fragment row's bytes at tap (0, 0), channel
  // block 0 (its patch pixel times the pixel stride, plus the lane's 16-byte half);
  // rows past the tile's valid pixels read pixel 0 (their results are never stored)
  int p_addr0[PATCH ? FM : 1];
  if constexpr (PATCH) {
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      int p = wm * TM + i * 32 + frag_row;
      if (p >= mvalid) p = 0;
      const int orow = static_cast<int>(__umulhi(static_cast<uint32_t>(p), g.ow_magic));
      p_addr0[i] = ((orow * g.pc + (p - orow * g.OW)) * pS + (lane >> 5)) * 16;
    }
  }
  // read cursor of A_PATCH for the step being read: the byte offset of its tap and
  // channel block in the patch ((kh * pc + kw) * pixel stride + cb * 64), that tap's
  // kw, and its channel block (scalars in registers)
  int q_off = 0, q_kw = 0, q_cb = 0;
  auto load_frags = [&](int stage, int kk, int off, int cb, v4i (&af)[FM], v4i (&bf)[FN]) {
    const int8_t* As = lds + stage * STAGE_BYTES;
    const int8_t* Bs = As + A_STAGE;
    const int pc = ((2 * kk + (lane >> 5)) ^ swz) << 4;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      if constexpr (PATCH) {
        af[i] = *reinterpret_cast<const v4i*>(patch + p_addr0[i] + off + kk * 32);
      } else {
        af[i] = *reinterpret_cast<const v4i*>(As + (wm * TM + i * 32 + frag_row) * KB + pc);
      }
    }
#pragma unroll
    for (int j = 0; j < FN; ++j)
      bf[j] = *reinterpret_cast<const v4i*>(Bs + (wn * TN + j * 32 + frag_row) * KB + pc);
  };
  auto mfma_all = [&](const v4i (&af)[FM], const v4i (&bf)[FN]) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
        acc[i * FN + j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i * FN + j], 0, 0, 0);
  };

  // Software pipeline, one barrier per stage: the MFMAs of each 32-byte K
  // step run on fragments read during the previous one, and the first step
  // of stage t+1 is read (after the barrier that publishes it) while the last
  // step of stage t multiplies.
  v4i a0[FM], b0[FN], a1[FM], b1[FN];
  if constexpr (STAGES == 1) {
    issue(0, 0);
    wait_vmcnt<0>();
    block_barrier();
    load_frags(0, 0, q_off, q_cb, a0, b0);
    load_frags(0, 1, q_off, q_cb, a1, b1);
    mfma_all(a0, b0);
    mfma_all(a1, b1);
  } else {
  if (KT >= STAGES - 1) wait_vmcnt<(STAGES - 2) * OPS>(); else wait_vmcnt<0>();
  block_barrier();
  load_frags(0, 0, q_off, q_cb, a0, b0);
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt % STAGES;
#pragma unroll
    for (int kk = 0; kk + 2 < NKK; kk += 2) {   // 128-byte stages: steps 0..NKK-3
      load_frags(cur, kk + 1, q_off, q_cb, a1, b1);
      mfma_all(a0, b0);
      load_frags(cur, kk + 2, q_off, q_cb, a0, b0);
      mfma_all(a1, b1);
    }
    load_frags(cur, NKK - 1, q_off, q_cb, a1, b1);
    if constexpr (PATCH) {   // advance the cursor to step kt + 1
      q_off += 64;
      if (++q_cb == g.cb_per_tap) {
        q_cb = 0;
        q_off += pS * 16 - g.cb_per_tap * 64;        // next tap: one pixel on
        if (++q_kw == g.KW) {
          q_kw = 0;
          q_off += (g.pc - g.KW) * pS * 16;         // next kernel row: pc - KW pixels on
        }
      }
    }
    mfma_all(a0, b0);
    if (kt + 1 < KT) {
      if (kt + STAGES - 2 < KT)
        wait_vmcnt<(STAGES - 3) * OPS>();
      else
        wait_vmcnt<0>();
      block_barrier();
      if (kt + STAGES - 1 < KT) issue(kt + STAGES - 1, (kt + STAGES - 1) % STAGES);
      load_frags((kt + 1) % STAGES, 0, q_off, q_cb, a0, b0);
    }
    mfma_all(a1, b1);
  }
  }  // STAGES >= 3

  // ---- fused epilogue.  The int32 tile goes through LDS one 32-row block row
  // per wave at a time; the whole workgroup then walks those rows with each
  // thread owning 4 adjacent columns: per-column constants are read once,
  // operands and results move as 16-byte (f32) / 4-byte (int8) accesses.
  constexpr int CG = BN / 4;                        // 4-column groups per row
  constexpr int RSTEP = (WM * WN * 64) / CG;        // rows walked concurrently
  static_assert((WM * WN * 64) % CG == 0, "epilogue thread mapping");
  int32_t* ep = reinterpret_cast<int32_t*>(lds);
  const int cgi = threadIdx.x % CG;
  const int col0 = n0 + cgi * 4;
  EpiCols4 cols;
  load_cols4(e, col0, g.N, cols);

#pragma unroll
  for (int pass = 0; pass < FM; ++pass) {
    block_barrier();   // LDS free: main-loop reads / previous pass's reads are done
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        ep[(wm * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * EP_LD + wn * TN + j * 32 + (lane & 31)] =
            acc[pass * FN + j][r];
    lds_store_barrier();
    if constexpr (EF >= EF_SPEC) {
      // a partial last column tile runs here too when N % 4 == 0: a thread's 4 columns are
      // then all in range or all past N, and a thread past N computes but stores nothing
      // (its residual loads read column 0 of the row instead)
      if (n0 + BN <= g.N || (g.N & 3) == 0) {
        const bool cok = col0 < g.N;
        const int rcol = cok ? col0 : 0;
        constexpr bool S_COL = EF & SF_COL, S_FULL = EF & SF_FULL, S_LO = EF & SF_LO, S_HI = EF & SF_HI;
        constexpr bool S_F32 = EF & SF_F32, S_I8 = EF & SF_I8, S_F16 = EF & SF_F16;
        constexpr int NR = EP_ROWS / RSTEP;
        static_assert(EP_ROWS % RSTEP == 0, "epilogue rows per thread");
        // rows in flight at once: all of them, or 4 when each also holds a residual
        // (2 for the 128x256 tiles held to 128 VGPRs, whose residual forms would spill with 4)
        constexpr int NRC = S_FULL && NR > 4 ? (BM == 128 && BN == 256 && KB == 64 ? 2 : 4) : NR;
        static_assert(NR % NRC == 0, "epilogue row chunks");
        // residual rows of chunk c (rows past the tile re-read its last row); the
        // next chunk's are loaded before this chunk's stores, which the compiler
        // may not move loads across
        // an f16 graph's residual read as halves and f32 result stored as halves
        constexpr bool res_h16 = EF & SF_H16R, out_h16 = EF & SF_H16O;
        // residual rows: 4 floats, or 4 halves (uint2)
        using ResT = std::conditional_t<res_h16, uint2, float4>;
        auto load_res = [&](int c0, ResT (&res)[S_FULL ? NRC : 1]) __attribute__((always_inline)) {
          if constexpr (S_FULL) {
#pragma unroll
            for (int k = 0; k < NRC; ++k) {
              const int rr = threadIdx.x / CG + (c0 + k) * RSTEP;
              const int lk = (rr >> 5) * TM + pass * 32 + (rr & 31);
              const int64_t r = mbase + min(lk, mvalid - 1);
              if constexpr (res_h16)
                res[k] = *reinterpret_cast<const uint2*>(reinterpret_cast<const __half*>(e.full_ptr) +
                                                         r * e.full_ld + rcol);
              else
                res[k] = *reinterpret_cast<const float4*>(e.full_ptr + r * e.full_ld + rcol);
            }
          }
        };
        // the tile's result rows as raw buffers: a row past mvalid lies past num_records,
        // so its store is dropped by the hardware, and offsets are 32-bit
        const __amdgpu_buffer_rsrc_t rf = __builtin_amdgcn_make_buffer_rsrc(
            reinterpret_cast<char*>(e.out_f32) + mbase * e.ldo * (out_h16 ? 2 : 4), 0,
            S_F32 ? mvalid * int(e.ldo) * (out_h16 ? 2 : 4) : 0, BUF_DWORD3);
        const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
            e.out_i8 + mbase * e.ldq, 0, S_I8 ? mvalid * int(e.ldq) : 0, BUF_DWORD3);
        ResT res_cur[S_FULL ? NRC : 1], res_next[S_FULL ? NRC : 1];
        load_res(0, res_cur);
#pragma unroll
        for (int k0 = 0; k0 < NR; k0 += NRC) {
        int local[NRC];
        v4i a[NRC];
#pragma unroll
        for (int k = 0; k < NRC; ++k) {
          const int rr = threadIdx.x / CG + (k0 + k) * RSTEP;
          local[k] = (rr >> 5) * TM + pass * 32 + (rr & 31);
          a[k] = *reinterpret_cast<const v4i*>(ep + rr * EP_LD + cgi * 4);
        }
        float y[NRC][4];
#pragma unroll
        for (int k = 0; k < NRC; ++k) {
          const ResT rb = res_cur[S_FULL ? k : 0];
          float o[4];
          if constexpr (res_h16) {
            o[0] = half_bits(rb.x); o[1] = half_bits(rb.x >> 16); o[2] = half_bits(rb.y); o[3] = half_bits(rb.y >> 16);
          } else {
            o[0] = rb.x; o[1] = rb.y; o[2] = rb.z; o[3] = rb.w;
          }
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            float t = dequant(a[k][c], cols.scale[c]);
            if constexpr (S_COL) t = __fadd_rn(t, cols.colv[c]);
            if constexpr (S_FULL) t = __fadd_rn(t, o[c]);
            if constexpr (S_LO) t = max_bound(t, cols.lo, cols.lo_nan);
            if constexpr (S_HI) t = min_bound(t, cols.hi, cols.hi_nan);
            if constexpr (S_F16) t = round_f16(t);
            y[k][c] = t;
          }
        }
        if (k0 + NRC < NR) load_res(k0 + NRC, res_next);
#pragma unroll
        for (int k = 0; k < NRC; ++k) {
          const int lr = local[k];       // rows past mvalid: dropped by the resource's bound
          if (!cok) continue;
          if constexpr (S_F32) {
            if constexpr (out_h16) {
              const v2i v = {int(pack_halves(y[k][0], y[k][1])), int(pack_halves(y[k][2], y[k][3]))};
              const int off = (lr * int(e.ldo) + col0) * 2;
              if (e.nt_f32)
                __builtin_amdgcn_raw_buffer_store_b64(v, rf, off, 0, 2);   // nt
              else
                __builtin_amdgcn_raw_buffer_store_b64(v, rf, off, 0, 0);
            } else {
              const v4i v = {int(__float_as_uint(y[k][0])), int(__float_as_uint(y[k][1])),
                             int(__float_as_uint(y[k][2])), int(__float_as_uint(y[k][3]))};
              const int off = (lr * int(e.ldo) + col0) * 4;
              if (e.nt_f32)
                __builtin_amdgcn_raw_buffer_store_b128(v, rf, off, 0, 2);   // nt
              else
                __builtin_amdgcn_raw_buffer_store_b128(v, rf, off, 0, 0);
            }
          }
          if constexpr (S_I8)
            __builtin_amdgcn_raw_buffer_store_b32(quantize4_med3(y[k], e.out_rxs), rq, lr * int(e.ldq) + col0, 0, 0);
        }
#pragma unroll
        for (int k = 0; k < (S_FULL ? NRC : 1); ++k) res_cur[k] = res_next[k];
        }
        continue;
      }
    }
    for (int rr = threadIdx.x / CG; rr < EP_ROWS; rr += RSTEP) {
      const int local = (rr >> 5) * TM + pass * 32 + (rr & 31);
      if (local >= mvalid || col0 >= g.N) continue;
      const int64_t row = mbase + local;
      const v4i a = *reinterpret_cast<const v4i*>(ep + rr * EP_LD + cgi * 4);
      store_row4<EF != EF_GENERIC, EF < EF_SPEC || (EF & (SF_H16R | SF_H16O)) != 0>(e, cols, a, row, col0, g.N);
    }
  }
}

// ---------------------------------------------------------------- host dispatch

template <int BM, int BN, int WM, int WN, int STAGES, int AMODE, int KB = 64>
static void launch_cfg(GemmArgs g, const EpiDev& e, hipStream_t stream) {
  g.tiles_m = AMODE == A_PATCH ? static_cast<int32_t>(g.M / (int64_t(g.OH) * g.OW)) * g.rg_per_img
                               : static_cast<int32_t>((g.M + BM - 1) / BM);
  g.tiles_n = (g.N + BN - 1) / BN;
  const dim3 grid(static_cast<unsigned>(int64_t(g.tiles_m) * g.tiles_n)), block(WM * WN * 64);
#define MR_QGEMM_LAUNCH(EFV) hipLaunchKernelGGL((qgemm_kernel<BM, BN, WM, WN, STAGES, AMODE, EFV, KB>), grid, block, 0, \
                                                stream, g, e)
  // compiled forms: the conv modes of the ResNet- and MobileNet-style networks and the dense GEMM
  constexpr bool CONV_SPEC = AMODE == A_CONV64 || AMODE == A_PATCH;
  if constexpr (CONV_SPEC || AMODE == A_DENSE) {
    switch (spec_form(e)) {
      case SPEC_RELU_I8: MR_QGEMM_LAUNCH(EF_SPEC | SPEC_RELU_I8); return;
      case SPEC_BIAS_F32: MR_QGEMM_LAUNCH(EF_SPEC | SPEC_BIAS_F32); return;
      default: break;
    }
  }
  if constexpr (CONV_SPEC) {
    switch (spec_form(e)) {
      case SPEC_RES_F32_I8: MR_QGEMM_LAUNCH(EF_SPEC | SPEC_RES_F32_I8); return;
      case SPEC_RES_I8: MR_QGEMM_LAUNCH(EF_SPEC | SPEC_RES_I8); return;
      case SPEC_RES_F32: MR_QGEMM_LAUNCH(EF_SPEC | SPEC_RES_F32); return;
      // the same ResNet block forms in f16 graphs
      case SPEC_RELU_I8 | SF_F16: MR_QGEMM_LAUNCH(EF_SPEC | SPEC_RELU_I8 | SF_F16); return;
      case SPEC_RES_F32_I8 | SF_F16: MR_QGEMM_LAUNCH(EF_SPEC | SPEC_RES_F32_I8 | SF_F16); return;
      case SPEC_BIAS_F32 | SF_F16: MR_QGEMM_LAUNCH(EF_SPEC | SPEC_BIAS_F32 | SF_F16); return;
      case SPEC_RES_I8 | SF_F16: MR_QGEMM_LAUNCH(EF_SPEC | SPEC_RES_I8 | SF_F16); return;
      case SPEC_RES_F32 | SF_F16: MR_QGEMM_LAUNCH(EF_SPEC | SPEC_RES_F32 | SF_F16); return;
      // and with their f16 values stored as halves (a residual path of halves; the last
      // block's f32 result for a reader that takes f32)
      case SPEC_RES_F32_I8 | SF_F16 | SF_H16R | SF_H16O:
        MR_QGEMM_LAUNCH(EF_SPEC | SPEC_RES_F32_I8 | SF_F16 | SF_H16R | SF_H16O); return;
      case SPEC_RES_I8 | SF_F16 | SF_H16R: MR_QGEMM_LAUNCH(EF_SPEC | SPEC_RES_I8 | SF_F16 | SF_H16R); return;
      case SPEC_RES_F32 | SF_F16 | SF_H16R: MR_QGEMM_LAUNCH(EF_SPEC | SPEC_RES_F32 | SF_F16 | SF_H16R); return;
      case SPEC_BIAS_F32 | SF_F16 | SF_H16O: MR_QGEMM_LAUNCH(EF_SPEC | SPEC_BIAS_F32 | SF_F16 | SF_H16O); return;
      default: break;
    }
  }
  // the MobileNet-style forms (also for dense mode: 1x1 convolutions run as GEMMs)
  if constexpr (AMODE == A_CONV16 || AMODE == A_CONV64 || AMODE == A_CONV4 || AMODE == A_DENSE) {
    switch (spec_form(e)) {
      case SPEC_RELU6_F32: MR_QGEMM_LAUNCH(EF_SPEC | SPEC_RELU6_F32); return;
      case SPEC_BIAS_F32_I8: MR_QGEMM_LAUNCH(EF_SPEC | SPEC_BIAS_F32_I8); return;
      case SPEC_BIAS_RES_F32_I8: MR_QGEMM_LAUNCH(EF_SPEC | SPEC_BIAS_RES_F32_I8); return;
      case SPEC_BIAS_I8: MR_QGEMM_LAUNCH(EF_SPEC | SPEC_BIAS_I8); return;
      case SPEC_BIAS_RES_I8: MR_QGEMM_LAUNCH(EF_SPEC | SPEC_BIAS_RES_I8); return;
      default: break;
    }
  }
  if (e.fixed)
    MR_QGEMM_LAUNCH(EF_FIXED);
  else
    MR_QGEMM_LAUNCH(EF_GENERIC);
#undef MR_QGEMM_LAUNCH
}

template <int AMODE>
static int launch(const GemmArgs& g, const EpiDev& e, hipStream_t stream) {
  // Tile choice, measured on the ResNet-18 conv shapes and dense GEMMs: three
  // LDS stages and small enough tiles that 3-4 workgroups share a CU (their
  // epilogues and barrier waits overlap each other's MFMAs), with wave tiles
  // of 32x64 (N <= 64), 64x64 (N <= 128) or 64x64 with 8 waves over a
  // 128x256 tile (larger N; 256x256 once the grid is large).
  const int64_t cus = device_cu_count();
  const int64_t mt256 = (g.M + 255) / 256;
  MR_REQUIRE((g.M + 63) / 64 * ((g.N + 31) / 32) < (int64_t(1) << 31), "problem too large");
  if constexpr (AMODE == A_PATCH) {   // the host picks this mode for N <= 128 only
    if (g.N <= 64)
      launch_cfg<PATCH_BM64, 64, 4, 1, 3, AMODE>(g, e, stream);
    else
      launch_cfg<PATCH_BM128, 128, 2, 2, 3, AMODE>(g, e, stream);
  } else if (g.N <= 32 || (g.M + 63) / 64 * ((g.N + 31) / 32) <= 2 * cus) {
    // N <= 32, or a grid so small (the fc layer of a CNN: M = batch) that even
    // 64x32 tiles give at most two per CU: the most workgroups wins.  The ring is
    // what limits how many share a CU (LDS), so it is 3 stages, or none when K is
    // one 64-byte step (MobileNetV2 B=128: 3-channel stem 100 -> 90 us with 3
    // stages instead of 4, 32 -> 16 projection 53 -> 45 us)
    const int64_t tiles = (g.M + 63) / 64 * ((g.N + 31) / 32);
    if (g.k_tiles == 1 && AMODE == A_DENSE && tiles >= 32 * cus) {
      // a very large grid of one-step tiles (MobileNetV2's 112x112 32 -> 16 projection at
      // batch 128: 25 088 tiles of 64x32): 128-row tiles (two waves of 64x32) halve the
      // workgroups and their fixed costs
      launch_cfg<128, 32, 2, 1, 1, AMODE>(g, e, stream);
    } else if (g.k_tiles == 1) {
      launch_cfg<64, 32, 2, 1, 1, AMODE>(g, e, stream);
    } else if (g.k_tiles >= 8 && tiles <= 2 * cus) {
      // a long K on a grid of at most two tiles per CU is a chain of ring stages per
      // workgroup, each paying the load latency, and LDS is no constraint: six stages
      // in flight, and 128-byte stages where every row holds two whole 64-byte steps,
      // which halves the chain (ResNet-18 at batch 1, layer 4: 72 -> 36 stages, 25.6
      // -> 19.5 us per conv)
      if constexpr (AMODE == A_DENSE || AMODE == A_CONV64) {
        if (g.k_tiles % 2 == 0 && (AMODE == A_DENSE || g.C_pad % 128 == 0)) {
          launch_cfg<64, 32, 2, 1, 6, AMODE, 128>(g, e, stream);
          MR_LAUNCH_CHECK("qgemm");
          return MR_OK;
        }
      }
      launch_cfg<64, 32, 2, 1, 6, AMODE>(g, e, stream);
    } else {
      launch_cfg<64, 32, 2, 1, 3, AMODE>(g, e, stream);
    }
  } else if (AMODE == A_DENSE && g.k_pad <= 1024) {
    // short K (the 1x1 convolutions of a MobileNet): the launch is bound by its
    // result stores, and small tiles -- more workgroups, shorter epilogues --
    // beat the MFMA-sized ones (56x56x24->144 at batch 128: 51 us on 128x64
    // against 113 us on 256x256); 64x32 once even those give under one per CU
    const int64_t mt128 = (g.M + 127) / 128;
    const bool n128 = g.N > 64 && g.N <= 128;   // one 128-column tile (else 64-column ones)
    if (n128 ? mt128 < cus : mt128 * ((g.N + 63) / 64) < cus)
      launch_cfg<64, 32, 2, 1, 3, AMODE>(g, e, stream);
    else if (g.k_tiles == 1 && n128)
      // K in one 64-byte step: no ring, so more workgroups share a CU (MobileNetV2
      // B=128 112x112 16->96: 161 -> 152 us)
      launch_cfg<128, 128, 2, 2, 1, AMODE>(g, e, stream);
    else if (g.k_tiles == 1)
      // and 64x64 tiles of 2 waves (56x56 24->144: 53 -> 45 us; 14x14 64->384: 16 -> 14 us)
      launch_cfg<64, 64, 1, 2, 1, AMODE>(g, e, stream);
    else if (n128)
      launch_cfg<128, 128, 2, 2, 3, AMODE>(g, e, stream);
    else
      launch_cfg<128, 64, 4, 1, 3, AMODE>(g, e, stream);
  } else if (g.N <= 64) {
    launch_cfg<128, 64, 4, 1, 3, AMODE>(g, e, stream);
  } else if (g.N <= 128) {
    launch_cfg<128, 128, 2, 2, 3, AMODE>(g, e, stream);
  } else if (mt256 * ((g.N + 255) / 256) >= 4 * cus) {
    launch_cfg<256, 256, 2, 4, 3, AMODE>(g, e, stream);
  } else if constexpr (AMODE == A_DENSE || AMODE == A_CONV64) {
    // 128-byte stages (144 KB of LDS: one workgroup per CU) where every row
    // holds two whole 64-byte K steps and the grid has at most one tile per CU
    const int64_t tiles = (g.M + 127) / 128 * ((g.N + 255) / 256);
    if (g.k_tiles % 2 == 0 && (AMODE == A_DENSE || g.C_pad % 128 == 0) && tiles <= cus)
      launch_cfg<128, 256, 2, 4, 3, AMODE, 128>(g, e, stream);
    else
      launch_cfg<128, 256, 2, 4, 3, AMODE>(g, e, stream);
  } else {
    launch_cfg<128, 256, 2, 4, 3, AMODE>(g, e, stream);
  }
  MR_LAUNCH_CHECK("qgemm");
  return MR_OK;
}

static bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

// Whether an f32 result goes out with the non-temporal hint.  Results larger than the
// 256 MB Infinity Cache do (MobileNetV2 B=128 112x112 16->96 expansion: 152 -> 112 us, and
// the depthwise conv reading it 160 -> 128 us).  So do those of 96 MiB or more whose
// epilogue adds a residual: a residual block's output, whose f32 copy is next read as the
// residual two launches later (ResNet-18 B=256 layer 1/2 blocks: the two writers and their
// residual readers 2-5 us faster each).  Smaller results, and those read by the very next
// launch (MobileNetV2's 231 MB expansions feeding their depthwise convs), stay cached.
static bool stream_f32(const EpiDev& e, int64_t M) {
  if (!e.out_f32) return false;
  const int64_t bytes = M * e.ldo * (e.out_h16 ? 2 : 4);
  return bytes >= (int64_t(256) << 20) || (e.fixed && e.f_full && bytes >= (int64_t(96) << 20));
}

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
  MR_REQUIRE(N < (int64_t(1) << 30) && k_pad < (int64_t(1) << 30) && M < (int64_t(1) << 31),
             "mr_qmatmul: problem too large");
  MR_REQUIRE(K <= mr::MAX_EXACT_K, "mr_qmatmul: K %lld > %lld: int32 accumulation could overflow", (long long)K,
             (long long)mr::MAX_EXACT_K);
  MR_REQUIRE(mr::aligned16(a) && mr::aligned16(b), "mr_qmatmul: operands must be 16-byte aligned");
  mr::EpiDev e;
  int rc = mr::make_epi(epi, N, true, &e, true);
  if (rc != MR_OK) return rc;
  if (M == 0) return MR_OK;
  e.nt_f32 = mr::stream_f32(e, M);
  mr::GemmArgs g = {};
  g.a = a;
  g.lda = lda;
  g.b = b;
  g.k_pad = k_pad;
  g.M = M;
  g.N = static_cast<int32_t>(N);
  g.n_pad = static_cast<int32_t>(n_pad);
  g.k_tiles = static_cast<int32_t>(k_pad / mr::BK);
  if (M <= 8) return mr::gemv_launch(a, lda, b, k_pad, n_pad, M, N, e, static_cast<hipStream_t>(stream));
  MR_REQUIRE(M * lda < (int64_t(1) << 31) && k_pad * n_pad < (int64_t(1) << 31),
             "mr_qmatmul: operands of 2 GiB or more are not supported (32-bit buffer offsets)");
  g.a_bytes = static_cast<uint32_t>(M * lda);
  g.b_bytes = static_cast<uint32_t>(k_pad * n_pad);
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
    // the 64-channel loader keeps one bit per kernel tap (at most 32 taps)
    mode = G.c_pad % 64 == 0 && G.kh * G.kw <= 32 ? mr::A_CONV64 : mr::A_CONV16;
    k_real = G.kh * G.kw * G.c_pad;
  }
  MR_REQUIRE(k_pad >= k_real && k_pad % 64 == 0, "mr_qconv2d: k_pad %lld must be >= %d and a multiple of 64",
             (long long)k_pad, k_real);
  MR_REQUIRE(mode != mr::A_CONV64 || k_pad == k_real, "mr_qconv2d: k_pad must equal kh*kw*c_pad");
  MR_REQUIRE(n_pad >= G.o && n_pad % 32 == 0, "mr_qconv2d: n_pad %lld must be >= o and a multiple of 32",
             (long long)n_pad);
  MR_REQUIRE(int64_t(G.n) * oh * ow < (int64_t(1) << 31) && int64_t(G.n) * G.h * G.w < (int64_t(1) << 31),
             "mr_qconv2d: too many pixels");
  MR_REQUIRE(int64_t(G.c) * G.kh * G.kw <= mr::MAX_EXACT_K, "mr_qconv2d: c*kh*kw > %lld: int32 accumulation could "
             "overflow", (long long)mr::MAX_EXACT_K);
  MR_REQUIRE(mr::aligned16(x) && mr::aligned16(b), "mr_qconv2d: operands must be 16-byte aligned");
  mr::EpiDev e;
  const int rc = mr::make_epi(epi, G.o, true, &e, true);
  if (rc != MR_OK) return rc;
  const int64_t M = int64_t(G.n) * oh * ow;
  if (M == 0) return MR_OK;
  e.nt_f32 = mr::stream_f32(e, M);
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
  g.cb_per_tap = G.c_pad / 64;
  MR_REQUIRE(k_pad * n_pad < (int64_t(1) << 31),
             "mr_qconv2d: packed weights of 2 GiB or more are not supported (32-bit buffer offsets)");
  const int64_t a_bytes = int64_t(G.n) * G.h * G.w * G.c_pad;
  g.a_bytes = static_cast<uint32_t>(std::min(a_bytes, int64_t(0x7fffffff)));
  g.b_bytes = static_cast<uint32_t>(k_pad * n_pad);
  // a 1x1 stride-1 unpadded convolution reads each output pixel's own input row: it is the
  // dense GEMM [n*h*w, c_pad] x [c_pad, o] over the NHWC rows.  Its K runs to k_pad, past
  // c_pad when c_pad % 64 != 0: those bytes belong to the next pixel's row, and the
  // products vanish only because packed weights are zero for k >= kh*kw*c_pad
  if (mode != mr::A_CONV4 && G.kh == 1 && G.kw == 1 && G.sh == 1 && G.sw == 1 && G.ph == 0 && G.pw == 0) {
    g.lda = G.c_pad;
    mode = mr::A_DENSE;
  }
  // stride-1 convolutions with a halo (3x3 and the like) read A from a
  // per-tile input patch: each input pixel crosses L2 -> LDS about
  // (tr + kh - 1) / tr times instead of kh * kw times
  if (mode == mr::A_CONV64 && (G.c_pad & (G.c_pad - 1)) == 0 && G.c_pad <= 256 && G.sh == 1 && G.sw == 1 &&
      G.dh == 1 && G.dw == 1 && G.kh * G.kw > 1 && G.o <= 128 && ow <= mr::patch_bm(G.o)) {
    const int32_t tr = std::min(mr::patch_bm(G.o) / ow, oh);
    const int32_t pr = tr + G.kh - 1, pc = ow + G.kw - 1;
    const int64_t slots = int64_t(pr) * pc * (G.c_pad / 16 + 1);   // one padding slot per pixel
    // the kernel divides patch pixel indices (< pr * pc) by pc and tile rows (< patch_bm)
    // by ow through multiplier magics, exact while n * d < 2^32
    const bool magic_ok = pc >= 2 && ow >= 2 && uint64_t(pr) * pc * pc < (uint64_t(1) << 32) &&
                          uint64_t(mr::patch_bm(G.o)) * ow < (uint64_t(1) << 32);
    if (slots * 16 <= mr::PATCH_MAX && magic_ok) {
      g.ps_magic = mr::div_magic(static_cast<uint32_t>(G.c_pad / 16 + 1));
      g.pc_magic = mr::div_magic(static_cast<uint32_t>(pc));
      g.ow_magic = mr::div_magic(static_cast<uint32_t>(ow));
      g.tr = tr;
      g.rg_per_img = (oh + tr - 1) / tr;
      g.pr = pr;
      g.pc = pc;
      g.patch_slots = static_cast<int32_t>(slots);
      MR_REQUIRE(int64_t(G.n) * g.rg_per_img < (int64_t(1) << 31), "mr_qconv2d: too many tiles");
      mode = mr::A_PATCH;
    }
  }
  // the dense and 64-channel loaders read A through a buffer resource (32-bit offsets); the
  // others form 64-bit addresses
  MR_REQUIRE((mode != mr::A_DENSE && mode != mr::A_CONV64) || a_bytes < (int64_t(1) << 31),
             "mr_qconv2d: an int8 input of 2 GiB or more is not supported by this loader (32-bit buffer offsets)");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (mode) {
    case mr::A_PATCH: return mr::launch<mr::A_PATCH>(g, e, s);
    case mr::A_CONV4: return mr::launch<mr::A_CONV4>(g, e, s);
    case mr::A_CONV64: return mr::launch<mr::A_CONV64>(g, e, s);
    case mr::A_DENSE: return mr::launch<mr::A_DENSE>(g, e, s);
    default: return mr::launch<mr::A_CONV16>(g, e, s);
  }
}

}  // extern "C"
