// Shared device helpers for the gfx950 DSA kernels: MFMA operand types,
// bf16 / e4m3 conversions, wave-level reductions and the per-thread error
// slot used by the C-ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include "../../include/dsa_hip.h"

namespace dsa {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegBig = -1.0e30f;  // finite "minus infinity" for running maxima

// ---------------------------------------------------------------------------
// bf16 <-> f32 (bit exact, round-to-nearest-even; NaN stays NaN)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
// Pack two floats into one dword of bf16 (lo in the low half), round to
// nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
// Same for fp16 (v_cvt_pk_f16_f32, round to nearest even).
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  const f16x2_t v = {(_Float16)lo, (_Float16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// ---------------------------------------------------------------------------
// Power-of-two scaled fp16 rows (dKV partial rows of the backward)
// ---------------------------------------------------------------------------
// Scale exponent s for a row whose max magnitude is amax: amax * 2^s lies in
// [2^13, 2^14), so the whole row fits fp16 with 11 significant bits relative
// to its max.  Zero, inf or NaN rows use s = 0.  |s| <= 127 fits an int8.
__device__ __forceinline__ int partial_row_exponent(float amax) {
  if (!(amax > 0.0f) || !(amax <= 3.402823466e38f)) return 0;
  int ex;
  (void)frexpf(amax, &ex);  // amax = m * 2^ex, m in [0.5, 1)
  int s = 14 - ex;
  s = s > 127 ? 127 : (s < -114 ? -114 : s);
  return s;
}
// The same exponent from an upper bound bnd of the row's magnitudes, known
// before the row is computed: bnd * 2^s lies in [2^15, 2^16).  Callers pass
// bnd with a relative margin of at least 2^-6 over every rounding in the row's
// computation, so each element scales below 2^16 / (1 + 2^-6) < 64528, inside
// fp16's finite range (65504).
__device__ __forceinline__ int partial_row_exponent_bound(float bnd) {
  if (!(bnd > 0.0f) || !(bnd <= 3.402823466e38f)) return 0;
  int ex;
  (void)frexpf(bnd, &ex);
  int s = 16 - ex;
  s = s > 127 ? 127 : (s < -114 ? -114 : s);
  return s;
}
// max |x| over the 8 bf16 values of v (NaNs ignored, as fmaxf does).
__device__ __forceinline__ float bf16x8_absmax(i32x4 v) {
  float m = 0.0f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t u = (uint32_t)v[e];
    m = fmaxf(m, fmaxf(__uint_as_float((u << 16) & 0x7fff0000u), __uint_as_float(u & 0x7fff0000u)));
  }
  return m;
}
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  const _Float16 h = (_Float16)f;  // round to nearest even
  return (uint32_t)__builtin_bit_cast(uint16_t, h);
}
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}
// 2^x by the hardware exp (v_exp_f32, ~1 ulp); results below the normal range
// flush to zero, which softmax weights in [0, 1] rounded to bf16 do not notice.
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// 2^s as a float for |s| <= 127 (exact).
__device__ __forceinline__ float exp2i(int s) { return ldexpf(1.0f, s); }

// ---------------------------------------------------------------------------
// OCP e4m3fn (bias 7, 3 mantissa bits, 0x7f / 0xff = NaN, max 448)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float e4m3_to_f32(uint32_t c) {
  const uint32_t s = (c & 0x80u) << 24;
  const uint32_t e = (c >> 3) & 0xfu;
  const uint32_t m = c & 0x7u;
  if (e == 0xfu && m == 0x7u) return __uint_as_float(s | 0x7fc00000u);
  if (e == 0) {  // subnormal: m * 2^-9, exact in fp32 (sign kept for m == 0)
    const float v = (float)m * 0.001953125f;
    return s ? -v : v;
  }
  return __uint_as_float(s | ((e + 120u) << 23) | (m << 20));
}

// Two e4m3 codes -> two exact floats by the hardware conversion
// (v_cvt_pk_f32_fp8, OCP e4m3fn on gfx950): bytes 0 and 1 of `word` when
// hi == false, bytes 2 and 3 when hi == true.  Same values as e4m3_to_f32
// (checked for all 256 codes through dsa_fp8_dequantize by the GPU tests).
typedef float f32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ f32x2 e4m3x2_to_f32(uint32_t word, bool hi) {
  return hi ? __builtin_amdgcn_cvt_pk_f32_fp8((int)word, true) : __builtin_amdgcn_cvt_pk_f32_fp8((int)word, false);
}

// Eight e4m3 codes (lo: bytes 0-3, hi: bytes 4-7) times one scale, as bf16
// (round to nearest even).  Exact when the scale is a power of two within
// mx_scale_exact's range: a code has at most 4 significant bits.
__device__ __forceinline__ bf16x8 e4m3x8_to_bf16_scaled(uint32_t lo, uint32_t hi, float s) {
  uint32_t w[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const f32x2 v2 = e4m3x2_to_f32(e < 2 ? lo : hi, (e & 1) != 0);
    w[e] = pack_bf16x2(v2[0] * s, v2[1] * s);
  }
  return __builtin_bit_cast(bf16x8, i32x4{(int)w[0], (int)w[1], (int)w[2], (int)w[3]});
}

// A block scale for which code * scale is exact in bf16 (and in fp32) for every
// e4m3 code: zero, or a power of two in [2^-40, 2^40], so the scaled values,
// their products and a d_qk-long sum of them stay normal and finite in fp32.
// OCP MX scales (E8M0) are powers of two.
__device__ __forceinline__ bool mx_scale_exact(float s) {
  const uint32_t u = __float_as_uint(s) & 0x7fffffffu;
  if (u == 0u) return true;
  const uint32_t e = u >> 23;
  return (u & 0x7fffffu) == 0u && e >= 87u && e <= 167u;
}

// Round-to-nearest-even, saturating at +-448; NaN -> 0x7f (sign kept).
__device__ __forceinline__ uint32_t f32_to_e4m3(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t s = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return s | 0x7fu;
  const float af = __uint_as_float(a);
  if (af >= 448.0f) return s | 0x7eu;
  if (af < 0.015625f) {  // below 2^-6: subnormal grid of 2^-9
    const float qv = __builtin_rintf(af * 512.0f);  // exact scaling, RNE
    return s | (uint32_t)qv;                        // 8 -> 0x08 = 2^-6
  }
  int32_t e = (int32_t)(a >> 23) - 127;  // -6 .. 8
  uint32_t mant = a & 0x7fffffu;
  uint32_t r = mant >> 20;
  const uint32_t rem = mant & 0xfffffu;
  if (rem > 0x80000u || (rem == 0x80000u && (r & 1u))) ++r;
  if (r == 8u) { r = 0; ++e; }
  uint32_t code = ((uint32_t)(e + 7) << 3) | r;
  if (code > 0x7eu) code = 0x7eu;
  return s | code;
}

// ---------------------------------------------------------------------------
// Wave helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & 63u); }
// Wave index within the workgroup, made explicitly wave-uniform (an SGPR), so
// that addresses and branches derived from it stay scalar.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

__device__ __forceinline__ float xor32(float v) { return __shfl_xor(v, 32, 64); }

// x(lane) + x(lane ^ 32) in every lane, by one v_permlane32_swap (the swap
// leaves lanes 0-31 of the first result holding the low half and lanes 0-31 of
// the second holding the high half, mirrored for lanes 32-63); the sum is
// low + high in both halves, so both get the same bits.
__device__ __forceinline__ float sum_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// max(x(lane), x(lane ^ 32)) in every lane, the same way.
__device__ __forceinline__ float max_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Make this wave's LDS writes visible to its own other lanes.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ bf16x8 as_bf16x8(i32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// ---------------------------------------------------------------------------
// Transposed LDS reads (ds_read_b64_tr_b16, gfx950)
// ---------------------------------------------------------------------------
// Within each group of 16 lanes, lane k supplies the address of 4 consecutive
// 16-bit elements M[k][0..3]; lane i receives {M[i/4][i%4], M[4 + i/4][i%4],
// M[8 + i/4][i%4], M[12 + i/4][i%4]}.  With lane k = 4j + q pointing at
// T[row_j][col0 + 4q], lane i therefore receives column col0 + i of rows
// row_0..row_3: a 4x16 block of a row-major tile, transposed.
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

__device__ __forceinline__ i32x2 ds_read_tr16(const unsigned char *p) {
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(const_cast<unsigned char *>(p)));
  return __builtin_bit_cast(i32x2, v);
}

// 32x32x16 MFMA operand whose M/N index (lane & 31) is column col0 + (lane & 31)
// of the row-major bf16 tile T (row stride `stride` bytes) and whose eight
// K elements e = 4h + j (h = 0, 1; j = 0..3) are rows
//   row(e) = rows_base + h * h_step + (lane >> 5) * g_step + j.
// (h_step, g_step) = (4, 8) gives rows rows_base + 8 * (lane >> 5) + e; (8, 4)
// gives the accumulator order rows_base + 8h + 4 * (lane >> 5) + j.
__device__ __forceinline__ i32x4 tr_operand(const unsigned char *T, int stride, int col0, int rows_base,
                                            int h_step, int g_step) {
  const int lane = lane_id();
  const int k = lane & 15, j = k >> 2, q = k & 3, cb = (lane >> 4) & 1, gg = lane >> 5;
  const unsigned char *base = T + (col0 + cb * 16 + 4 * q) * 2 + (rows_base + gg * g_step + j) * stride;
  const i32x2 r0 = ds_read_tr16(base);
  const i32x2 r1 = ds_read_tr16(base + h_step * stride);
  return i32x4{r0[0], r0[1], r1[0], r1[1]};
}

// tr_operand(T, stride, col0, rows_base, 8, 4) over a tile whose 16-byte
// chunks are swizzled by row bit 3 (chunk c of row R at c ^ ((R >> 3) & 1),
// gather_store_k<..., true>): rows_base is a multiple of 16, so the first
// read's rows have bit 3 clear and the second's (8 rows on) set.
__device__ __forceinline__ i32x4 tr_operand_swz(const unsigned char *T, int stride, int col0, int rows_base) {
  const int lane = lane_id();
  const int k = lane & 15, j = k >> 2, q = k & 3, cb = (lane >> 4) & 1, gg = lane >> 5;
  const int col = (col0 + cb * 16 + 4 * q) * 2;  // bytes
  const unsigned char *row0 = T + (rows_base + gg * 4 + j) * stride;
  const i32x2 r0 = ds_read_tr16(row0 + col);
  const i32x2 r1 = ds_read_tr16(row0 + 8 * stride + (col ^ 16));
  return i32x4{r0[0], r0[1], r1[0], r1[1]};
}

// tr_operand with (h_step, g_step) = (8, 4) and the four 4-column groups of
// each 16-column half permuted, so that accumulator row m = 8i + 4g + j of the
// product maps to column col0 + 16(i >> 1) + 8g + 4(i & 1) + j: a lane's 16
// accumulator values then cover two runs of 8 consecutive columns (16-byte
// stores), and the two lane halves' runs are adjacent.
__device__ __forceinline__ i32x4 tr_operand_perm(const unsigned char *T, int stride, int col0, int rows_base) {
  const int lane = lane_id();
  const int k = lane & 15, j = k >> 2, q = k & 3, cb = (lane >> 4) & 1, gg = lane >> 5;
  const unsigned char *base =
      T + (col0 + cb * 16 + 8 * (q & 1) + 4 * (q >> 1)) * 2 + (rows_base + gg * 4 + j) * stride;
  const i32x2 r0 = ds_read_tr16(base);
  const i32x2 r1 = ds_read_tr16(base + 8 * stride);
  return i32x4{r0[0], r0[1], r1[0], r1[1]};
}

// Streaming (non-temporal) 16-byte global store / load: for data written once
// and read once much later (the backward's partial dKV rows), so it neither
// lingers as dirty lines in the caches nor evicts the working set of the
// kernels in between.
__device__ __forceinline__ void st_stream_16(void *p, i32x4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<i32x4 *>(p));
}
__device__ __forceinline__ void st_stream_16(void *p, f32x4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<f32x4 *>(p));
}
__device__ __forceinline__ i32x4 ld_stream_16(const void *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const i32x4 *>(p));
}

__device__ __forceinline__ i32x4 ld_global_16(const void *p) {
  return *reinterpret_cast<const i32x4 *>(p);
}
__device__ __forceinline__ i32x2 ld_global_8(const void *p) {
  return *reinterpret_cast<const i32x2 *>(p);
}

// Raw buffer access: a resource covering `num_bytes` from `base`; loads at byte
// offsets outside it return 0 instead of touching memory (gfx9-family
// descriptor word 3 = 0x00020000).
// The base and size are wave-uniform by contract; they are read from the
// first lane so the descriptor lives in SGPRs even where the compiler cannot
// prove uniformity (otherwise every access becomes a waterfall loop).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_buffer_rsrc(const void *base, uint32_t num_bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  void *pb = reinterpret_cast<void *>(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(pb, (short)0, (int)__builtin_amdgcn_readfirstlane(num_bytes), 0x00020000);
}
__device__ __forceinline__ float buffer_load_f32(__amdgpu_buffer_rsrc_t r, int voffset, int soffset) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voffset, soffset, 0));
}

// Remap a linear block id so that consecutive logical blocks land on the
// same XCD (blocks are dispatched round-robin over the 8 XCDs of MI355X).
__device__ __forceinline__ int64_t xcd_remap(int64_t bid, int64_t nblocks) {
  if (nblocks % 8 != 0) return bid;
  const int64_t per = nblocks / 8;
  return (bid % 8) * per + bid / 8;
}

}  // namespace dsa

// ---------------------------------------------------------------------------
// Host-side status helpers (defined in dsa_abi.hip)
// ---------------------------------------------------------------------------
namespace dsa {
int set_error(int code, const char *fmt, ...);
int check_launch(const char *what);
// Top-k over nbatch batches of rows in one launch (defined in topk_select.hip).
int topk_batched(const float *scores, int64_t rows_per_batch, int64_t nbatch, int64_t row_len, int64_t row_stride,
                 int causal, int64_t causal_offset, int64_t topk, int32_t *out, int64_t out_bstride,
                 void *ws, size_t ws_bytes, hipStream_t st);
// Stage timing of multi-kernel entry points (no-ops unless dsa_stage_timing(1)).
void stage_begin(hipStream_t st);
void stage_mark(hipStream_t st);
}  // namespace dsa

#define DSA_REQUIRE(cond, ...)                                   \
  do {                                                           \
    if (!(cond)) return ::dsa::set_error(DSA_ERR_INVALID_ARG, __VA_ARGS__); \
  } while (0)
