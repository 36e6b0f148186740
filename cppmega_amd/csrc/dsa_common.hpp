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
// Pack two floats into one dword of bf16 (lo in the low half).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}

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
__device__ __forceinline__ int wave_id() { return (int)(threadIdx.x >> 6); }

__device__ __forceinline__ float xor32(float v) { return __shfl_xor(v, 32, 64); }

// Make this wave's LDS writes visible to its own other lanes.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ bf16x8 as_bf16x8(i32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ i32x4 ld_global_16(const void *p) {
  return *reinterpret_cast<const i32x4 *>(p);
}
__device__ __forceinline__ i32x2 ld_global_8(const void *p) {
  return *reinterpret_cast<const i32x2 *>(p);
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
}  // namespace dsa

#define DSA_REQUIRE(cond, ...)                                   \
  do {                                                           \
    if (!(cond)) return ::dsa::set_error(DSA_ERR_INVALID_ARG, __VA_ARGS__); \
  } while (0)
