// Wave-wide reductions, scans and lane reads on gfx950 without LDS: DPP row
// operations within each 16-lane row, then readlane across the four rows.
#pragma once

#include "dsa_common.hpp"

namespace dsa {
namespace wv {

template <int CTRL, int ROW_MASK = 0xf, bool BOUND_ZERO = false>
__device__ __forceinline__ uint32_t dpp(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xf, BOUND_ZERO);
}
// lanes whose predicate holds (the compare result itself, no 0/1 round trip)
__device__ __forceinline__ uint64_t ballot(bool b) { return __builtin_amdgcn_ballot_w64(b); }
__device__ __forceinline__ uint32_t readlane(uint32_t v, int l) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, l);
}
// every lane of each 16-lane row gets op over the row
template <class Op>
__device__ __forceinline__ uint32_t row_reduce(uint32_t x, Op op) {
  x = op(x, dpp<0xB1>(x));   // quad_perm [1,0,3,2]
  x = op(x, dpp<0x4E>(x));   // quad_perm [2,3,0,1]
  x = op(x, dpp<0x141>(x));  // row_half_mirror
  x = op(x, dpp<0x140>(x));  // row_mirror
  return x;
}
template <class Op>
__device__ __forceinline__ uint32_t wave_reduce(uint32_t x, Op op) {
  x = row_reduce(x, op);
  return op(op(readlane(x, 0), readlane(x, 16)), op(readlane(x, 32), readlane(x, 48)));
}
struct MinU { __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a < b ? a : b; } };
struct MaxU { __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a > b ? a : b; } };
struct AddU { __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a + b; } };
struct OrU { __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a | b; } };
struct MinF {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const {
    return __float_as_uint(fminf(__uint_as_float(a), __uint_as_float(b)));
  }
};
struct MaxF {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const {
    return __float_as_uint(fmaxf(__uint_as_float(a), __uint_as_float(b)));
  }
};
// inclusive prefix sum over the wave
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t x) {
  x += dpp<0x111, 0xf, true>(x);  // row_shr:1
  x += dpp<0x112, 0xf, true>(x);  // row_shr:2
  x += dpp<0x114, 0xf, true>(x);  // row_shr:4
  x += dpp<0x118, 0xf, true>(x);  // row_shr:8
  x += dpp<0x142, 0xa>(x);        // row_bcast:15 into rows 1, 3
  x += dpp<0x143, 0xc>(x);        // row_bcast:31 into rows 2, 3
  return x;
}
}  // namespace wv

}  // namespace dsa
