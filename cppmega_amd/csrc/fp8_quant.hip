// Tensorwise (current-scaling) quantisation to OCP e4m3 on gfx950.
//
// Reference: per_token_cast_to_fp8 -> _te_tensorwise_cast_to_fp8
// (cppmega/megatron/sparse_mla_ops/tilelang_sparse_mla_fwd_fp8.py:74-99,396-412),
// which calls Transformer Engine's Float8CurrentScalingQuantizer: one amax
// over the tensor, scale = 448 / amax, data = e4m3(x * scale),
// scale_inv = 1 / scale.  Three stream-ordered kernels, no atomics and no
// memset (safe under graph capture): per-block maxima, a one-block final
// reduction that derives scale / scale_inv, and the elementwise cast
// (round-to-nearest-even, saturating at +-448).
#include "dsa_common.hpp"

namespace dsa {

constexpr int kQuantBlocks = 1024;

__device__ __forceinline__ float load_elem(const void *x, int64_t i, int bf16) {
  return bf16 ? bf16_bits_to_f32(static_cast<const uint16_t *>(x)[i]) : static_cast<const float *>(x)[i];
}

__global__ void __launch_bounds__(256) amax_partial_kernel(const void *x, int64_t n, int bf16, float *part) {
  __shared__ float red[4];
  float m = 0.0f;
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    m = fmaxf(m, fabsf(load_elem(x, i, bf16)));
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  if (lane_id() == 0) red[wave_id()] = m;
  __syncthreads();
  if (threadIdx.x == 0) part[blockIdx.x] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// part[0..nparts) -> ws_scale[0] = scale, scale_inv[0] = 1 / scale.
__global__ void __launch_bounds__(256) amax_final_kernel(const float *part, int nparts, float *ws_scale,
                                                         float *scale_inv) {
  __shared__ float red[4];
  float m = 0.0f;
  for (int i = threadIdx.x; i < nparts; i += 256) m = fmaxf(m, part[i]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  if (lane_id() == 0) red[wave_id()] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    const float amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float scale = (amax > 0.0f && amax <= 3.402823466e38f) ? 448.0f / amax : 1.0f;
    ws_scale[0] = scale;
    scale_inv[0] = 1.0f / scale;
  }
}

__global__ void __launch_bounds__(256) quantize_kernel(const void *x, int64_t n, int bf16, const float *ws_scale,
                                                       uint8_t *out) {
  const float scale = ws_scale[0];
  const int64_t n4 = n / 4;
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256) {
    uint32_t packed = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) packed |= f32_to_e4m3(load_elem(x, 4 * i + e, bf16) * scale) << (8 * e);
    reinterpret_cast<uint32_t *>(out)[i] = packed;
  }
  for (int64_t i = 4 * n4 + blockIdx.x * 256ll + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    out[i] = (uint8_t)f32_to_e4m3(load_elem(x, i, bf16) * scale);
}

}  // namespace dsa

using namespace dsa;

extern "C" size_t dsa_fp8_quantize_workspace_size(void) { return (kQuantBlocks + 64) * sizeof(float); }

extern "C" int dsa_fp8_tensorwise_quantize(const void *x, int64_t n, int in_dtype, uint8_t *out_fp8,
                                           float *scale_inv, void *workspace, size_t workspace_bytes,
                                           void *stream) {
  DSA_REQUIRE(n >= 0, "dsa_fp8_tensorwise_quantize: n < 0");
  DSA_REQUIRE(in_dtype == DSA_DTYPE_BF16 || in_dtype == DSA_DTYPE_F32,
              "dsa_fp8_tensorwise_quantize: input dtype must be bf16 or f32 (got %d)", in_dtype);
  DSA_REQUIRE(scale_inv, "dsa_fp8_tensorwise_quantize: null scale_inv");
  DSA_REQUIRE(n == 0 || (x && out_fp8), "dsa_fp8_tensorwise_quantize: null tensor pointer");
  if (!workspace || workspace_bytes < dsa_fp8_quantize_workspace_size())
    return set_error(DSA_ERR_WORKSPACE, "dsa_fp8_tensorwise_quantize: workspace %zu < %zu", workspace_bytes,
                     dsa_fp8_quantize_workspace_size());
  DSA_REQUIRE((reinterpret_cast<uintptr_t>(out_fp8) & 3u) == 0, "dsa_fp8_tensorwise_quantize: out must be 4-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  float *part = static_cast<float *>(workspace);
  float *ws_scale = part + kQuantBlocks;
  const int bf16 = in_dtype == DSA_DTYPE_BF16;
  int64_t blocks = (n + 255) / 256;
  if (blocks > kQuantBlocks) blocks = kQuantBlocks;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(amax_partial_kernel, dim3((unsigned)blocks), dim3(256), 0, st, x, n, bf16, part);
  hipLaunchKernelGGL(amax_final_kernel, dim3(1), dim3(256), 0, st, part, (int)blocks, ws_scale, scale_inv);
  if (n > 0) {
    int64_t qb = (n / 4 + 255) / 256;
    if (qb > 4096) qb = 4096;
    if (qb < 1) qb = 1;
    hipLaunchKernelGGL(quantize_kernel, dim3((unsigned)qb), dim3(256), 0, st, x, n, bf16, ws_scale, out_fp8);
  }
  return check_launch("fp8_tensorwise_quantize");
}
