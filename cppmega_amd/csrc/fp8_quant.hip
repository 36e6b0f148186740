// Tensorwise (current-scaling) quantisation to OCP e4m3 on gfx950.
//
// Reference: per_token_cast_to_fp8 -> _te_tensorwise_cast_to_fp8
// (cppmega/megatron/sparse_mla_ops/tilelang_sparse_mla_fwd_fp8.py:74-99,396-412),
// which calls Transformer Engine's Float8CurrentScalingQuantizer: one amax
// over the tensor, scale = 448 / amax, data = e4m3(x * scale),
// scale_inv = 1 / scale.  Three stream-ordered kernels, no atomics and no
// memset (safe under graph capture): per-block maxima, a one-block final
// reduction that derives scale / scale_inv, and the elementwise cast
// (round-to-nearest-even, saturating at +-448).  dsa_fp8_dequantize is the
// inverse view (code value * scale_inv, the reference's Float8Tensor
// dequantize) through the hardware e4m3 conversion the SparseMLA kernels use.
#include <mutex>

#include "dsa_common.hpp"

namespace dsa {

constexpr int kQuantBlocks = 1024;
constexpr int kQuantScratchFloats = kQuantBlocks + 64;  // block maxima, then the scale

// Scratch of dsa_fp8_tensorwise_quantize_noalloc: one copy per GPU, held
// until the process ends.  Host code never uses this name as an address (it
// is a host-side stand-in there); it uses the per-device pointer that
// hipGetSymbolAddress returns below.
static __device__ __align__(256) float scratch[kQuantScratchFloats];

__device__ __forceinline__ float load_elem(const void *x, int64_t i, int bf16) {
  return bf16 ? bf16_bits_to_f32(static_cast<const uint16_t *>(x)[i]) : static_cast<const float *>(x)[i];
}

// Per-block max |x| (NaN ignored).  With a 16-byte aligned x every thread
// reads 16-byte chunks (8 bf16 or 4 f32), four chunks in flight per loop trip.
__global__ void __launch_bounds__(256) amax_partial_kernel(const void *x, int64_t n, int bf16, int vec, float *part) {
  __shared__ float red[4];
  float m = 0.0f;
  const int64_t tid = blockIdx.x * 256ll + threadIdx.x, nth = (int64_t)gridDim.x * 256;
  int64_t head = 0;  // elements covered by whole chunks
  if (vec) {
    const int per = bf16 ? 8 : 4;
    const int64_t nch = n / per;
    head = nch * per;
    const i32x4 *xc = static_cast<const i32x4 *>(x);
#pragma unroll 4
    for (int64_t i = tid; i < nch; i += nth) {
      const i32x4 v = xc[i];
      if (bf16) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t w = (uint32_t)v[e];
          m = fmaxf(m, fmaxf(fabsf(__uint_as_float(w << 16)), fabsf(__uint_as_float(w & 0xffff0000u))));
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) m = fmaxf(m, fabsf(__int_as_float(v[e])));
      }
    }
  }
  for (int64_t i = head + tid; i < n; i += nth) m = fmaxf(m, fabsf(load_elem(x, i, bf16)));
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

// Four floats -> four e4m3 codes by the hardware pair conversion
// (v_cvt_pk_fp8_f32, round to nearest even).  Inputs are clamped to +-448
// first, which gives the saturating encoding of f32_to_e4m3; a NaN input keeps
// that encoding's code (sign | 0x7f).
__device__ __forceinline__ uint32_t e4m3x4_encode(float a, float b, float c, float d) {
  const float v[4] = {a, b, c, d};
  float cl[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) cl[e] = fminf(fmaxf(v[e], -448.0f), 448.0f);
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(cl[0], cl[1], 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(cl[2], cl[3], w, true);
  uint32_t out = (uint32_t)w;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (v[e] != v[e])
      out = (out & ~(0xffu << (8 * e))) | (((__float_as_uint(v[e]) >> 24) & 0x80u | 0x7fu) << (8 * e));
  return out;
}

// Elementwise cast.  With a 16-byte aligned x (and 8-byte aligned out) every
// thread converts chunks of 8 elements: 16 (bf16) or 32 (f32) bytes in, one
// 8-byte store of 8 codes out.
__global__ void __launch_bounds__(256) quantize_kernel(const void *x, int64_t n, int bf16, int vec,
                                                       const float *ws_scale, uint8_t *out) {
  const float scale = ws_scale[0];
  const int64_t tid = blockIdx.x * 256ll + threadIdx.x, nth = (int64_t)gridDim.x * 256;
  int64_t head = 0;
  if (vec) {
    const int64_t n8 = n / 8;
    head = n8 * 8;
#pragma unroll 2
    for (int64_t i = tid; i < n8; i += nth) {
      float f[8];
      if (bf16) {
        const i32x4 v = static_cast<const i32x4 *>(x)[i];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          f[2 * e] = __uint_as_float((uint32_t)v[e] << 16);
          f[2 * e + 1] = __uint_as_float((uint32_t)v[e] & 0xffff0000u);
        }
      } else {
        const i32x4 v0 = static_cast<const i32x4 *>(x)[2 * i], v1 = static_cast<const i32x4 *>(x)[2 * i + 1];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          f[e] = __int_as_float(v0[e]);
          f[4 + e] = __int_as_float(v1[e]);
        }
      }
      float y[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = f[e] * scale;
      const uint32_t lo = e4m3x4_encode(y[0], y[1], y[2], y[3]);
      const uint32_t hi = e4m3x4_encode(y[4], y[5], y[6], y[7]);
      reinterpret_cast<i32x2 *>(out)[i] = i32x2{(int)lo, (int)hi};
    }
  }
  for (int64_t i = head + tid; i < n; i += nth) out[i] = (uint8_t)f32_to_e4m3(load_elem(x, i, bf16) * scale);
}

// e4m3 codes -> code value * scale as bf16 (RNE) or f32, four codes per
// thread through the hardware pair conversion; scale = scale_inv[0]
// (block == 0) or scale_inv[i / block] (block a multiple of 4: one scale per
// `block` consecutive elements, e.g. 32 for MXFP8 rows).
__global__ void __launch_bounds__(256) dequantize_kernel(const uint8_t *x, int64_t n, const float *scale_inv,
                                                         int64_t block, int out_bf16, void *out) {
  const int64_t tid = blockIdx.x * 256ll + threadIdx.x, nth = (int64_t)gridDim.x * 256;
  for (int64_t i = tid; 4 * i < n; i += nth) {
    const float s = block ? scale_inv[(4 * i) / block] : scale_inv[0];
    uint32_t w = 0;
    const int64_t rem = n - 4 * i;
    if (rem >= 4 && (reinterpret_cast<uintptr_t>(x) & 3u) == 0) {
      w = reinterpret_cast<const uint32_t *>(x)[i];
    } else {
      for (int e = 0; e < 4 && e < rem; ++e) w |= (uint32_t)x[4 * i + e] << (8 * e);
    }
    const f32x2 a = e4m3x2_to_f32(w, false), b = e4m3x2_to_f32(w, true);
    const float v[4] = {a[0] * s, a[1] * s, b[0] * s, b[1] * s};
    for (int e = 0; e < 4 && e < rem; ++e) {
      if (out_bf16)
        static_cast<uint16_t *>(out)[4 * i + e] = (uint16_t)f32_to_bf16_bits(v[e]);
      else
        static_cast<float *>(out)[4 * i + e] = v[e];
    }
  }
}

}  // namespace dsa

using namespace dsa;

extern "C" size_t dsa_fp8_quantize_workspace_size(void) { return kQuantScratchFloats * sizeof(float); }

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
  const int vec = (reinterpret_cast<uintptr_t>(x) & 15u) == 0 && (reinterpret_cast<uintptr_t>(out_fp8) & 7u) == 0;
  hipLaunchKernelGGL(amax_partial_kernel, dim3((unsigned)blocks), dim3(256), 0, st, x, n, bf16, vec, part);
  hipLaunchKernelGGL(amax_final_kernel, dim3(1), dim3(256), 0, st, part, (int)blocks, ws_scale, scale_inv);
  if (n > 0) {
    int64_t qb = (n / 8 + 255) / 256;
    if (qb > 4096) qb = 4096;
    if (qb < 1) qb = 1;
    hipLaunchKernelGGL(quantize_kernel, dim3((unsigned)qb), dim3(256), 0, st, x, n, bf16, vec, ws_scale, out_fp8);
  }
  return check_launch("fp8_tensorwise_quantize");
}

// Device address of `scratch` on the current device, looked up once per device.
static int quant_scratch(float **out) {
  static std::mutex mu;
  static float *addr[64] = {nullptr};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(DSA_ERR_HIP, "dsa_fp8_tensorwise_quantize_noalloc: hipGetDevice: %s",
                                        hipGetErrorString(e));
  if (dev < 0 || dev >= 64) return set_error(DSA_ERR_UNSUPPORTED, "dsa_fp8_tensorwise_quantize_noalloc: device %d", dev);
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(DSA_ERR_HIP, "dsa_fp8_tensorwise_quantize_noalloc: hipGetSymbolAddress(scratch): %s",
                       hipGetErrorString(e));
    addr[dev] = static_cast<float *>(p);
  }
  *out = addr[dev];
  return DSA_OK;
}

extern "C" int dsa_fp8_tensorwise_quantize_noalloc(const void *x, int64_t n, int in_dtype, uint8_t *out_fp8,
                                                   float *scale_inv, void *stream) {
  static_assert(sizeof(scratch) >= kQuantScratchFloats * sizeof(float), "scratch holds the quantiser workspace");
  const size_t need = dsa_fp8_quantize_workspace_size();
  if (need > sizeof(scratch))
    return set_error(DSA_ERR_WORKSPACE, "dsa_fp8_tensorwise_quantize_noalloc: needs %zu scratch bytes, the "
                                        "static scratch holds %zu", need, sizeof(scratch));
  float *ws = nullptr;
  const int rc = quant_scratch(&ws);
  if (rc) return rc;
  // Every element of the scratch that a call reads is written earlier in the
  // same call (block maxima, then the scale), so nothing needs clearing.
  return dsa_fp8_tensorwise_quantize(x, n, in_dtype, out_fp8, scale_inv, ws, sizeof(scratch), stream);
}

static int dequantize(const uint8_t *x_fp8, int64_t n, const float *scale_inv, int64_t block, void *out,
                      int out_dtype, void *stream) {
  DSA_REQUIRE(n >= 0, "dsa_fp8_dequantize: n < 0");
  DSA_REQUIRE(out_dtype == DSA_DTYPE_BF16 || out_dtype == DSA_DTYPE_F32,
              "dsa_fp8_dequantize: output dtype must be bf16 or f32 (got %d)", out_dtype);
  if (n == 0) return DSA_OK;
  DSA_REQUIRE(x_fp8 && scale_inv && out, "dsa_fp8_dequantize: null pointer");
  int64_t blocks = (n / 4 + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(dequantize_kernel, dim3((unsigned)blocks), dim3(256), 0, static_cast<hipStream_t>(stream), x_fp8,
                     n, scale_inv, block, out_dtype == DSA_DTYPE_BF16 ? 1 : 0, out);
  return check_launch("fp8_dequantize");
}

extern "C" int dsa_fp8_dequantize(const uint8_t *x_fp8, int64_t n, const float *scale_inv, void *out,
                                  int out_dtype, void *stream) {
  return dequantize(x_fp8, n, scale_inv, 0, out, out_dtype, stream);
}

extern "C" int dsa_fp8_dequantize_blockwise(const uint8_t *x_fp8, int64_t n, int64_t block, const float *scales,
                                            void *out, int out_dtype, void *stream) {
  DSA_REQUIRE(block > 0 && block % 4 == 0, "dsa_fp8_dequantize_blockwise: block %lld is not a positive multiple of 4",
              (long long)block);
  return dequantize(x_fp8, n, scales, block, out, out_dtype, stream);
}
