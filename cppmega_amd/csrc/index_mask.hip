// Top-k index mask of the DSA sparse indexer loss on gfx950.
//
// Reference: Megatron's _scatter_topk_into_index_mask in the CUDA-graph-safe
// form cppmega patches in (cppmega/megatron/upstream_patches/apply_dsa_cg_patches.py:267-291,
// restated with its eager oracle in
// upstream_prs/examples/01_dsa_cuda_graph_safety/reproducer.py:90-138): rows
// [s0, s1) of a [b, s_q, s_kv] mask that the caller filled with -inf get 0 at
// every top-k column, -1 sentinels are skipped.  The upstream form branches on
// device reductions (host syncs); the patched one clamps sentinels to column 0
// and repairs column 0 afterwards with four extra tensor passes.
//
// Here either kernel is a single launch with no host synchronisation:
//  * index_mask_scatter_kernel  one thread per (row, slot): writes `value` at
//    the listed column when it lies in [0, s_kv) -- the in-place scatter of
//    the reference, every other element untouched;
//  * index_mask_fill_kernel     one workgroup per row: the row's columns are
//    collected as a bitmask in LDS, then the whole row is written once,
//    `value` on listed columns and `fill` elsewhere (16-byte stores), which
//    replaces the caller's full -inf fill plus the scatter.
// Both are idempotent and order-free (every write of an element stores the
// same value), so they are deterministic and replay identically in a graph.
#include "dsa_common.hpp"

namespace dsa {
namespace imask {

constexpr int kNT = 256;
constexpr int kMaxWords = 8192;  // fill mode: s_kv <= 262144 columns per row

struct Params {
  const void *idx;     // [B, rows, K] int32 / int64
  float *mask;         // [B, Sq, Sk]
  int64_t B, Sq, Sk, row0, rows, K;
  int i64;
  float value, fill;
};

__device__ __forceinline__ int64_t load_idx(const Params &p, int64_t i) {
  return p.i64 ? static_cast<const int64_t *>(p.idx)[i] : (int64_t) static_cast<const int32_t *>(p.idx)[i];
}

__global__ void __launch_bounds__(kNT) index_mask_scatter_kernel(Params p) {
  const int64_t i = (int64_t)blockIdx.x * kNT + threadIdx.x;
  if (i >= p.B * p.rows * p.K) return;
  const int64_t s = load_idx(p, i);
  if (s < 0 || s >= p.Sk) return;
  const int64_t br = i / p.K, b = br / p.rows, r = br % p.rows;
  p.mask[(b * p.Sq + p.row0 + r) * p.Sk + s] = p.value;
}

__global__ void __launch_bounds__(kNT) index_mask_fill_kernel(Params p) {
  __shared__ uint32_t bits[kMaxWords];
  const int64_t br = blockIdx.x, b = br / p.rows, r = br % p.rows;
  const int W = (int)((p.Sk + 31) / 32);
  for (int i = threadIdx.x; i < W; i += kNT) bits[i] = 0u;
  __syncthreads();
  for (int64_t j = threadIdx.x; j < p.K; j += kNT) {
    const int64_t s = load_idx(p, br * p.K + j);
    if (s >= 0 && s < p.Sk) atomicOr(&bits[s >> 5], 1u << (s & 31));
  }
  __syncthreads();
  float *out = p.mask + (b * p.Sq + p.row0 + r) * p.Sk;
  if ((p.Sk & 3) == 0) {  // 16-byte aligned rows
    for (int64_t s = 4 * (int64_t)threadIdx.x; s < p.Sk; s += 4 * kNT) {
      const uint32_t w = bits[s >> 5] >> (s & 31);
      f32x4 v;
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = ((w >> j) & 1u) ? p.value : p.fill;
      *reinterpret_cast<f32x4 *>(out + s) = v;
    }
  } else {
    for (int64_t s = threadIdx.x; s < p.Sk; s += kNT)
      out[s] = ((bits[s >> 5] >> (s & 31)) & 1u) ? p.value : p.fill;
  }
}

}  // namespace imask
}  // namespace dsa

extern "C" int dsa_topk_index_mask(const void *topk_indices, int topk_dtype, int64_t topk, float *mask,
                                   int64_t B, int64_t Sq, int64_t Sk, int64_t row0, int64_t rows, float value,
                                   float fill, int fill_rows, void *stream) {
  using namespace dsa;
  using namespace dsa::imask;
  DSA_REQUIRE(mask, "dsa_topk_index_mask: null mask");
  DSA_REQUIRE(B > 0 && Sq > 0 && Sk > 0 && rows >= 0 && topk >= 0,
              "dsa_topk_index_mask: bad shape B=%lld Sq=%lld Sk=%lld rows=%lld topk=%lld", (long long)B,
              (long long)Sq, (long long)Sk, (long long)rows, (long long)topk);
  DSA_REQUIRE(row0 >= 0 && row0 + rows <= Sq, "dsa_topk_index_mask: rows [%lld, %lld) outside [0, %lld)",
              (long long)row0, (long long)(row0 + rows), (long long)Sq);
  DSA_REQUIRE(topk == 0 || topk_indices, "dsa_topk_index_mask: null indices");
  DSA_REQUIRE(topk_dtype == DSA_DTYPE_I32 || topk_dtype == DSA_DTYPE_I64,
              "dsa_topk_index_mask: index dtype %d is not int32/int64", topk_dtype);
  if (rows == 0) return DSA_OK;
  Params p{};
  p.idx = topk_indices;
  p.mask = mask;
  p.B = B; p.Sq = Sq; p.Sk = Sk; p.row0 = row0; p.rows = rows; p.K = topk;
  p.i64 = topk_dtype == DSA_DTYPE_I64;
  p.value = value;
  p.fill = fill;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (fill_rows) {
    DSA_REQUIRE(Sk <= 32 * (int64_t)kMaxWords, "dsa_topk_index_mask: fill mode supports Sk <= %d (got %lld)",
                32 * kMaxWords, (long long)Sk);
    hipLaunchKernelGGL(index_mask_fill_kernel, dim3((unsigned)(B * rows)), dim3(kNT), 0, st, p);
    return check_launch("index_mask_fill_kernel");
  }
  const int64_t n = B * rows * topk;
  if (n == 0) return DSA_OK;
  hipLaunchKernelGGL(index_mask_scatter_kernel, dim3((unsigned)((n + kNT - 1) / kNT)), dim3(kNT), 0, st, p);
  return check_launch("index_mask_scatter_kernel");
}
