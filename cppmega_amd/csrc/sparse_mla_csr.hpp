// Inverse index (kv row -> entries) and the deterministic dKV reduction used
// by the SparseMLA backward.
#pragma once

#include "dsa_common.hpp"

namespace dsa {

// ---------------------------------------------------------------------------
// Inverse index: stable counting sort of entries by kv row
// ---------------------------------------------------------------------------
// Entry e = ((b*S + t)*G + g)*topk + slot; its row (within batch b) is
// r = j*G + g for a valid index j.  Tokens are grouped into chunks of CT
// within one batch; hist[b][chunk][r] counts a chunk's entries per row.

struct CsrParams {
  const int32_t *idx;
  int32_t *hist;    // [B][NC][R]
  int32_t *tot;     // [B*R]
  int32_t *rowptr;  // [B*R + 1]
  int32_t *refs;    // [entries]
  int64_t S, S_kv, G, topk;
  int64_t R;        // rows per batch = S_kv * G
  int CT, NC;       // tokens per chunk, chunks per batch
};

__global__ void fill_i32_kernel(int32_t *p, int64_t n, int32_t v) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

// grid (NC, B), 256 threads, dynamic LDS = R ints
__global__ void __launch_bounds__(256) csr_hist_kernel(const CsrParams p) {
  extern __shared__ int32_t cnt[];
  const int c = blockIdx.x;
  const int64_t b = blockIdx.y;
  for (int64_t r = threadIdx.x; r < p.R; r += 256) cnt[r] = 0;
  __syncthreads();
  const int64_t t0 = (int64_t)c * p.CT;
  const int64_t t1 = t0 + p.CT < p.S ? t0 + p.CT : p.S;
  const int64_t e0 = ((b * p.S + t0) * p.G) * p.topk;
  const int64_t e1 = ((b * p.S + t1) * p.G) * p.topk;
  for (int64_t e = e0 + threadIdx.x; e < e1; e += 256) {
    const int32_t j = p.idx[e];
    if (j >= 0 && j < p.S_kv) {
      const int64_t g = (e / p.topk) % p.G;
      atomicAdd(&cnt[j * p.G + g], 1);
    }
  }
  __syncthreads();
  int32_t *h = p.hist + (b * p.NC + c) * p.R;
  for (int64_t r = threadIdx.x; r < p.R; r += 256) h[r] = cnt[r];
}

// one thread per (b, r): total over chunks
__global__ void csr_rowsum_kernel(const CsrParams p, int64_t B) {
  const int64_t x = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (x >= B * p.R) return;
  const int64_t b = x / p.R, r = x % p.R;
  const int32_t *h = p.hist + b * p.NC * p.R + r;
  int32_t s = 0;
  for (int c = 0; c < p.NC; ++c) s += h[(int64_t)c * p.R];
  p.tot[x] = s;
}

// Exclusive scan of cnt[0..n) into rowptr[0..n] with one 1024-thread workgroup.
__global__ void __launch_bounds__(1024) csr_scan_kernel(const int32_t *cnt, int32_t *rowptr, int64_t n) {
  __shared__ int32_t wsum[16];
  const int tid = threadIdx.x;
  const int64_t per = (n + 1023) / 1024;
  const int64_t lo = tid * per, hi = lo + per < n ? lo + per : n;
  int32_t s = 0;
  for (int64_t i = lo; i < hi; ++i) s += cnt[i];
  int32_t v = s;
  const int lane = tid & 63;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int32_t o = __shfl_up(v, off, 64);
    if (lane >= off) v += o;
  }
  if (lane == 63) wsum[tid >> 6] = v;
  __syncthreads();
  if (tid < 16) {
    int32_t x = wsum[tid];
    for (int off = 1; off < 16; off <<= 1) {
      const int32_t o = __shfl_up(x, off, 16);
      if ((tid & 15) >= off) x += o;
    }
    wsum[tid] = x;
  }
  __syncthreads();
  const int wv = tid >> 6;
  int32_t run = (wv > 0 ? wsum[wv - 1] : 0) + v - s;
  for (int64_t i = lo; i < hi; ++i) {
    rowptr[i] = run;
    run += cnt[i];
  }
  if (tid == 1023) rowptr[n] = wsum[15];
}

// one thread per (b, r): hist[b][c][r] <- absolute start of chunk c's entries of row r
__global__ void csr_bases_kernel(const CsrParams p, int64_t B) {
  const int64_t x = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (x >= B * p.R) return;
  const int64_t b = x / p.R, r = x % p.R;
  int32_t *h = p.hist + b * p.NC * p.R + r;
  int32_t run = p.rowptr[x];
  for (int c = 0; c < p.NC; ++c) {
    const int32_t t = h[(int64_t)c * p.R];
    h[(int64_t)c * p.R] = run;
    run += t;
  }
}

// grid (NC, B), 256 threads, dynamic LDS = R ints.  Tokens of the chunk are
// placed one after another; within a token the slots take LDS cursors
// concurrently, which is order-independent as long as no row repeats inside
// the token.  A token whose valid indices are not strictly increasing (so a
// row could repeat) is placed by one thread in slot order instead.
__global__ void __launch_bounds__(256) csr_scatter_kernel(const CsrParams p) {
  extern __shared__ int32_t cur[];
  __shared__ int32_t wmax[4];
  __shared__ int32_t unordered;
  const int c = blockIdx.x;
  const int64_t b = blockIdx.y;
  const int tid = threadIdx.x, lane = lane_id(), w = wave_id();
  const int32_t *h = p.hist + (b * p.NC + c) * p.R;
  for (int64_t r = tid; r < p.R; r += 256) cur[r] = h[r];
  const int64_t t0 = (int64_t)c * p.CT;
  const int64_t t1 = t0 + p.CT < p.S ? t0 + p.CT : p.S;
  for (int64_t t = t0; t < t1; ++t) {
    for (int64_t g = 0; g < p.G; ++g) {
      const int64_t e0 = ((b * p.S + t) * p.G + g) * p.topk;
      if (tid == 0) unordered = 0;
      __syncthreads();
      // strictly-increasing check over valid slots, in chunks of 256 slots
      int32_t carry = -1;
      for (int64_t s0 = 0; s0 < p.topk; s0 += 256) {
        const int64_t s = s0 + tid;
        int32_t j = -1;
        if (s < p.topk) {
          j = p.idx[e0 + s];
          if (j < 0 || j >= p.S_kv) j = -1;
        }
        // inclusive max-scan of j over the chunk
        int32_t m = j;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          const int32_t o = __shfl_up(m, off, 64);
          if (lane >= off) m = max(m, o);
        }
        const int32_t m_prev_lane = __shfl_up(m, 1, 64);  // inclusive max up to lane - 1
        if (lane == 63) wmax[w] = m;
        __syncthreads();
        int32_t before = carry;  // max over all earlier slots of the token
        for (int i = 0; i < w; ++i) before = max(before, wmax[i]);
        const int32_t prev = lane > 0 ? max(before, m_prev_lane) : before;
        if (j >= 0 && prev >= j) unordered = 1;
        const int32_t chunk_max = max(max(wmax[0], wmax[1]), max(wmax[2], wmax[3]));
        carry = max(carry, chunk_max);
        __syncthreads();
      }
      if (!unordered) {
        for (int64_t s = tid; s < p.topk; s += 256) {
          const int32_t j = p.idx[e0 + s];
          if (j >= 0 && j < p.S_kv) {
            const int32_t pos = atomicAdd(&cur[j * p.G + g], 1);
            p.refs[pos] = (int32_t)(e0 + s);
          }
        }
      } else if (tid == 0) {
        for (int64_t s = 0; s < p.topk; ++s) {
          const int32_t j = p.idx[e0 + s];
          if (j >= 0 && j < p.S_kv) p.refs[cur[j * p.G + g]++] = (int32_t)(e0 + s);
        }
      }
      __syncthreads();
    }
  }
}

// One workgroup per kv row: the row's entries (CSR order) are split into four
// contiguous quarters, one per wave; each wave sums its quarter in order in
// fp32 and the four partial sums are combined as ((q0 + q1) + q2) + q3.  The
// association is fixed by the entry count alone, so results are bitwise
// reproducible.  Lane l handles element pairs l, l + 64, ...
template <int D_QK, bool F32P>
__global__ void __launch_bounds__(256)
dkv_reduce_kernel(const int32_t *rowptr, const int32_t *refs, const unsigned char *partials,
                  const int8_t *partial_exp, uint16_t *dkv, int64_t nrows, int ntiles) {
  constexpr int NP = D_QK / 2;          // element pairs per row
  constexpr int PPL = (NP + 63) / 64;   // pairs per lane
  constexpr int U = 8;                  // entries in flight per wave
  constexpr int64_t ROWB = (int64_t)D_QK * (F32P ? 4 : 2);
  __shared__ float part[4][2 * 64 * PPL];
  const int lane = lane_id(), w = wave_id();
  const int64_t r = blockIdx.x;
  if (r >= nrows) return;
  const int32_t base = rowptr[r], n = rowptr[r + 1] - base;
  const int q0 = (int)((int64_t)n * w / 4), q1 = (int)((int64_t)n * (w + 1) / 4);
  float acc[PPL][2];
#pragma unroll
  for (int k = 0; k < PPL; ++k) acc[k][0] = acc[k][1] = 0.0f;
  int32_t e_next[U];
#pragma unroll
  for (int u = 0; u < U; ++u) e_next[u] = (q0 + u < q1) ? refs[base + q0 + u] : 0;
  for (int i = q0; i < q1; i += U) {
    int32_t e[U];
#pragma unroll
    for (int u = 0; u < U; ++u) e[u] = e_next[u];
#pragma unroll
    for (int u = 0; u < U; ++u) e_next[u] = (i + U + u < q1) ? refs[base + i + U + u] : 0;
    for (int t = 0; t < ntiles; ++t) {
      float v[U][PPL][2];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t pr = (int64_t)e[u] * ntiles + t;
        const unsigned char *row = partials + pr * ROWB;
        float sc = 1.0f;
        if constexpr (!F32P) sc = exp2i(-(int)partial_exp[pr]);
#pragma unroll
        for (int k = 0; k < PPL; ++k) {
          const int pi = lane + 64 * k;
          v[u][k][0] = v[u][k][1] = 0.0f;
          if (pi < NP) {
            if constexpr (F32P) {
              const float2 x = reinterpret_cast<const float2 *>(row)[pi];
              v[u][k][0] = x.x;
              v[u][k][1] = x.y;
            } else {
              const uint32_t x = reinterpret_cast<const uint32_t *>(row)[pi];
              v[u][k][0] = f16_bits_to_f32(x & 0xffffu) * sc;  // exact: sc is a power of two
              v[u][k][1] = f16_bits_to_f32(x >> 16) * sc;
            }
          }
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (i + u < q1) {
#pragma unroll
          for (int k = 0; k < PPL; ++k) {
            acc[k][0] += v[u][k][0];
            acc[k][1] += v[u][k][1];
          }
        }
      }
    }
  }
#pragma unroll
  for (int k = 0; k < PPL; ++k) {
    part[w][2 * (lane + 64 * k)] = acc[k][0];
    part[w][2 * (lane + 64 * k) + 1] = acc[k][1];
  }
  __syncthreads();
  uint32_t *out = reinterpret_cast<uint32_t *>(dkv + r * D_QK);
  for (int pi = threadIdx.x; pi < NP; pi += 256) {
    const float x0 = ((part[0][2 * pi] + part[1][2 * pi]) + part[2][2 * pi]) + part[3][2 * pi];
    const float x1 = ((part[0][2 * pi + 1] + part[1][2 * pi + 1]) + part[2][2 * pi + 1]) + part[3][2 * pi + 1];
    out[pi] = pack_bf16x2(x0, x1);
  }
}

// Host side: build the inverse index (five stream-ordered kernels).
static int launch_csr(const CsrParams &cp, int64_t B, hipStream_t st) {
  const size_t hist_lds = (size_t)cp.R * 4;
  if (hist_lds > 64 * 1024) {
    hipError_t e1 = hipFuncSetAttribute((const void *)csr_hist_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                        (int)hist_lds);
    hipError_t e2 = hipFuncSetAttribute((const void *)csr_scatter_kernel,
                                        hipFuncAttributeMaxDynamicSharedMemorySize, (int)hist_lds);
    if (e1 != hipSuccess || e2 != hipSuccess)
      return set_error(DSA_ERR_HIP, "sparse_mla_bwd: csr LDS attribute failed");
  }
  const int64_t rows = B * cp.R;
  const dim3 cgrid((unsigned)cp.NC, (unsigned)B);
  const unsigned rgrid = (unsigned)((rows + 255) / 256);
  hipLaunchKernelGGL(csr_hist_kernel, cgrid, dim3(256), hist_lds, st, cp);
  hipLaunchKernelGGL(csr_rowsum_kernel, dim3(rgrid), dim3(256), 0, st, cp, B);
  hipLaunchKernelGGL(csr_scan_kernel, dim3(1), dim3(1024), 0, st, cp.tot, cp.rowptr, rows);
  hipLaunchKernelGGL(csr_bases_kernel, dim3(rgrid), dim3(256), 0, st, cp, B);
  hipLaunchKernelGGL(csr_scatter_kernel, cgrid, dim3(256), hist_lds, st, cp);
  return check_launch("sparse_mla_bwd(csr)");
}

}  // namespace dsa
