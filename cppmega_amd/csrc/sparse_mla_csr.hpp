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
// within one batch (NC chunks per batch); chunks form groups of CG = 16.
//   csr_hist     hist[b][c][r]  = entries of chunk c in row r
//   csr_gsum     gsum[b][q][r]  = sum of hist over the chunks of group q
//   csr_rows     tot[b*R + r]   = row total; gsum -> exclusive prefix over groups
//   csr_scan     rowptr         = exclusive prefix of tot
//   csr_bases    hist[b][c][r] <- rowptr + entries of row r in earlier chunks
//   csr_scatter  pos_of[e]      = CSR position of entry e, tokens in order (stable)
// Every thread touches at most CG chunks, so no kernel walks a long serial
// chain of global loads.

constexpr int kChunkGroup = 16;

struct CsrParams {
  const int32_t *idx;
  int32_t *hist;    // [B][NC][R]
  int32_t *gsum;    // [B][NQ][R]
  int32_t *tot;     // [B*R]
  int32_t *rowptr;  // [B*R + 1]
  int32_t *pos_of;  // [entries]: CSR position of each entry, -1 for a masked slot
  int64_t S, S_kv, G, topk;
  int64_t R;        // rows per batch = S_kv * G
  int CT, NC, NQ;   // tokens per chunk, chunks per batch, chunk groups per batch
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

// one thread per (b, q, r): sum of hist over the chunks of group q
__global__ void csr_gsum_kernel(const CsrParams p, int64_t B) {
  const int64_t x = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (x >= B * p.NQ * p.R) return;
  const int64_t r = x % p.R, bq = x / p.R, q = bq % p.NQ, b = bq / p.NQ;
  const int c0 = (int)q * kChunkGroup;
  const int32_t *h = p.hist + (b * p.NC + c0) * p.R + r;
  int32_t v[kChunkGroup];
#pragma unroll
  for (int k = 0; k < kChunkGroup; ++k) v[k] = (c0 + k < p.NC) ? h[(int64_t)k * p.R] : 0;
  int32_t s = 0;
#pragma unroll
  for (int k = 0; k < kChunkGroup; ++k) s += v[k];
  p.gsum[x] = s;
}

// one thread per (b, r): row total, and gsum -> exclusive prefix over groups
__global__ void csr_rows_kernel(const CsrParams p, int64_t B) {
  const int64_t x = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (x >= B * p.R) return;
  const int64_t b = x / p.R, r = x % p.R;
  int32_t *gs = p.gsum + b * p.NQ * p.R + r;
  int32_t run = 0;
  for (int q = 0; q < p.NQ; ++q) {
    const int32_t t = gs[(int64_t)q * p.R];
    gs[(int64_t)q * p.R] = run;
    run += t;
  }
  p.tot[x] = run;
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

// one thread per (b, q, r): hist[b][c][r] <- absolute start of chunk c's entries of row r
__global__ void csr_bases_kernel(const CsrParams p, int64_t B) {
  const int64_t x = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (x >= B * p.NQ * p.R) return;
  const int64_t r = x % p.R, bq = x / p.R, q = bq % p.NQ, b = bq / p.NQ;
  const int c0 = (int)q * kChunkGroup;
  int32_t *h = p.hist + (b * p.NC + c0) * p.R + r;
  int32_t v[kChunkGroup];
#pragma unroll
  for (int k = 0; k < kChunkGroup; ++k) v[k] = (c0 + k < p.NC) ? h[(int64_t)k * p.R] : 0;
  int32_t run = p.rowptr[b * p.R + r] + p.gsum[x];
#pragma unroll
  for (int k = 0; k < kChunkGroup; ++k) {
    if (c0 + k < p.NC) h[(int64_t)k * p.R] = run;
    run += v[k];
  }
}

// grid (NC, B), 256 threads, dynamic LDS = R ints + 2 * topk ints.  Tokens of
// the chunk are placed one after another (their indices are staged in LDS one
// token ahead); within a token the slots take LDS cursors concurrently, which
// is order-independent as long as no row repeats inside the token.  A token
// whose valid indices are not strictly increasing (so a row could repeat) is
// placed by one thread in slot order instead.
__global__ void __launch_bounds__(256) csr_scatter_kernel(const CsrParams p) {
  extern __shared__ int32_t lds_i32[];
  int32_t *cur = lds_i32;                 // [R]
  int32_t *tidx = lds_i32 + p.R;          // [2][topk]
  __shared__ int32_t wmax[4];
  __shared__ int32_t unordered;
  const int c = blockIdx.x;
  const int64_t b = blockIdx.y;
  const int tid = threadIdx.x, lane = lane_id(), w = wave_id();
  const int32_t *h = p.hist + (b * p.NC + c) * p.R;
  for (int64_t r = tid; r < p.R; r += 256) cur[r] = h[r];
  const int64_t t0 = (int64_t)c * p.CT;
  const int64_t t1 = t0 + p.CT < p.S ? t0 + p.CT : p.S;
  const int64_t nseg = (t1 - t0) * p.G;  // (token, group) segments of topk entries
  const int64_t e_first = ((b * p.S + t0) * p.G) * p.topk;
  // stage segment 0
  for (int64_t s = tid; s < p.topk; s += 256) tidx[s] = p.idx[e_first + s];
  for (int64_t sg = 0; sg < nseg; ++sg) {
    const int64_t e0 = e_first + sg * p.topk;
    const int64_t g = sg % p.G;
    int32_t *cur_idx = tidx + (sg & 1) * p.topk;
    int32_t *nxt_idx = tidx + ((sg + 1) & 1) * p.topk;
    __syncthreads();  // segment sg staged; every thread is done with segment sg - 1
    // (the first barrier of the check loop below orders this reset before
    // any thread sets the flag)
    if (tid == 0) unordered = 0;
    // prefetch the next segment while this one is placed
    if (sg + 1 < nseg)
      for (int64_t s = tid; s < p.topk; s += 256) nxt_idx[s] = p.idx[e0 + p.topk + s];
    // strictly-increasing check over valid slots, in chunks of 256 slots
    int32_t carry = -1;
    for (int64_t s0 = 0; s0 < p.topk; s0 += 256) {
      const int64_t s = s0 + tid;
      int32_t j = -1;
      if (s < p.topk) {
        j = cur_idx[s];
        if (j < 0 || j >= p.S_kv) j = -1;
      }
      int32_t m = j;  // inclusive max-scan within the wave
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int32_t o = __shfl_up(m, off, 64);
        if (lane >= off) m = max(m, o);
      }
      const int32_t m_prev_lane = __shfl_up(m, 1, 64);
      if (lane == 63) wmax[w] = m;
      __syncthreads();
      int32_t before = carry;
      for (int i = 0; i < w; ++i) before = max(before, wmax[i]);
      const int32_t prev = lane > 0 ? max(before, m_prev_lane) : before;
      if (j >= 0 && prev >= j) unordered = 1;
      carry = max(carry, max(max(wmax[0], wmax[1]), max(wmax[2], wmax[3])));
      __syncthreads();
    }
    if (!unordered) {
      for (int64_t s = tid; s < p.topk; s += 256) {
        const int32_t j = cur_idx[s];
        int32_t pos = -1;
        if (j >= 0 && j < p.S_kv) pos = atomicAdd(&cur[j * p.G + g], 1);
        p.pos_of[e0 + s] = pos;
      }
    } else if (tid == 0) {
      for (int64_t s = 0; s < p.topk; ++s) {
        const int32_t j = cur_idx[s];
        p.pos_of[e0 + s] = (j >= 0 && j < p.S_kv) ? cur[j * p.G + g]++ : -1;
      }
    }
  }
}

// One workgroup per kv row.  The main kernel wrote each entry's partial rows
// at its CSR position, so the row's items are the contiguous partial rows
// [rowptr[r] * ntiles, rowptr[r + 1] * ntiles) in CSR order; they are split
// into four contiguous quarters, one per wave.  A partial row is read as
// 16-byte chunks by a group of LPE lanes (rows over 1 KiB: all 64 lanes, CPL
// chunks each), so one load instruction covers EPI = 64 / LPE items and every
// lane keeps about 8 loads in flight.  Lane group g of a wave sums items g,
// g + EPI, ... of its quarter in order (fp32); the groups are combined by a
// fixed xor tree and the four waves as ((w0 + w1) + w2) + w3.  The association
// depends on the item count alone, so the result is bitwise reproducible.
template <int D_QK, bool F32P>
__global__ void __launch_bounds__(256)
dkv_reduce_kernel(const int32_t *rowptr, const unsigned char *partials, const int8_t *partial_exp,
                  uint16_t *dkv, int64_t nrows, int ntiles) {
  constexpr int ROWB = D_QK * (F32P ? 4 : 2);  // bytes per partial row
  constexpr int NCR = ROWB / 16;                // 16-byte chunks per partial row
  constexpr int LPE = NCR <= 8 ? 8 : (NCR <= 16 ? 16 : (NCR <= 32 ? 32 : 64));  // lanes per item
  constexpr int CPL = (NCR + 63) / 64;          // chunks per lane (rows over 1 KiB)
  constexpr int EPI = 64 / LPE;                 // items per load instruction
  constexpr int EPC = F32P ? 4 : 8;             // elements per chunk
  constexpr int U = CPL > 1 ? (8 + CPL - 1) / CPL : 8;  // items in flight per lane
  static_assert(NCR * 16 == ROWB, "partial rows must be whole 16-byte chunks");
  __shared__ float part[4][D_QK];
  const int lane = lane_id(), w = wave_id();
  const int grp = lane / LPE, c = lane % LPE;
  const int64_t r = blockIdx.x;
  if (r >= nrows) return;
  const int64_t base = rowptr[r], n = (int64_t)(rowptr[r + 1] - rowptr[r]) * ntiles;
  const int64_t k0 = base * ntiles + n * w / 4, k1 = base * ntiles + n * (w + 1) / 4;
  float acc[CPL][EPC];
#pragma unroll
  for (int q = 0; q < CPL; ++q)
#pragma unroll
    for (int x = 0; x < EPC; ++x) acc[q][x] = 0.0f;
  for (int64_t kb = k0; kb < k1; kb += EPI * U) {
    i32x4 v[U][CPL];
    float sc[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t k = kb + EPI * u + grp;
      sc[u] = 0.0f;
      if constexpr (!F32P) {
        if (k < k1) sc[u] = exp2i(-(int)partial_exp[k]);
      }
#pragma unroll
      for (int q = 0; q < CPL; ++q) {
        const int cc = c + 64 * q;
        v[u][q] = i32x4{0, 0, 0, 0};
        if (k < k1 && cc < NCR) v[u][q] = ld_global_16(partials + k * ROWB + cc * 16);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int q = 0; q < CPL; ++q) {
#pragma unroll
        for (int x = 0; x < EPC; ++x) {
          if constexpr (F32P) {
            acc[q][x] += __int_as_float(v[u][q][x]);
          } else {
            const uint32_t h = ((uint32_t)v[u][q][x >> 1] >> (16 * (x & 1))) & 0xffffu;
            acc[q][x] += f16_bits_to_f32(h) * sc[u];  // exact: sc is a power of two
          }
        }
      }
    }
  }
#pragma unroll
  for (int off = LPE; off < 64; off *= 2) {
#pragma unroll
    for (int q = 0; q < CPL; ++q)
#pragma unroll
      for (int x = 0; x < EPC; ++x) acc[q][x] += __shfl_xor(acc[q][x], off, 64);
  }
  if (grp == 0) {
#pragma unroll
    for (int q = 0; q < CPL; ++q) {
      const int cc = c + 64 * q;
      if (cc < NCR) {
#pragma unroll
        for (int x = 0; x < EPC; ++x) part[w][cc * EPC + x] = acc[q][x];
      }
    }
  }
  __syncthreads();
  uint32_t *out = reinterpret_cast<uint32_t *>(dkv + r * D_QK);
  for (int pi = threadIdx.x; pi < D_QK / 2; pi += 256) {
    const float x0 = ((part[0][2 * pi] + part[1][2 * pi]) + part[2][2 * pi]) + part[3][2 * pi];
    const float x1 = ((part[0][2 * pi + 1] + part[1][2 * pi + 1]) + part[2][2 * pi + 1]) + part[3][2 * pi + 1];
    out[pi] = pack_bf16x2(x0, x1);
  }
}

// Chunking of the inverse index: 16 tokens per chunk unless the chunk
// histogram (NC * R counters per batch) would exceed 2^24 entries.
static void csr_plan(int64_t S, int64_t R, int *CT, int *NC, int *NQ) {
  int ct = 16;
  while ((int64_t)((S + ct - 1) / ct) * R > (1ll << 24) && ct < (1 << 20)) ct *= 2;
  *CT = ct;
  *NC = (int)((S + ct - 1) / ct);
  *NQ = (*NC + kChunkGroup - 1) / kChunkGroup;
}

// Host side: build the inverse index (six stream-ordered kernels, no atomics
// on global memory, no memset).
static int launch_csr(const CsrParams &cp, int64_t B, hipStream_t st) {
  const size_t hist_lds = (size_t)cp.R * 4;
  const size_t scat_lds = hist_lds + 2 * (size_t)cp.topk * 4;
  if (scat_lds > 160 * 1024)
    return set_error(DSA_ERR_UNSUPPORTED, "sparse_mla_bwd: inverse index needs %zu bytes of LDS", scat_lds);
  if (hist_lds > 64 * 1024 &&
      hipFuncSetAttribute((const void *)csr_hist_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)hist_lds) != hipSuccess)
    return set_error(DSA_ERR_HIP, "sparse_mla_bwd: csr LDS attribute failed");
  if (scat_lds > 64 * 1024 &&
      hipFuncSetAttribute((const void *)csr_scatter_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)scat_lds) != hipSuccess)
    return set_error(DSA_ERR_HIP, "sparse_mla_bwd: csr LDS attribute failed");
  const int64_t rows = B * cp.R;
  const dim3 cgrid((unsigned)cp.NC, (unsigned)B);
  const unsigned rgrid = (unsigned)((rows + 255) / 256);
  const unsigned qgrid = (unsigned)((B * cp.NQ * cp.R + 255) / 256);
  hipLaunchKernelGGL(csr_hist_kernel, cgrid, dim3(256), hist_lds, st, cp);
  hipLaunchKernelGGL(csr_gsum_kernel, dim3(qgrid), dim3(256), 0, st, cp, B);
  hipLaunchKernelGGL(csr_rows_kernel, dim3(rgrid), dim3(256), 0, st, cp, B);
  hipLaunchKernelGGL(csr_scan_kernel, dim3(1), dim3(1024), 0, st, cp.tot, cp.rowptr, rows);
  hipLaunchKernelGGL(csr_bases_kernel, dim3(qgrid), dim3(256), 0, st, cp, B);
  hipLaunchKernelGGL(csr_scatter_kernel, cgrid, dim3(256), scat_lds, st, cp);
  return check_launch("sparse_mla_bwd(csr)");
}

}  // namespace dsa
