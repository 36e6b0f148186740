// Deterministic per-row top-k on gfx950: radix select in LDS.
//
// Reference: the top-k of Megatron's fused_qk_topk_naive
// (`index_scores.topk(min(topk, seqlen), dim=-1)[1]`, restated in
// scripts/modal_dsa_indexer_bench.py:188-194) and the radix idea of
// tilelang_sparse_mla/topk_selector.py:30-186 (histogram of key bytes, then
// refinement).  Unlike both, the result here is fully determined by the
// scores: candidates are the columns [start, end) of a row, the
// min(topk, end - start) largest are taken, equal scores prefer the lower
// column, NaN ranks as +inf, -0.0 equals +0.0, and the chosen columns are
// written in ascending order, padded with -1.
//
// One workgroup per row.  Each thread holds a contiguous chunk of the row as
// order-preserving 32-bit keys in registers.  Up to four 8-bit radix passes
// (LDS histogram + block suffix scan) find the key prefix of the k-th largest
// element and how many elements equal to it are still needed; a pass stops
// early once the selected bucket is taken whole.  Selection is then a rank
// among equal keys by column (block prefix sum) and the chosen columns are
// compacted in column order with a second prefix sum, which yields the
// ascending output directly.
#include "dsa_common.hpp"

namespace dsa {

struct TopkParams {
  const float *scores;
  int64_t rows, row_len, row_stride, seq_q, causal_offset;
  const int32_t *starts;
  const int32_t *ends;
  int causal;
  int topk;
  int32_t *out;
};

__device__ __forceinline__ uint32_t score_key(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) u = 0x7f800000u;  // NaN ranks as +inf
  if (u == 0x80000000u) u = 0u;                           // -0.0 == +0.0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Block-wide exclusive prefix sum of one int per thread; returns the total.
template <int THREADS>
__device__ __forceinline__ int block_excl_scan(int v, int *excl, int *wtot) {
  constexpr int NW = THREADS / 64;
  const int lane = lane_id(), w = wave_id();
  int incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int o = __shfl_up(incl, off, 64);
    if (lane >= off) incl += o;
  }
  __syncthreads();
  if (lane == 63) wtot[w] = incl;
  __syncthreads();
  int before = 0, total = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    const int t = wtot[i];
    before += (i < w) ? t : 0;
    total += t;
  }
  *excl = before + incl - v;
  return total;
}

template <int THREADS, int ITEMS>
__global__ void __launch_bounds__(THREADS) topk_select_kernel(const TopkParams p) {
  __shared__ int hist[256];
  __shared__ int wtot[THREADS / 64];
  __shared__ int sel_digit, sel_above;
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  int64_t st, en;
  if (p.starts) {
    st = p.starts[row];
    en = p.ends[row];
  } else if (p.causal) {
    st = 0;
    en = (row % p.seq_q) + 1 + p.causal_offset;
  } else {
    st = 0;
    en = p.row_len;
  }
  if (st < 0) st = 0;
  if (en > p.row_len) en = p.row_len;
  const int n = en > st ? (int)(en - st) : 0;
  int32_t *orow = p.out + row * p.topk;

  if (n <= p.topk) {  // everything in the window is selected
    for (int i = tid; i < p.topk; i += THREADS) orow[i] = i < n ? (int32_t)(st + i) : -1;
    return;
  }

  // ---- load keys (blocked: thread owns columns [tid*ITEMS, tid*ITEMS + ITEMS)) ----
  const float *src = p.scores + row * p.row_stride + st;
  uint32_t key[ITEMS];
  const int c0 = tid * ITEMS;
  const bool vec = ((reinterpret_cast<uintptr_t>(src) & 15u) == 0) && (ITEMS % 4 == 0);
  if (vec && c0 + ITEMS <= n) {
#pragma unroll
    for (int i = 0; i < ITEMS; i += 4) {
      const f32x4 v = *reinterpret_cast<const f32x4 *>(src + c0 + i);
      key[i] = score_key(v[0]);
      key[i + 1] = score_key(v[1]);
      key[i + 2] = score_key(v[2]);
      key[i + 3] = score_key(v[3]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) key[i] = (c0 + i < n) ? score_key(src[c0 + i]) : 0u;
  }
  int nvalid = n - c0;
  nvalid = nvalid < 0 ? 0 : (nvalid > ITEMS ? ITEMS : nvalid);

  // ---- radix select: find prefix of the k-th largest key ----
  uint32_t prefix = 0;
  int plen = 0;  // number of determined high bits
  int krem = p.topk;
#pragma unroll 1
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    if (tid < 256) hist[tid] = 0;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const bool match = plen == 0 || (key[i] >> (32 - plen)) == prefix;
      if (i < nvalid && match) atomicAdd(&hist[(key[i] >> shift) & 255u], 1);
    }
    __syncthreads();
    // suffix counts: thread tid (< 256) takes digit 255 - tid
    int hv = 0;
    if (tid < 256) hv = hist[255 - tid];
    int excl;
    block_excl_scan<THREADS>(hv, &excl, wtot);
    if (tid < 256) {
      const int incl = excl + hv;  // keys with digit >= 255 - tid
      if (incl >= krem && excl < krem) {
        sel_digit = 255 - tid;
        sel_above = excl;
      }
    }
    __syncthreads();
    const int d = sel_digit;
    krem -= sel_above;
    prefix = (prefix << 8) | (uint32_t)d;
    plen += 8;
    const int cnt = hist[d];
    __syncthreads();
    if (cnt == krem) break;  // the whole bucket is selected
  }

  // ---- selection: keys above the prefix, plus the first krem equal ones by column ----
  const int sh = 32 - plen;
  const uint32_t P = prefix;
  int neq = 0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i)
    if (i < nvalid && (key[i] >> sh) == P) ++neq;
  int eq_before;
  block_excl_scan<THREADS>(neq, &eq_before, wtot);
  bool take[ITEMS];
  int nsel = 0;
  int er = eq_before;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    bool t = false;
    if (i < nvalid) {
      const uint32_t hi = key[i] >> sh;
      if (hi > P) t = true;
      else if (hi == P) {
        t = er < krem;
        ++er;
      }
    }
    take[i] = t;
    nsel += t ? 1 : 0;
  }
  int pos;
  block_excl_scan<THREADS>(nsel, &pos, wtot);
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    if (take[i]) {
      orow[pos] = (int32_t)(st + c0 + i);
      ++pos;
    }
  }
}

template <int THREADS, int ITEMS>
static int launch_topk(const TopkParams &p, hipStream_t st) {
  hipLaunchKernelGGL((topk_select_kernel<THREADS, ITEMS>), dim3((unsigned)p.rows), dim3(THREADS), 0, st, p);
  return check_launch("topk_select");
}

}  // namespace dsa

using namespace dsa;

extern "C" int dsa_topk(const float *scores, int64_t rows, int64_t row_len, int64_t row_stride, int64_t seq_q,
                        int causal, int64_t causal_offset, const int32_t *starts, const int32_t *ends,
                        int64_t topk, int32_t *out_idx, void *stream) {
  DSA_REQUIRE(rows >= 0 && row_len >= 0 && topk > 0, "dsa_topk: bad dims rows=%lld row_len=%lld topk=%lld",
              (long long)rows, (long long)row_len, (long long)topk);
  DSA_REQUIRE(row_stride >= row_len, "dsa_topk: row_stride %lld < row_len %lld", (long long)row_stride,
              (long long)row_len);
  DSA_REQUIRE((starts == nullptr) == (ends == nullptr), "dsa_topk: starts and ends must both be given or both NULL");
  DSA_REQUIRE(!causal || starts || seq_q > 0, "dsa_topk: causal windows need seq_q > 0");
  DSA_REQUIRE(topk < (1ll << 30) && rows < (1ll << 31), "dsa_topk: sizes too large");
  if (rows == 0) return DSA_OK;
  DSA_REQUIRE(out_idx && (scores || row_len == 0), "dsa_topk: null pointer");
  TopkParams p;
  p.scores = scores;
  p.rows = rows;
  p.row_len = row_len;
  p.row_stride = row_stride;
  p.seq_q = seq_q > 0 ? seq_q : 1;
  p.causal_offset = causal_offset;
  p.starts = starts;
  p.ends = ends;
  p.causal = causal;
  p.topk = (int)topk;
  p.out = out_idx;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (row_len <= 1024) return launch_topk<256, 4>(p, st);
  if (row_len <= 4096) return launch_topk<256, 16>(p, st);
  if (row_len <= 8192) return launch_topk<512, 16>(p, st);
  if (row_len <= 16384) return launch_topk<1024, 16>(p, st);
  if (row_len <= 32768) return launch_topk<1024, 32>(p, st);
  return set_error(DSA_ERR_UNSUPPORTED, "dsa_topk: rows longer than 32768 columns are not supported (got %lld)",
                   (long long)row_len);
}
