// Deterministic per-row top-k on gfx950: adaptive bucket select in LDS.
//
// Reference: the top-k of Megatron's fused_qk_topk_naive
// (`index_scores.topk(min(topk, seqlen), dim=-1)[1]`, restated in
// scripts/modal_dsa_indexer_bench.py:188-194) and the radix idea of
// tilelang_sparse_mla/topk_selector.py:30-186 (histogram of key bits, then
// refinement).  Unlike both, the result here is fully determined by the
// scores: candidates are the columns [start, end) of a row, the
// min(topk, end - start) largest are taken, equal scores prefer the lower
// column, NaN ranks as +inf, -0.0 equals +0.0, and the chosen columns are
// written in ascending order, padded with -1.
//
// Rows of up to 8192 columns run one wave per row (topk_wave_kernel), longer
// rows one workgroup of NW waves per row (topk_block_kernel).  The row stays
// in registers; a lower bound of the k-th largest score from per-lane subset
// maxima keeps the lower scores out of the value-linear histogram, which
// usually leaves a handful of members in the bucket holding the k-th largest;
// those are ranked exactly, and the output is compacted in column order by
// ballots.
#include "dsa_common.hpp"
#include "wave_ops.hpp"

namespace dsa {

struct TopkParams {
  const float *scores;
  int64_t rows, row_len, row_stride, seq_q, causal_offset;
  const int32_t *starts;
  const int32_t *ends;
  int causal;
  int topk;
  int32_t *out;
  // 0: output rows are contiguous; else the output of row r is at
  // out + (r / seq_q) * out_bstride + (r % seq_q) * topk (batches of seq_q rows
  // whose outputs sit out_bstride elements apart)
  int64_t out_bstride;
  // segment mode (nseg > 1, rows over one pass's reach): launch row v is
  // segment v % nseg (columns [seg * seg_len, +seg_len)) of row v / nseg, whose
  // window is cut to the segment; rows counts launch rows, and the output of
  // launch row v is out + v * topk
  int64_t seg_len;
  int nseg;
  int64_t row0;  // launch row v is row row0 + v (a launch over part of the rows)
};

// Launch row v: its scores row `row` and window [st, en) (clamped to the row
// and, in segment mode, to the segment).
__device__ __forceinline__ void topk_window(const TopkParams &p, int64_t v, int64_t &row, int64_t &st, int64_t &en) {
  row = p.nseg > 1 ? v / p.nseg : v;
  if (p.starts) {
    st = p.starts[row];
    en = p.ends[row];
  } else if (p.causal) {
    st = 0;
    en = (int64_t)((uint64_t)row % (uint64_t)p.seq_q) + 1 + p.causal_offset;
  } else {
    st = 0;
    en = p.row_len;
  }
  if (st < 0) st = 0;
  if (en > p.row_len) en = p.row_len;
  if (p.nseg > 1) {
    const int64_t c0 = (v - row * p.nseg) * p.seg_len;
    st = st > c0 ? st : c0;
    en = en < c0 + p.seg_len ? en : c0 + p.seg_len;
  }
}

__device__ __forceinline__ int32_t *topk_out_row(const TopkParams &p, int64_t row) {
  if (p.out_bstride == 0) return p.out + row * p.topk;
  const int64_t b = row / p.seq_q;
  return p.out + b * p.out_bstride + (row - b * p.seq_q) * p.topk;
}

__device__ __forceinline__ uint32_t score_key(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) u = 0x7f800000u;  // NaN ranks as +inf
  if (u == 0x80000000u) u = 0u;                           // -0.0 == +0.0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// ---------------------------------------------------------------------------
// Wave-per-row kernel for rows of at most 64 * IPL columns (no block barriers).
// ---------------------------------------------------------------------------
// Lane l holds columns 64i + l (i < IPL) as normalised scores: every load
// instruction reads 256 B contiguously.  The undecided elements are always the
// scores in an interval [A, B], so no masks are kept.
//  * Round 0 finds the maximum and a lower bound L of the k-th largest score
//    (the least of 4 interleaved per-lane subset maxima, see subset_bound),
//    then buckets the finite scores >= L linearly in value over [L, max]
//    (1024 LDS bins).  Real
//    score rows spread evenly this way, so the bucket holding the k-th largest
//    usually has a handful of members, and only the scores >= L (the upper
//    tail) take part in the LDS atomics.
//  * Further rounds, if more than 64 members remain, histogram the 10 key bits
//    below the highest bit in which the members' min and max keys differ (the
//    span shrinks by 2^10 per round, so they end).
//  * At most 64 members are ranked exactly (each lane holds one, the others are
//    read with v_readlane), giving the k-th largest key K* and how many
//    K*-equal elements are taken.
// All keys > K* and the lowest-column K*-equal ones are taken; the output is
// compacted in column order through two LDS bitmaps read back lane-blocked.
// Wave-wide reductions and scans use DPP row operations and readlane.

constexpr int kWaveBins = 1024;
constexpr int kNoLimit = 0x7fffffff;
constexpr int kGroup = 16;  // items per group: passes skip whole groups past the window

// Score normalised for ranking: NaN -> +inf.  -0 stays: every float
// comparison (and the linear buckets) treats it as +0, and score_key maps it
// to the key of +0, so normalised scores order exactly as the keys do.
__device__ __forceinline__ float rank_value(float f) { return f != f ? INFINITY : f; }

// Linear bucket of x >= L (see the round-0 comment in topk_wave_kernel):
// fma(x, scale, cbin) lies in [1.5 * 2^23, 1.5 * 2^23 + 1024), so its bit
// pattern less kBinBits is the bin.
constexpr uint32_t kBinBits = 0x4B400000u;
__device__ __forceinline__ uint32_t lin_bits(float x, float scale, float cbin) {
  return __float_as_uint(fmaf(x, scale, cbin));
}

// Lower bound of the r-th largest score.  Item i of each lane feeds the
// running maximum of subset i % KSUB (sm).  Subsets are disjoint, so if c of
// them hold a score above -inf (pads past the window and -inf scores hold
// none), at least c scores are >= the least of their maxima, which bounds the
// r-th largest from below whenever c >= r.  Returns the wave's least non-empty
// subset maximum and its count of non-empty subsets; also the wave maximum.
template <int KSUB>
__device__ __forceinline__ float subset_bound(const float (&sm)[KSUB], int &count, float &hi) {
  float L = INFINITY, h = -INFINITY;
  int c = 0;
#pragma unroll
  for (int j = 0; j < KSUB; ++j) {
    const bool has = sm[j] > -INFINITY;
    L = has ? fminf(L, sm[j]) : L;
    h = fmaxf(h, sm[j]);
    c += __popcll(wv::ballot(has));
  }
  count = c;
  hi = __uint_as_float(wv::wave_reduce(__float_as_uint(h), wv::MaxF()));
  return __uint_as_float(wv::wave_reduce(__float_as_uint(L), wv::MinF()));
}

// Make the compiler treat the row values as freshly defined, so predicates of
// one pass are recomputed in the next instead of being kept alive as 64-bit
// lane masks across the whole kernel (which exhausts the scalar registers).
template <int IPL>
__device__ __forceinline__ void fence_values(float (&x)[IPL], int &ng) {
#pragma unroll
  for (int i = 0; i < IPL; ++i) asm volatile("" : "+v"(x[i]));
  asm volatile("" : "+s"(ng));
}

__device__ __forceinline__ int lane_rank(uint64_t mask) {  // set lanes below this one
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

// Suffix scan of a wave's 1024-bin histogram: the bin holding the r-th largest
// element and the count above it.
template <int NBINS = kWaveBins>
__device__ __forceinline__ void find_bucket(const int *hist, int r, int &bsel, int &above) {
  constexpr int BPL = NBINS / 64;
  const int lane = lane_id();
  int cnt[BPL];
  uint32_t local = 0u;
#pragma unroll
  for (int q = 0; q < BPL; ++q) {
    cnt[q] = hist[NBINS - 1 - (lane * BPL + q)];
    local += (uint32_t)cnt[q];
  }
  const int excl = (int)(wv::wave_incl_scan(local) - local);
  const bool cross = excl < r && excl + (int)local >= r;
  int bsel_l = 0, above_l = 0;
  if (cross) {
    int acc = excl;
#pragma unroll
    for (int q = 0; q < BPL; ++q) {
      if (acc < r && acc + cnt[q] >= r) {
        bsel_l = NBINS - 1 - (lane * BPL + q);
        above_l = acc;
      }
      acc += cnt[q];
    }
  }
  const int cl = __ffsll((unsigned long long)wv::ballot(cross)) - 1;  // exactly one lane crosses
  bsel = (int)wv::readlane((uint32_t)bsel_l, cl < 0 ? 0 : cl);
  above = (int)wv::readlane((uint32_t)above_l, cl < 0 ? 0 : cl);
}

// Exact rank among <= 64 values held one per lane (lanes >= mm hold padding):
// the r-th largest value K and how many K-equal values are taken (kNoLimit: all).
__device__ __forceinline__ void rank_list(float v, int mm, int r, float &K, int &c_eq) {
  const int lane = lane_id();
  int g = 0, e = 0;
  for (int j = 0; j < mm; ++j) {
    const float vj = __uint_as_float(wv::readlane(__float_as_uint(v), j));
    g += vj > v ? 1 : 0;
    e += vj == v ? 1 : 0;
  }
  const bool found = lane < mm && g < r && r <= g + e;
  const int fl = __ffsll((unsigned long long)wv::ballot(found)) - 1;
  const int src = fl < 0 ? 0 : fl;
  K = __uint_as_float(wv::readlane(__float_as_uint(v), src));
  const int gk = (int)wv::readlane((uint32_t)g, src);
  const int ek = (int)wv::readlane((uint32_t)e, src);
  c_eq = (r - gk >= ek) ? kNoLimit : r - gk;
}

template <int IPL>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(IPL <= 64 ? 4 : 2)))
topk_wave_kernel(const TopkParams p) {
  static_assert(IPL % kGroup == 0, "items come in whole groups");
  constexpr int NG = IPL / kGroup;
  constexpr int BPL = kWaveBins / 64;
  __shared__ int s_hist[4][kWaveBins + 64];
  __shared__ float s_list[4][64];
  // the wave index is uniform: make the row and everything derived from it scalar
  const int w = __builtin_amdgcn_readfirstlane(wave_id()), lane = lane_id();
  const int64_t lrow = (int64_t)blockIdx.x * 4 + w;
  if (lrow >= p.rows) return;
  const int64_t vrow = p.row0 + lrow;
  int *hist = s_hist[w];
  float *list = s_list[w];
  int64_t row, st, en;
  topk_window(p, vrow, row, st, en);
  const int n = __builtin_amdgcn_readfirstlane(en > st ? (int)(en - st) : 0);
  int32_t *orow = topk_out_row(p, vrow);
  if (n <= p.topk) {
    for (int i = lane; i < p.topk; i += 64) orow[i] = i < n ? (int32_t)(st + i) : -1;
    return;
  }

  // ---- load: lane l holds columns 64i + l; NaN pads columns past the window ----
  // Buffer loads bounded to the window (out-of-range reads return 0 without
  // touching memory); all loads of the row are in flight together.
  const float *src = p.scores + row * p.row_stride + st;
  const __amdgpu_buffer_rsrc_t rsrc = make_buffer_rsrc(src, (uint32_t)n * 4u);
  int ng = (n + 64 * kGroup - 1) / (64 * kGroup);  // groups holding window columns
  const float kPad = __uint_as_float(0x7fc00000u);
  // groups wholly past the window (half of a causal matrix) issue no loads
  float x[IPL];
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    if (g < ng) {
#pragma unroll
      for (int i = g * kGroup; i < (g + 1) * kGroup; ++i) x[i] = buffer_load_f32(rsrc, 4 * lane, 256 * i);
    } else {
#pragma unroll
      for (int i = g * kGroup; i < (g + 1) * kGroup; ++i) x[i] = kPad;
    }
  }
#pragma unroll
  for (int q = 0; q < BPL; ++q) hist[lane * BPL + q] = 0;
  // only the last loaded group reaches past the window
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    if (g < ng) {
      const bool last = g == ng - 1;
#pragma unroll
      for (int i = g * kGroup; i < (g + 1) * kGroup; ++i) {
        x[i] = rank_value(x[i]);
        if (last) x[i] = (64 * i + lane < n) ? x[i] : kPad;
      }
    }
  }

  int r = p.topk;  // elements still to take
  float K = 0.0f;  // result: take x > K and the first c_eq (column order) of x == K
  int c_eq = kNoLimit;
  bool decided = false;
  float vA, vB;    // member interval for the key rounds
  int m = n;

  // ---- round 0: maximum and a lower bound L of the r-th largest score ----
  // L from 4 interleaved subset maxima per lane (subset_bound): scores below L
  // are never taken and stay out of every later pass (IEEE min / max skip the
  // NaN pads, which also fail every x >= L test).  With fewer than r non-empty
  // subsets, L is the row minimum.
  constexpr int kSub = 4;
  fence_values(x, ng);
  float smax[kSub];
#pragma unroll
  for (int j = 0; j < kSub; ++j) smax[j] = -INFINITY;
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    if (g < ng) {
#pragma unroll
      for (int i = g * kGroup; i < (g + 1) * kGroup; ++i) smax[i % kSub] = fmaxf(smax[i % kSub], x[i]);
    }
  }
  int nsub;
  float hi;
  float L = subset_bound(smax, nsub, hi);
  if (r > nsub) {
    fence_values(x, ng);
    float lo = INFINITY;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      if (g < ng) {
#pragma unroll
        for (int i = g * kGroup; i < (g + 1) * kGroup; ++i) lo = fminf(lo, x[i]);
      }
    }
    L = __uint_as_float(wv::wave_reduce(__float_as_uint(lo), wv::MinF()));
  }
  vA = L;
  vB = hi;
  if (L == hi) {  // the r largest all equal the maximum
    K = hi;
    c_eq = r;
    decided = true;
  } else if (__builtin_isfinite(L) && __builtin_isfinite(hi)) {
    // Value-linear buckets over [L, hi]: the bin of x >= L is the integer that
    // fma(x, scale, cbin) rounds to in the binade [2^23, 2^24) (unit spacing),
    // less 1.5 * 2^23, i.e. round((x - L) * scale + 1 + d) with |d| <= 0.5625
    // (0.5 from rounding cbin, 1/16 from rounding -L * scale while
    // |x| * scale < 2^20), so bins run over [0, 1023] and rise with x.
    const float scale = 1021.0f / (hi - L);
    const float cbin = -L * scale + 12582913.0f;   // 1.5 * 2^23 + 1
    if (isfinite(scale) && fmaxf(fabsf(L), fabsf(hi)) * scale < 1048576.0f) {
      wave_lds_sync();  // the zeroed histogram (cleared while the row loaded)
      fence_values(x, ng);
      // bins addressed from the raw fma bits: one shift-add per element
      int *const hist_b = hist - kBinBits;
      int one = 1;
      asm volatile("" : "+v"(one));
      // lanes whose score is below L count in a bin of their own past the
      // histogram: no branch around the atomic, distinct addresses
      const uint32_t dummy = kBinBits + (uint32_t)kWaveBins + (uint32_t)lane;
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        if (g < ng) {
#pragma unroll
          for (int i = g * kGroup; i < (g + 1) * kGroup; ++i) {
            const uint32_t bi = x[i] >= L ? lin_bits(x[i], scale, cbin) : dummy;
            atomicAdd(&hist_b[bi], one);
          }
        }
      }
      wave_lds_sync();
      int bsel, above;
      find_bucket(hist, r, bsel, above);
      m = hist[bsel];
      r -= above;
      const uint32_t bsel_bits = kBinBits + (uint32_t)bsel;
      wave_lds_sync();  // histogram reads finish before it is reused
      fence_values(x, ng);
      if (m <= 64) {
        // the bucket's members to LDS (any order), then an exact rank; most
        // items hold no member in any lane and skip the placement
        int base = 0;
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          if (g < ng) {
#pragma unroll
            for (int i = g * kGroup; i < (g + 1) * kGroup; ++i) {
              // two ballots of plain compares, combined on the scalar unit
              const uint64_t bm =
                  wv::ballot(x[i] >= L) & wv::ballot(lin_bits(x[i], scale, cbin) == bsel_bits);
              if (bm) {
                if ((bm >> lane) & 1u) list[base + lane_rank(bm)] = x[i];
                base += __popcll(bm);
              }
            }
          }
        }
        wave_lds_sync();
        rank_list(lane < m ? list[lane] : kPad, m, r, K, c_eq);
        decided = true;
        wave_lds_sync();
      } else {
        float mlo = INFINITY, mhi = -INFINITY;
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          if (g < ng) {
#pragma unroll
            for (int i = g * kGroup; i < (g + 1) * kGroup; ++i) {
              const bool mem = x[i] >= L && lin_bits(x[i], scale, cbin) == bsel_bits;
              mlo = mem ? fminf(mlo, x[i]) : mlo;
              mhi = mem ? fmaxf(mhi, x[i]) : mhi;
            }
          }
        }
        vA = __uint_as_float(wv::wave_reduce(__float_as_uint(mlo), wv::MinF()));
        vB = __uint_as_float(wv::wave_reduce(__float_as_uint(mhi), wv::MaxF()));
        if (r == m) {  // the whole bucket is taken
          K = vA;
          c_eq = kNoLimit;
          decided = true;
        }
      }
    }
  }

  // ---- key rounds (infinities, extreme ranges, crowded buckets) ----
  // members are the scores in [vA, vB]; each round histograms the 10 key bits
  // below the highest bit in which the members' extreme keys differ, so the
  // interval shrinks by 2^10 per round and at most four rounds run
#pragma unroll 1
  for (int round = 0; round < 6 && !decided; ++round) {
    const uint32_t A = score_key(vA), B = score_key(vB);
    if (A == B) {
      K = vA;
      c_eq = r;
      decided = true;
      break;
    }
    const int bl = 32 - __clz((int)(B - A));
    const int shift = bl > 10 ? bl - 10 : 0;
#pragma unroll
    for (int q = 0; q < BPL; ++q) hist[lane * BPL + q] = 0;
    wave_lds_sync();
    fence_values(x, ng);
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      if (g < ng) {
#pragma unroll
        for (int i = g * kGroup; i < (g + 1) * kGroup; ++i)
          if (x[i] >= vA && x[i] <= vB) atomicAdd(&hist[(score_key(x[i]) - A) >> shift], 1);
      }
    }
    wave_lds_sync();
    int bsel, above;
    find_bucket(hist, r, bsel, above);
    m = hist[bsel];
    wave_lds_sync();
    r -= above;
    fence_values(x, ng);
    float mlo = INFINITY, mhi = -INFINITY;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      if (g < ng) {
#pragma unroll
        for (int i = g * kGroup; i < (g + 1) * kGroup; ++i) {
          const bool mem = x[i] >= vA && x[i] <= vB && ((score_key(x[i]) - A) >> shift) == (uint32_t)bsel;
          mlo = mem ? fminf(mlo, x[i]) : mlo;
          mhi = mem ? fmaxf(mhi, x[i]) : mhi;
        }
      }
    }
    vA = __uint_as_float(wv::wave_reduce(__float_as_uint(mlo), wv::MinF()));
    vB = __uint_as_float(wv::wave_reduce(__float_as_uint(mhi), wv::MaxF()));
    if (r == m) {
      K = vA;
      c_eq = kNoLimit;
      decided = true;
    } else if (m <= 64) {
      fence_values(x, ng);
      int base = 0;
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        if (g < ng) {
#pragma unroll
          for (int i = g * kGroup; i < (g + 1) * kGroup; ++i) {
            const bool mem = x[i] >= vA && x[i] <= vB;
            const uint64_t bm = wv::ballot(mem);
            if (mem) list[base + lane_rank(bm)] = x[i];
            base += __popcll(bm);
          }
        }
      }
      wave_lds_sync();
      rank_list(lane < m ? list[lane] : kPad, m, r, K, c_eq);
      decided = true;
      wave_lds_sync();
    }
  }

  // ---- output in column order: x > K, and the first c_eq of x == K ----
  // Stores go through a resource of exactly topk entries; lanes that take
  // nothing (and any position past topk) store past it and are dropped, so
  // the pass runs without branches.
  const __amdgpu_buffer_rsrc_t orsrc = make_buffer_rsrc(orow, (uint32_t)p.topk * 4u);
  constexpr int kDrop = 0x7ffffffc;
  fence_values(x, ng);
  int pos = 0;
  if (c_eq == kNoLimit) {
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      if (g < ng) {
#pragma unroll
        for (int i = g * kGroup; i < (g + 1) * kGroup; ++i) {
          const bool t = x[i] >= K;
          const uint64_t tm = wv::ballot(t);
          const int at = pos + lane_rank(tm);
          __builtin_amdgcn_raw_buffer_store_b32((uint32_t)(st + 64 * i + lane), orsrc, t ? 4 * at : kDrop, 0, 0);
          pos += __popcll(tm);
        }
      }
    }
  } else {
    int eq_before = 0;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      if (g < ng) {
#pragma unroll
        for (int i = g * kGroup; i < (g + 1) * kGroup; ++i) {
          const bool eqv = x[i] == K;
          const uint64_t em = wv::ballot(eqv);
          const bool t = x[i] > K || (eqv && eq_before + lane_rank(em) < c_eq);
          const uint64_t tm = wv::ballot(t);
          const int at = pos + lane_rank(tm);
          __builtin_amdgcn_raw_buffer_store_b32((uint32_t)(st + 64 * i + lane), orsrc, t ? 4 * at : kDrop, 0, 0);
          pos += __popcll(tm);
          eq_before += __popcll(em);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Workgroup-per-row kernel for rows of up to NW * 64 * IPL columns: the wave
// kernel's passes with NW waves per row.  Wave w holds the contiguous segment
// of 64 * IPL columns from w * 64 * IPL (lane l: columns w * 64 * IPL + 64i + l),
// the histogram (2048 bins) is shared in LDS, and minima, maxima, counts and
// the output positions are combined across the waves through LDS.  Every wave
// scans the shared histogram itself, so all of them reach the same bucket
// without a broadcast.  The lower bound L comes from 8 interleaved subset
// maxima per lane (subset_bound), counted over the whole workgroup.
// ---------------------------------------------------------------------------
constexpr int kBlockBins = 2048;

template <int NW>
struct BlockLds {
  int hist[kBlockBins + 64];  // + one bin per lane for the scores below the bound
  float list[NW][64];   // bucket members, one region per wave
  float redf[2 * NW];
  int redi[2 * NW];
};

// Block-wide (min, max) of one wave-uniform pair; the leading barrier lets the
// previous readers of the exchange slots finish.
template <int NW>
__device__ __forceinline__ void block_minmax_f(float &lo, float &hi, BlockLds<NW> &sm, int w) {
  __syncthreads();
  if (lane_id() == 0) {
    sm.redf[w] = lo;
    sm.redf[NW + w] = hi;
  }
  __syncthreads();
  lo = sm.redf[0];
  hi = sm.redf[NW];
#pragma unroll
  for (int i = 1; i < NW; ++i) {
    lo = fminf(lo, sm.redf[i]);
    hi = fmaxf(hi, sm.redf[NW + i]);
  }
}

// Members (at most 64 over the block) to lanes: wave w wrote its `c` members
// to its own region; lane l of every wave then holds member l (in wave order).
template <int NW>
__device__ __forceinline__ float gather_members(BlockLds<NW> &sm, int w, int c, float pad) {
  __syncthreads();
  if (lane_id() == 0) sm.redi[w] = c;
  __syncthreads();
  const int lane = lane_id();
  float v = pad;
  int acc = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    const int ci = sm.redi[i];
    if (lane >= acc && lane < acc + ci) v = sm.list[i][lane - acc];
    acc += ci;
  }
  return v;
}

template <int NW, int IPL>
__global__ void __launch_bounds__(64 * NW) topk_block_kernel(const TopkParams p) {
  static_assert(IPL % kGroup == 0, "items come in whole groups");
  constexpr int NG = IPL / kGroup;
  constexpr int SEG = 64 * IPL;
  constexpr int kSub = 8;
  static_assert(kGroup % kSub == 0, "every group feeds every subset");
  __shared__ BlockLds<NW> sm;
  int *hist = sm.hist;
  const int w = __builtin_amdgcn_readfirstlane(wave_id()), lane = lane_id();
  const int tid = threadIdx.x;
  const int64_t vrow = p.row0 + blockIdx.x;
  int64_t row, st, en;
  topk_window(p, vrow, row, st, en);
  const int n = __builtin_amdgcn_readfirstlane(en > st ? (int)(en - st) : 0);
  int32_t *orow = topk_out_row(p, vrow);
  if (n <= p.topk) {  // block-uniform: the whole workgroup leaves together
    for (int i = tid; i < p.topk; i += 64 * NW) orow[i] = i < n ? (int32_t)(st + i) : -1;
    return;
  }

  // ---- load this wave's segment; groups past the window issue no loads ----
  const float *src = p.scores + row * p.row_stride + st;
  const __amdgpu_buffer_rsrc_t rsrc = make_buffer_rsrc(src, (uint32_t)n * 4u);
  const int seg0 = w * SEG;
  const int nseg = n - seg0;
  int ng = nseg <= 0 ? 0 : (nseg + 64 * kGroup - 1) / (64 * kGroup);
  ng = __builtin_amdgcn_readfirstlane(ng < NG ? ng : NG);
  const float kPad = __uint_as_float(0x7fc00000u);
  float x[IPL];
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    if (g < ng) {
#pragma unroll
      for (int i = g * kGroup; i < (g + 1) * kGroup; ++i) x[i] = buffer_load_f32(rsrc, 4 * lane, 4 * seg0 + 256 * i);
    } else {
#pragma unroll
      for (int i = g * kGroup; i < (g + 1) * kGroup; ++i) x[i] = kPad;
    }
  }
  for (int q = tid; q < kBlockBins; q += 64 * NW) hist[q] = 0;
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    if (g < ng) {
      const bool last = g == ng - 1;
#pragma unroll
      for (int i = g * kGroup; i < (g + 1) * kGroup; ++i) {
        x[i] = rank_value(x[i]);
        if (last) x[i] = (64 * i + lane < nseg) ? x[i] : kPad;
      }
    }
  }

  int r = p.topk;
  float K = 0.0f;
  int c_eq = kNoLimit;
  bool decided = false;  // block-uniform throughout
  float vA, vB;
  int m = n;

  // ---- round 0: maximum and the lower bound L (see the wave kernel) ----
  fence_values(x, ng);
  float smax[kSub];
#pragma unroll
  for (int j = 0; j < kSub; ++j) smax[j] = -INFINITY;
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    if (g < ng) {
#pragma unroll
      for (int i = g * kGroup; i < (g + 1) * kGroup; ++i) smax[i % kSub] = fmaxf(smax[i % kSub], x[i]);
    }
  }
  int nsub;
  float hi;
  float L = subset_bound(smax, nsub, hi);
  if (lane == 0) sm.redi[NW + w] = nsub;
  block_minmax_f<NW>(L, hi, sm, w);
  nsub = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) nsub += sm.redi[NW + i];
  if (r > nsub) {
    fence_values(x, ng);
    float lo = INFINITY, unused = -INFINITY;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      if (g < ng) {
#pragma unroll
        for (int i = g * kGroup; i < (g + 1) * kGroup; ++i) lo = fminf(lo, x[i]);
      }
    }
    lo = __uint_as_float(wv::wave_reduce(__float_as_uint(lo), wv::MinF()));
    block_minmax_f<NW>(lo, unused, sm, w);
    L = lo;
  }
  vA = L;
  vB = hi;
  if (L == hi) {
    K = hi;
    c_eq = r;
    decided = true;
  } else if (__builtin_isfinite(L) && __builtin_isfinite(hi)) {
    // linear buckets as in the wave kernel, 2048 of them: bins round((x - L) * scale + 1 + d)
    const float scale = (float)(kBlockBins - 3) / (hi - L);
    const float cbin = -L * scale + 12582913.0f;
    if (isfinite(scale) && fmaxf(fabsf(L), fabsf(hi)) * scale < 1048576.0f) {
      __syncthreads();  // the zeroed histogram
      fence_values(x, ng);
      int *const hist_b = hist - kBinBits;
      int one = 1;
      asm volatile("" : "+v"(one));
      // scores below L count in their lane's bin past the histogram: no
      // branch around the atomic, distinct addresses within each wave
      const uint32_t dummy = kBinBits + (uint32_t)kBlockBins + (uint32_t)lane;
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        if (g < ng) {
#pragma unroll
          for (int i = g * kGroup; i < (g + 1) * kGroup; ++i) {
            const uint32_t bi = x[i] >= L ? lin_bits(x[i], scale, cbin) : dummy;
            atomicAdd(&hist_b[bi], one);
          }
        }
      }
      __syncthreads();
      int bsel, above;
      find_bucket<kBlockBins>(hist, r, bsel, above);
      m = hist[bsel];
      r -= above;
      const uint32_t bsel_bits = kBinBits + (uint32_t)bsel;
      fence_values(x, ng);
      if (m <= 64) {
        int base = 0;
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          if (g < ng) {
#pragma unroll
            for (int i = g * kGroup; i < (g + 1) * kGroup; ++i) {
              const uint64_t bm =
                  wv::ballot(x[i] >= L) & wv::ballot(lin_bits(x[i], scale, cbin) == bsel_bits);
              if (bm) {
                if ((bm >> lane) & 1u) sm.list[w][base + lane_rank(bm)] = x[i];
                base += __popcll(bm);
              }
            }
          }
        }
        rank_list(gather_members<NW>(sm, w, base, kPad), m, r, K, c_eq);
        decided = true;
      } else {
        float mlo = INFINITY, mhi = -INFINITY;
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          if (g < ng) {
#pragma unroll
            for (int i = g * kGroup; i < (g + 1) * kGroup; ++i) {
              const bool mem = x[i] >= L && lin_bits(x[i], scale, cbin) == bsel_bits;
              mlo = mem ? fminf(mlo, x[i]) : mlo;
              mhi = mem ? fmaxf(mhi, x[i]) : mhi;
            }
          }
        }
        mlo = __uint_as_float(wv::wave_reduce(__float_as_uint(mlo), wv::MinF()));
        mhi = __uint_as_float(wv::wave_reduce(__float_as_uint(mhi), wv::MaxF()));
        block_minmax_f<NW>(mlo, mhi, sm, w);
        vA = mlo;
        vB = mhi;
        if (r == m) {
          K = vA;
          c_eq = kNoLimit;
          decided = true;
        }
      }
    }
  }

  // ---- key rounds: 11 key bits per round over the shared histogram ----
#pragma unroll 1
  for (int round = 0; round < 5 && !decided; ++round) {
    const uint32_t A = score_key(vA), B = score_key(vB);
    if (A == B) {
      K = vA;
      c_eq = r;
      decided = true;
      break;
    }
    const int bl = 32 - __clz((int)(B - A));
    const int shift = bl > 11 ? bl - 11 : 0;
    __syncthreads();  // earlier readers of the histogram are done
    for (int q = tid; q < kBlockBins; q += 64 * NW) hist[q] = 0;
    __syncthreads();
    fence_values(x, ng);
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      if (g < ng) {
#pragma unroll
        for (int i = g * kGroup; i < (g + 1) * kGroup; ++i)
          if (x[i] >= vA && x[i] <= vB) atomicAdd(&hist[(score_key(x[i]) - A) >> shift], 1);
      }
    }
    __syncthreads();
    int bsel, above;
    find_bucket<kBlockBins>(hist, r, bsel, above);
    m = hist[bsel];
    r -= above;
    fence_values(x, ng);
    float mlo = INFINITY, mhi = -INFINITY;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      if (g < ng) {
#pragma unroll
        for (int i = g * kGroup; i < (g + 1) * kGroup; ++i) {
          const bool mem = x[i] >= vA && x[i] <= vB && ((score_key(x[i]) - A) >> shift) == (uint32_t)bsel;
          mlo = mem ? fminf(mlo, x[i]) : mlo;
          mhi = mem ? fmaxf(mhi, x[i]) : mhi;
        }
      }
    }
    mlo = __uint_as_float(wv::wave_reduce(__float_as_uint(mlo), wv::MinF()));
    mhi = __uint_as_float(wv::wave_reduce(__float_as_uint(mhi), wv::MaxF()));
    block_minmax_f<NW>(mlo, mhi, sm, w);
    vA = mlo;
    vB = mhi;
    if (r == m) {
      K = vA;
      c_eq = kNoLimit;
      decided = true;
    } else if (m <= 64) {
      fence_values(x, ng);
      int base = 0;
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        if (g < ng) {
#pragma unroll
          for (int i = g * kGroup; i < (g + 1) * kGroup; ++i) {
            const uint64_t bm = wv::ballot(x[i] >= vA) & wv::ballot(x[i] <= vB);
            if (bm) {
              if ((bm >> lane) & 1u) sm.list[w][base + lane_rank(bm)] = x[i];
              base += __popcll(bm);
            }
          }
        }
      }
      rank_list(gather_members<NW>(sm, w, base, kPad), m, r, K, c_eq);
      decided = true;
    }
  }

  // ---- output in column order across the waves ----
  // per-wave counts of x >= K (or of x > K and x == K), then each wave's start
  fence_values(x, ng);
  const bool nolimit = c_eq == kNoLimit;
  int c1 = 0, c2 = 0;
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    if (g < ng) {
#pragma unroll
      for (int i = g * kGroup; i < (g + 1) * kGroup; ++i) {
        if (nolimit) {
          c1 += __popcll(wv::ballot(x[i] >= K));
        } else {
          c1 += __popcll(wv::ballot(x[i] > K));
          c2 += __popcll(wv::ballot(x[i] == K));
        }
      }
    }
  }
  __syncthreads();
  if (lane == 0) {
    sm.redi[w] = c1;
    sm.redi[NW + w] = c2;
  }
  __syncthreads();
  int pos = 0, eq_before = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    if (i < w) {
      const int ci = sm.redi[i], ei = sm.redi[NW + i];
      const int room = c_eq - eq_before;
      pos += nolimit ? ci : ci + (ei < room ? ei : (room > 0 ? room : 0));
      eq_before += ei;
    }
  }
  const __amdgpu_buffer_rsrc_t orsrc = make_buffer_rsrc(orow, (uint32_t)p.topk * 4u);
  constexpr int kDrop = 0x7ffffffc;
  const int64_t col0 = st + seg0 + lane;
  fence_values(x, ng);
  if (nolimit) {
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      if (g < ng) {
#pragma unroll
        for (int i = g * kGroup; i < (g + 1) * kGroup; ++i) {
          const bool t = x[i] >= K;
          const uint64_t tm = wv::ballot(t);
          const int at = pos + lane_rank(tm);
          __builtin_amdgcn_raw_buffer_store_b32((uint32_t)(col0 + 64 * i), orsrc, t ? 4 * at : kDrop, 0, 0);
          pos += __popcll(tm);
        }
      }
    }
  } else {
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      if (g < ng) {
#pragma unroll
        for (int i = g * kGroup; i < (g + 1) * kGroup; ++i) {
          const bool eqv = x[i] == K;
          const uint64_t em = wv::ballot(eqv);
          const bool t = x[i] > K || (eqv && eq_before + lane_rank(em) < c_eq);
          const uint64_t tm = wv::ballot(t);
          const int at = pos + lane_rank(tm);
          __builtin_amdgcn_raw_buffer_store_b32((uint32_t)(col0 + 64 * i), orsrc, t ? 4 * at : kDrop, 0, 0);
          pos += __popcll(tm);
          eq_before += __popcll(em);
        }
      }
    }
  }
}

template <int NW, int IPL>
static int launch_topk_block(const TopkParams &p, hipStream_t st) {
  hipLaunchKernelGGL((topk_block_kernel<NW, IPL>), dim3((unsigned)p.rows), dim3(64 * NW), 0, st, p);
  return check_launch("topk_select(block)");
}

template <int IPL>
static int launch_topk_wave(const TopkParams &p, hipStream_t st) {
  hipLaunchKernelGGL((topk_wave_kernel<IPL>), dim3((unsigned)((p.rows + 3) / 4)), dim3(256), 0, st, p);
  return check_launch("topk_select(wave)");
}

}  // namespace dsa

using namespace dsa;

namespace dsa {
constexpr int64_t kTopkOnePass = 32768;  // the longest row (or segment) one kernel takes

// One launch over rows (segment mode: segments) of up to kTopkOnePass columns.
static int topk_run(const TopkParams &p, hipStream_t st) {
  const int64_t len = p.nseg > 1 ? p.seg_len : p.row_len;
  // causal rows longer than 8192 columns: the rows whose window still fits
  // 8192 columns (t < 8192 - causal_offset in each batch) take one wave per
  // row instead of a workgroup whose later waves would hold no column
  if (p.nseg <= 1 && p.causal && !p.starts && len > 8192 && len <= kTopkOnePass && p.row0 == 0 &&
      p.rows % p.seq_q == 0) {
    int64_t nshort = 8192 - p.causal_offset;
    nshort = nshort < 0 ? 0 : (nshort > p.seq_q ? p.seq_q : nshort);
    if (nshort > 0 && nshort < p.seq_q) {
      for (int64_t b = 0; b < p.rows / p.seq_q; ++b) {
        TopkParams q = p;
        q.row0 = b * p.seq_q;
        q.rows = nshort;
        int rc = launch_topk_wave<128>(q, st);
        if (rc) return rc;
        q.row0 = b * p.seq_q + nshort;
        q.rows = p.seq_q - nshort;
        rc = len <= 16384 ? launch_topk_block<4, 64>(q, st) : launch_topk_block<8, 64>(q, st);
        if (rc) return rc;
      }
      return DSA_OK;
    }
  }
  if (len <= 2048) return launch_topk_wave<32>(p, st);
  if (len <= 4096) return launch_topk_wave<64>(p, st);
  if (len <= 8192) return launch_topk_wave<128>(p, st);
  if (len <= 16384) return launch_topk_block<4, 64>(p, st);
  if (len <= kTopkOnePass) return launch_topk_block<8, 64>(p, st);
  return set_error(DSA_ERR_UNSUPPORTED, "dsa_topk: rows longer than %lld columns need a workspace (dsa_topk_ws)",
                   (long long)kTopkOnePass);
}

// Rows longer than kTopkOnePass: nseg segments of seg_len columns each.  The
// chosen set under the order (value descending, NaN as +inf, ties to the lower
// column) restricted to a segment is contained in that segment's own top-k,
// so the union of the segments' picks holds the row's top-k:
//   1. segment mode: every segment's top-k columns, in column order (cand);
//   2. topk_compact_kernel: per row the segments' valid picks concatenated in
//      segment order (so still in column order) with their scores, and the
//      row's window [0, total) for the next pass;
//   3. one pass over those candidate rows (ties to the lower position are ties
//      to the lower column), positions out;
//   4. topk_map_kernel: positions back to columns.
struct TopkLong {
  int64_t nseg, seg_len, crow;  // crow = nseg * topk: candidate row length
  size_t cand, cscore, ccol, starts, ends, pos, total;  // workspace offsets
};

static TopkLong topk_long_plan(int64_t rows, int64_t row_len, int64_t topk) {
  TopkLong t;
  t.nseg = (row_len + kTopkOnePass - 1) / kTopkOnePass;
  t.seg_len = (row_len + t.nseg - 1) / t.nseg;
  t.crow = t.nseg * topk;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off += (bytes + 255) & ~(size_t)255;
    return o;
  };
  t.cand = take((size_t)rows * t.crow * 4);
  t.cscore = take((size_t)rows * t.crow * 4);
  t.ccol = take((size_t)rows * t.crow * 4);
  t.starts = take((size_t)rows * 4);
  t.ends = take((size_t)rows * 4);
  t.pos = take((size_t)rows * topk * 4);
  t.total = off;
  return t;
}

// One workgroup per row: the segments' valid picks (a segment of n window
// columns yields min(n, topk), the rest of its output is -1 padding) packed
// in segment order, with their scores.
__global__ void __launch_bounds__(256) topk_compact_kernel(const TopkParams p, const int32_t *cand, float *cscore,
                                                           int32_t *ccol, int32_t *starts2, int32_t *ends2) {
  const int64_t row = blockIdx.x;
  const int64_t crow = (int64_t)p.nseg * p.topk;
  __shared__ int off[65];
  if (threadIdx.x == 0) {
    int run = 0;
    for (int sg = 0; sg < p.nseg; ++sg) {
      int64_t r, st, en;
      topk_window(p, row * p.nseg + sg, r, st, en);
      const int64_t n = en > st ? en - st : 0;
      off[sg] = run;
      run += (int)(n < p.topk ? n : p.topk);
    }
    off[p.nseg] = run;
    starts2[row] = 0;
    ends2[row] = run;
  }
  __syncthreads();
  const float *srow = p.scores + row * p.row_stride;
  for (int64_t i = threadIdx.x; i < crow; i += 256) {
    const int sg = (int)(i / p.topk), k = (int)(i - (int64_t)sg * p.topk);
    const int dst = off[sg] + k;
    if (dst < off[sg + 1]) {
      const int32_t col = cand[row * crow + i];
      cscore[row * crow + dst] = srow[col];
      ccol[row * crow + dst] = col;
    }
  }
}

__global__ void topk_map_kernel(const TopkParams p, const int32_t *pos, const int32_t *ccol, int64_t crow) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= p.rows * p.topk) return;
  const int64_t row = i / p.topk, k = i - row * p.topk;
  const int32_t q = pos[i];
  topk_out_row(p, row)[k] = q >= 0 ? ccol[row * crow + q] : -1;
}

// p: rows of p.row_len > kTopkOnePass columns (nseg / seg_len unset).
static int topk_long(const TopkParams &p, void *ws, size_t ws_bytes, hipStream_t st) {
  const TopkLong t = topk_long_plan(p.rows, p.row_len, p.topk);
  if (t.crow > kTopkOnePass || t.nseg > 64)
    return set_error(DSA_ERR_UNSUPPORTED,
                     "dsa_topk: %lld segments x topk %d exceed one candidate pass (%lld columns)", (long long)t.nseg,
                     p.topk, (long long)kTopkOnePass);
  if (!ws || ws_bytes < t.total)
    return set_error(DSA_ERR_WORKSPACE, "dsa_topk: rows of %lld columns need a %zu-byte workspace (got %zu)",
                     (long long)p.row_len, t.total, ws_bytes);
  if (p.rows * t.nseg >= (1ll << 31) || p.rows * t.crow >= (1ll << 40))
    return set_error(DSA_ERR_INVALID_ARG, "dsa_topk: too many rows for the segment passes");
  unsigned char *w = static_cast<unsigned char *>(ws);
  int32_t *cand = reinterpret_cast<int32_t *>(w + t.cand);
  float *cscore = reinterpret_cast<float *>(w + t.cscore);
  int32_t *ccol = reinterpret_cast<int32_t *>(w + t.ccol);
  int32_t *starts2 = reinterpret_cast<int32_t *>(w + t.starts);
  int32_t *ends2 = reinterpret_cast<int32_t *>(w + t.ends);
  int32_t *pos = reinterpret_cast<int32_t *>(w + t.pos);
  TopkParams p1 = p;  // 1. per segment
  p1.rows = p.rows * t.nseg;
  p1.nseg = (int)t.nseg;
  p1.seg_len = t.seg_len;
  p1.out = cand;
  p1.out_bstride = 0;
  int rc = topk_run(p1, st);
  if (rc) return rc;
  hipLaunchKernelGGL(topk_compact_kernel, dim3((unsigned)p.rows), dim3(256), 0, st, p1, cand, cscore, ccol,
                     starts2, ends2);  // 2.
  rc = check_launch("dsa_topk(compact)");
  if (rc) return rc;
  TopkParams p2;  // 3. over the candidates
  p2.scores = cscore;
  p2.rows = p.rows;
  p2.row_len = t.crow;
  p2.row_stride = t.crow;
  p2.seq_q = 1;
  p2.causal_offset = 0;
  p2.starts = starts2;
  p2.ends = ends2;
  p2.causal = 0;
  p2.topk = p.topk;
  p2.out = pos;
  p2.out_bstride = 0;
  p2.seg_len = 0;
  p2.nseg = 1;
  p2.row0 = 0;
  rc = topk_run(p2, st);
  if (rc) return rc;
  const int64_t nout = p.rows * p.topk;  // 4.
  hipLaunchKernelGGL(topk_map_kernel, dim3((unsigned)((nout + 255) / 256)), dim3(256), 0, st, p, pos, ccol,
                     t.crow);
  return check_launch("dsa_topk(map)");
}

// nbatch batches of rows_per_batch rows (scores rows consecutive, row_stride
// apart), causal windows [0, t + 1 + causal_offset) for row t of a batch, and
// the outputs of batch b from out + b * out_bstride: one launch for all batches
// (rows over kTopkOnePass columns: the segment passes, in ws).
int topk_batched(const float *scores, int64_t rows_per_batch, int64_t nbatch, int64_t row_len, int64_t row_stride,
                 int causal, int64_t causal_offset, int64_t topk, int32_t *out, int64_t out_bstride, void *ws,
                 size_t ws_bytes, hipStream_t st) {
  DSA_REQUIRE(rows_per_batch > 0 && nbatch > 0 && row_len >= 0 && row_stride >= row_len && topk > 0 &&
                  topk < (1ll << 30) && rows_per_batch * nbatch < (1ll << 31),
              "topk_batched: bad dims");
  TopkParams p;
  p.scores = scores;
  p.rows = rows_per_batch * nbatch;
  p.row_len = row_len;
  p.row_stride = row_stride;
  p.seq_q = rows_per_batch;
  p.causal_offset = causal_offset;
  p.starts = nullptr;
  p.ends = nullptr;
  p.causal = causal;
  p.topk = (int)topk;
  p.out = out;
  p.out_bstride = out_bstride;
  p.seg_len = 0;
  p.nseg = 1;
  p.row0 = 0;
  if (row_len > kTopkOnePass) return topk_long(p, ws, ws_bytes, st);
  return topk_run(p, st);
}
}  // namespace dsa

static int topk_impl(const float *scores, int64_t rows, int64_t row_len, int64_t row_stride, int64_t seq_q,
                     int causal, int64_t causal_offset, const int32_t *starts, const int32_t *ends, int64_t topk,
                     int32_t *out_idx, void *ws, size_t ws_bytes, hipStream_t stream) {
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
  p.out_bstride = 0;
  p.seg_len = 0;
  p.nseg = 1;
  p.row0 = 0;
  if (row_len > kTopkOnePass) return topk_long(p, ws, ws_bytes, stream);
  return topk_run(p, stream);
}

extern "C" int dsa_topk(const float *scores, int64_t rows, int64_t row_len, int64_t row_stride, int64_t seq_q,
                        int causal, int64_t causal_offset, const int32_t *starts, const int32_t *ends,
                        int64_t topk, int32_t *out_idx, void *stream) {
  return topk_impl(scores, rows, row_len, row_stride, seq_q, causal, causal_offset, starts, ends, topk, out_idx,
                   nullptr, 0, static_cast<hipStream_t>(stream));
}

extern "C" size_t dsa_topk_workspace_size(int64_t rows, int64_t row_len, int64_t topk) {
  if (rows <= 0 || topk <= 0 || row_len <= kTopkOnePass) return 0;
  return topk_long_plan(rows, row_len, topk).total;
}

extern "C" int dsa_topk_ws(const float *scores, int64_t rows, int64_t row_len, int64_t row_stride, int64_t seq_q,
                           int causal, int64_t causal_offset, const int32_t *starts, const int32_t *ends,
                           int64_t topk, int32_t *out_idx, void *workspace, size_t ws_bytes, void *stream) {
  return topk_impl(scores, rows, row_len, row_stride, seq_q, causal, causal_offset, starts, ends, topk, out_idx,
                   workspace, ws_bytes, static_cast<hipStream_t>(stream));
}
