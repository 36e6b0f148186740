// Exact top-k of a bounded candidate list held in LDS by one wave, under the
// deterministic top-k contract (value descending, NaN as +inf, -0 equal to +0,
// ties to the lower list position): the selection step of the fused indexer +
// top-k (indexer_score.hip).
#pragma once

#include "dsa_common.hpp"
#include "wave_ops.hpp"

namespace dsa {

// Order key of a score under the top-k contract: larger key = ranks higher.
// Integer tests only (callers may be compiled with NaNs declared absent).
__device__ __forceinline__ uint32_t score_okey(uint32_t b) {
  b = (b & 0x7fffffffu) > 0x7f800000u ? 0x7f800000u : b;  // NaN ranks as +inf
  b = (b & 0x7fffffffu) == 0u ? 0u : b;                   // -0 ranks as +0
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ int below_count(uint64_t mask) {  // set lanes below this one
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t x) { return wv::wave_reduce(x, wv::MinU()); }
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) { return wv::wave_reduce(x, wv::MaxU()); }

// Keeps the top r entries of list c (1 <= r <= n <= 64 NPL) at its front, in
// list order, under the top-k contract; returns the order key K of the r-th
// largest (every kept entry ranks at or above it) and the count kept (r).
// With prune > 0 the call may stop after the first binning round that leaves
// at most 1/prune of the n - r surplus: it then keeps every entry whose key is
// at least the least key K of the bin holding the r-th largest (at least r of
// them), in list order, and returns that K and their count.  A later entry of
// key K has a higher column than every kept entry of key K and ranks below at
// least r kept entries, so later entries need a key above K either way.
// The entries stay in registers for the whole call (order key 0 marks an
// absent one: no score has it).  Selection: each round bins the keys of the
// current range [lo, hi] into 256 bins linear in the key, keeps the bin
// holding the r-th largest and narrows the range to that bin's keys, about
// 256x per round (float bin arithmetic is exact below 2^24 and monotone
// above), until the range is one key or holds at most 64 keys, which are
// ranked exactly.  hist: this wave's 256 ints (16-byte aligned).
// The workgroup's dynamic LDS (key tiles, candidate lists, histograms).
extern __shared__ __attribute__((aligned(16))) unsigned char fsmem[];

// Not inlined: one copy of the selection code serves every call site (inlined
// at each, the kernel's code outgrew the instruction cache and every selection
// ran cold).  The list and histogram are byte offsets into fsmem, so their
// accesses stay LDS instructions.
template <int NPL>
__device__ __noinline__ uint2 cand_keep_top(uint32_t c_off, int n, int r, uint32_t hist_off, int prune) {
  prune = __builtin_amdgcn_readfirstlane(prune);
  uint2 *c = reinterpret_cast<uint2 *>(fsmem + c_off);
  int *hist = reinterpret_cast<int *>(fsmem + hist_off);
  const int lane = lane_id();
  uint32_t raw[NPL], col[NPL], key[NPL];
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const int e = lane + 64 * i;
    const uint2 v = e < n ? c[e] : make_uint2(0u, 0u);
    raw[i] = v.x;
    col[i] = v.y;
    key[i] = e < n ? score_okey(v.x) : 0u;
  }
  uint32_t mn = 0xffffffffu, mx = 0u;
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    mn = key[i] != 0u && key[i] < mn ? key[i] : mn;
    mx = key[i] > mx ? key[i] : mx;
  }
  uint32_t lo = wave_min_u32(mn), hi = wave_max_u32(mx);
  uint32_t K = lo;
  int c_eq = r;
  const int r0 = r;
#pragma unroll 1
  for (int round = 0; round < 12; ++round) {
    if (lo == hi) {
      K = lo;
      c_eq = r;
      break;
    }
    // the keys as fresh values each round: the predicates on them are
    // recomputed instead of kept as 64-bit lane masks across the rounds
#pragma unroll
    for (int i = 0; i < NPL; ++i) asm volatile("" : "+v"(key[i]));
    int m = 0;
#pragma unroll
    for (int i = 0; i < NPL; ++i) m += __popcll(__ballot(key[i] != 0u && key[i] >= lo && key[i] <= hi));
    if (m <= 64) {
      // the range's keys to LDS (any order), then each one's rank by broadcast reads
      uint32_t *list = reinterpret_cast<uint32_t *>(hist);
      int base = 0;
#pragma unroll
      for (int i = 0; i < NPL; ++i) {
        const bool in = key[i] != 0u && key[i] >= lo && key[i] <= hi;
        const uint64_t bm = __ballot(in);
        if (in) list[base + below_count(bm)] = key[i];
        base += __popcll(bm);
      }
      wave_lds_sync();
      const uint32_t v = lane < m ? list[lane] : 0u;
      int g = 0, e = 0;
#pragma unroll
      for (int j4 = 0; j4 < 16; ++j4) {
        const uint4 q4 = *reinterpret_cast<const uint4 *>(list + 4 * j4);
        const uint32_t qv[4] = {q4.x, q4.y, q4.z, q4.w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const bool ok = 4 * j4 + t < m;
          g += (ok && qv[t] > v) ? 1 : 0;
          e += (ok && qv[t] == v) ? 1 : 0;
        }
      }
      const bool found = lane < m && g < r && r <= g + e;
      const int fl = __ffsll((unsigned long long)__ballot(found)) - 1;
      const int src = fl < 0 ? 0 : fl;
      K = wv::readlane(v, src);
      c_eq = r - (int)wv::readlane((uint32_t)g, src);
      wave_lds_sync();
      break;
    }
    const float scale = 255.99f / (float)(hi - lo);
#pragma unroll
    for (int q = 0; q < 4; ++q) hist[4 * lane + q] = 0;
    wave_lds_sync();
    int bin[NPL];  // -1: outside the range
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const bool in = key[i] != 0u && key[i] >= lo && key[i] <= hi;
      const int bb = (int)((float)(in ? key[i] - lo : 0u) * scale);  // in [0, 255]
      bin[i] = in ? (bb > 255 ? 255 : bb) : -1;
      if (in) atomicAdd(&hist[bin[i]], 1);
    }
    wave_lds_sync();
    // lane l covers bins 255 - 4l - q (q = 0..3), highest first
    const int4 h4 = *reinterpret_cast<const int4 *>(hist + 252 - 4 * lane);
    const int cq[4] = {h4.w, h4.z, h4.y, h4.x};
    const int local = cq[0] + cq[1] + cq[2] + cq[3];
    const int incl = (int)wv::wave_incl_scan((uint32_t)local);
    const int excl = incl - local;
    const bool cross = excl < r && incl >= r;
    int d_l = 0, above_l = 0, inbin_l = 0;
    if (cross) {
      int acc = excl;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (acc < r && acc + cq[q] >= r) {
          d_l = 255 - 4 * lane - q;
          above_l = acc;
          inbin_l = cq[q];
        }
        acc += cq[q];
      }
    }
    const int cl = __ffsll((unsigned long long)__ballot(cross)) - 1;  // exactly one lane crosses
    const int src = cl < 0 ? 0 : cl;
    const int d = (int)wv::readlane((uint32_t)d_l, src);
    r -= (int)wv::readlane((uint32_t)above_l, src);
    const int inbin = (int)wv::readlane((uint32_t)inbin_l, src);
    wave_lds_sync();  // the histogram reads finish before it is reused
#pragma unroll
    for (int i = 0; i < NPL; ++i) asm volatile("" : "+v"(bin[i]));
    uint32_t bmn = 0xffffffffu, bmx = 0u;
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const bool in = bin[i] == d;
      bmn = in && key[i] < bmn ? key[i] : bmn;
      bmx = in && key[i] > bmx ? key[i] : bmx;
    }
    lo = wave_min_u32(bmn);
    hi = wave_max_u32(bmx);
    K = lo;  // (the loop ends on a one-key range well within its bound)
    c_eq = r;
    // pruning: every key of the bin and above stays, once that frees at
    // least 1 - 1/prune of what the exact selection would
    if (prune > 0 && prune * ((r0 - r) + inbin - r0) <= n - r0) {
      c_eq = 0x7fffffff;
      break;
    }
  }
  // keep the entries above K and the first c_eq equal to it, in list order
  // (entry e = lane + 64 i: list order is i-major); every entry is in
  // registers, so the writes cannot clobber an unread one
  int kept = 0, eq_seen = 0;
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const bool eq = key[i] != 0u && key[i] == K;
    const uint64_t em = __ballot(eq);
    const bool keep = key[i] > K || (eq && eq_seen + below_count(em) < c_eq);
    const uint64_t km = __ballot(keep);
    if (keep) c[kept + below_count(km)] = make_uint2(raw[i], col[i]);
    kept += __popcll(km);
    eq_seen += __popcll(em);
  }
  wave_lds_sync();
  return make_uint2(K, (uint32_t)kept);
}

}  // namespace dsa
