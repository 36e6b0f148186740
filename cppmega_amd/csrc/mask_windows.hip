// Row windows of an additive attention mask, and the last step of the masked
// top-k, on gfx950.
//
// Megatron's fused_qk_topk_naive(q, k, weights, topk, mask) ranks the rows of
// index_scores + mask (call shapes cppmega/megatron/lemyx_dsa_warmup.py:169-176,
// index_cache_patch.py:148-153); its additive mask is 0 / -inf (causal,
// sliding window, packed sequences) or carries finite biases.  This build
// turns the mask into per-row candidate windows, so the indexer computes only
// the key tiles inside them and the top-k ranks only their columns:
//
//  * mask_windows_kernel   one wave per mask row: the first finite column,
//    one past the last, and whether the row is "plain" -- every entry of that
//    span is +0.0 (bit pattern 0), so the row adds exactly +0.0 inside its
//    window and -inf outside.  For a plain row the window-mode indexer writes
//    score + 0.0f without reading the mask (the same bits as score + mask)
//    and no top-k pick can land on a -inf hole.  The mask is read once, 16
//    bytes per lane where the rows are 16-byte aligned.
//  * topk_finalize_kernel  one wave per row: the top-k's int32 picks (ascending,
//    -1 padded) become int64; on a row that is not plain, picks whose score is
//    -inf (holes inside the window, taken when the window holds fewer finite
//    columns than topk) are dropped and the rest stay ascending with -1
//    padding at the end.
// Both are single launches with no host synchronisation (graph-capturable),
// and deterministic (no atomics).
#include "dsa_common.hpp"

namespace dsa {
namespace mwin {

constexpr int kNT = 256;  // four waves per workgroup, one row each

struct WinParams {
  const float *mask;     // [R, Sq, Sk] (R = 1: one mask for every batch, or R = B)
  int64_t R, B, Sq, Sk;
  int32_t *starts;       // [B, Sq]
  int32_t *ends;         // [B, Sq]
  int32_t *plain;        // [B, Sq]: 1 when the row's window holds only +0.0
};

__global__ void __launch_bounds__(kNT) mask_windows_kernel(const WinParams p) {
  const int lane = lane_id();
  const int64_t row = (int64_t)blockIdx.x * (kNT / 64) + __builtin_amdgcn_readfirstlane(wave_id());
  if (row >= p.R * p.Sq) return;
  const float *src = p.mask + row * p.Sk;
  int64_t first = p.Sk, last = -1, nfin = 0, nzero = 0;
  auto visit = [&](int64_t s, float v) {
    const uint32_t u = __float_as_uint(v);
    const bool fin = (u & 0x7f800000u) != 0x7f800000u;
    first = fin && s < first ? s : first;
    last = fin && s > last ? s : last;
    nfin += fin ? 1 : 0;
    nzero += u == 0u ? 1 : 0;
  };
  if ((p.Sk & 3) == 0 && (reinterpret_cast<uintptr_t>(p.mask) & 15) == 0) {
    // four 16-byte loads per lane in flight per round (1 KiB per load instruction)
    const f32x4 *src4 = reinterpret_cast<const f32x4 *>(src);
    const int64_t n4 = p.Sk / 4;
    int64_t c0 = 0;
    for (; c0 + 256 <= n4; c0 += 256) {
      f32x4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = __builtin_nontemporal_load(src4 + c0 + 64 * u + lane);
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int j = 0; j < 4; ++j) visit(4 * (c0 + 64 * u + lane) + j, v[u][j]);
    }
    for (int64_t c = c0 + lane; c < n4; c += 64) {
      const f32x4 v = __builtin_nontemporal_load(src4 + c);
#pragma unroll
      for (int j = 0; j < 4; ++j) visit(4 * c + j, v[j]);
    }
  } else {
    for (int64_t s = lane; s < p.Sk; s += 64) visit(s, src[s]);
  }
  // wave reductions (64-bit values as two 32-bit halves are not needed: Sk < 2^31)
  int f = (int)first, l = (int)last, nf = (int)nfin, nz = (int)nzero;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const int fo = __shfl_xor(f, off, 64), lo = __shfl_xor(l, off, 64);
    f = fo < f ? fo : f;
    l = lo > l ? lo : l;
    nf += __shfl_xor(nf, off, 64);
    nz += __shfl_xor(nz, off, 64);
  }
  const bool any = l >= 0;
  const int st = any ? f : 0, en = any ? l + 1 : 0;
  // plain: every finite entry is +0.0 and the span has no -inf / NaN hole
  const int pl = (nz == nf && en - st == nf) ? 1 : 0;
  // one mask row serves every batch when R == 1
  const int64_t r = row / p.Sq, t = row % p.Sq;
  const int64_t b0 = p.R == 1 ? 0 : r, b1 = p.R == 1 ? p.B : r + 1;
  for (int64_t b = b0 + lane; b < b1; b += 64) {
    p.starts[b * p.Sq + t] = st;
    p.ends[b * p.Sq + t] = en;
    p.plain[b * p.Sq + t] = pl;
  }
}

struct FinParams {
  const float *scores;   // [rows] x row_stride (the masked scores the picks were ranked on)
  int64_t row_stride;
  const int32_t *idx;    // [rows, topk] int32, ascending, -1 padded
  const int32_t *plain;  // [rows] or NULL (no row is plain: every row is checked)
  int64_t rows, topk;
  int64_t *out;          // [rows, topk] int64
};

__global__ void __launch_bounds__(kNT) topk_finalize_kernel(const FinParams p) {
  const int lane = lane_id();
  const int64_t row = (int64_t)blockIdx.x * (kNT / 64) + __builtin_amdgcn_readfirstlane(wave_id());
  if (row >= p.rows) return;
  const int32_t *in = p.idx + row * p.topk;
  int64_t *out = p.out + row * p.topk;
  const bool plain = p.plain != nullptr && p.plain[row] != 0;  // wave-uniform
  if (plain) {
    for (int64_t i = lane; i < p.topk; i += 64) out[i] = (int64_t)in[i];
    return;
  }
  const float *srow = p.scores + row * p.row_stride;
  int64_t pos = 0;
  for (int64_t i0 = 0; i0 < p.topk; i0 += 64) {
    const int64_t i = i0 + lane;
    const int32_t c = i < p.topk ? in[i] : -1;
    const bool inrow = c >= 0 && c < p.row_stride;
    const bool keep = inrow && __float_as_uint(srow[inrow ? c : 0]) != 0xff800000u;
    const uint64_t bm = __builtin_amdgcn_ballot_w64(keep);
    const int64_t at = pos + __popcll(bm & ((1ull << lane) - 1ull));
    if (keep) out[at] = (int64_t)c;
    pos += __popcll(bm);
  }
  for (int64_t i = pos + lane; i < p.topk; i += 64) out[i] = -1;
}

}  // namespace mwin
}  // namespace dsa

using namespace dsa;

extern "C" int dsa_mask_windows(const float *mask, int64_t mask_batches, int64_t B, int64_t Sq, int64_t Sk,
                                int32_t *starts, int32_t *ends, int32_t *plain, void *stream) {
  using namespace dsa::mwin;
  DSA_REQUIRE(B > 0 && Sq >= 0 && Sk > 0 && Sk < (1ll << 31),
              "dsa_mask_windows: bad shape B=%lld Sq=%lld Sk=%lld", (long long)B, (long long)Sq, (long long)Sk);
  DSA_REQUIRE(mask_batches == 1 || mask_batches == B, "dsa_mask_windows: mask_batches %lld is neither 1 nor B=%lld",
              (long long)mask_batches, (long long)B);
  if (Sq == 0) return DSA_OK;
  DSA_REQUIRE(mask && starts && ends && plain, "dsa_mask_windows: null pointer");
  WinParams p{};
  p.mask = mask;
  p.R = mask_batches;
  p.B = B;
  p.Sq = Sq;
  p.Sk = Sk;
  p.starts = starts;
  p.ends = ends;
  p.plain = plain;
  const int64_t rows = mask_batches * Sq;
  const int64_t grid = (rows + kNT / 64 - 1) / (kNT / 64);
  DSA_REQUIRE(grid < (1ll << 31), "dsa_mask_windows: grid too large");
  hipLaunchKernelGGL(mask_windows_kernel, dim3((unsigned)grid), dim3(kNT), 0, static_cast<hipStream_t>(stream), p);
  return check_launch("mask_windows_kernel");
}

extern "C" int dsa_topk_finalize(const float *scores, int64_t row_stride, const int32_t *idx, int64_t rows,
                                 int64_t topk, const int32_t *plain, int64_t *out, void *stream) {
  using namespace dsa::mwin;
  DSA_REQUIRE(rows >= 0 && topk > 0, "dsa_topk_finalize: bad shape rows=%lld topk=%lld", (long long)rows,
              (long long)topk);
  if (rows == 0) return DSA_OK;
  DSA_REQUIRE(scores && idx && out, "dsa_topk_finalize: null pointer");
  DSA_REQUIRE(row_stride > 0, "dsa_topk_finalize: row_stride must be positive");
  FinParams p{};
  p.scores = scores;
  p.row_stride = row_stride;
  p.idx = idx;
  p.plain = plain;
  p.rows = rows;
  p.topk = topk;
  p.out = out;
  const int64_t grid = (rows + kNT / 64 - 1) / (kNT / 64);
  DSA_REQUIRE(grid < (1ll << 31), "dsa_topk_finalize: grid too large");
  hipLaunchKernelGGL(topk_finalize_kernel, dim3((unsigned)grid), dim3(kNT), 0, static_cast<hipStream_t>(stream), p);
  return check_launch("topk_finalize_kernel");
}
