// DSA indexer scores on gfx950 MFMA (bf16 and OCP-e4m3 with per-tensor scales).
//
// score[b, t, s] = sum_h w[t, b, h] * act(q[t, b, h, :] . k[s, b, :]), fp32,
// act = ReLU (use_relu) or identity.  Reference: compute_index_scores_fused_bf16
// (cppmega/megatron/dsa_indexer_fused_patch.py:71-133), which loops over heads
// with one fp32 bmm + ReLU + weight + add over the whole [b, sq, sk] matrix per
// head.  Here the head loop disappears into the MFMA M dimension: rows are
// (token, head) pairs, so one 32x32x16 accumulator holds 32 (token, head) rows
// by 32 keys, and the ReLU, the weight and the sum over heads run on the
// accumulator registers (in-lane adds plus one cross-half exchange) before a
// single fp32 store per (token, key).
//
// Tiling: a wave keeps the q rows of 2 x 32 (token, head) rows as A operands
// in registers (4 tokens at h = 16) and streams keys through them; a workgroup
// (4 waves, 4 * 64 / h tokens) walks a 512-key chunk in 64-key tiles that are
// double-buffered in LDS and shared by its waves.  Per 32 keys a wave runs
// 2 * d / 16 MFMAs, then ReLU * w and the in-lane head sum on the
// accumulators, one permlane32 swap for the other half of the heads, and one
// coalesced fp32 store per (token, 32 keys).  Causal: chunks wholly above a
// token block do no work (mode 1 writes their -inf), and a wave skips the key
// tiles above its last token.  Late (longer) token blocks are scheduled first.
// This file is compiled with IEEE mode off and NaN inputs left undefined, so
// the ReLU is a single v_max_f32 per element.
#include <type_traits>

#include "dsa_common.hpp"
#include "wave_ops.hpp"
#include "topk_list.hpp"

namespace dsa {

struct IdxParams {
  const unsigned char *q;
  const void *w;
  const unsigned char *k;
  float *out;
  const float *q_scale;
  const float *k_scale;
  // window mode (causal == 3): row t of batch b keeps columns [starts, ends) of
  // its [B, Sq] windows, plus the additive mask (batch stride mask_bstride
  // elements, 0 = one mask for every batch; NULL = no mask); -inf elsewhere.
  // row_plain ([B, Sq], or NULL): rows whose mask holds only +0.0 inside the
  // window; their mask is not read (score + 0.0f has the bits of score + mask)
  const int32_t *starts;
  const int32_t *ends;
  const float *mask;
  int64_t mask_bstride;
  const int32_t *row_plain;
  int64_t B, Sq, Sk;
  int64_t coff;  // causal modes 1 / 2: row t keeps keys s <= t + coff (q starts coff tokens into the sequence)
  int w_f32;
  int causal;
  int relu;
};

constexpr int kCausalWindow = 3;

template <int H, int D, bool FP8>
struct IdxCfg {
  static constexpr int ELT = FP8 ? 1 : 2;
  static constexpr int MT = 2;                  // 32-row M tiles per wave
  static constexpr int TPW = MT * 32 / H;       // tokens per wave
  static constexpr int WAVES = 4;
  static constexpr int TT = TPW * WAVES;        // tokens per workgroup
  static constexpr int ROWB = D * ELT;          // bytes per key row
  static constexpr int KT = 16384 / ROWB;       // keys per LDS tile (16 KiB of key rows)
  static constexpr int SUBS = KT / 32;          // 32-key sub-tiles per tile
  static constexpr int CHUNK = 2048;            // keys per workgroup
  static constexpr int NKT = CHUNK / KT;        // tiles per workgroup chunk
  static constexpr int KS_STRIDE = ROWB + 16;
  static constexpr int KSTEPS = FP8 ? D / 64 : D / 16;  // MFMA k-steps: 32x32x64 f8f6f4 or 32x32x16 bf16
  static constexpr int CPR = ROWB / 16;         // 16-byte chunks per key row
  static constexpr int NT = 64 * WAVES;         // threads per workgroup
  static constexpr int LOADS = KT * CPR / NT;   // 16-byte loads per thread per tile
  static_assert(H == 16 || H == 32 || H == 64, "index heads must be 16, 32 or 64");
  static_assert(D % (FP8 ? 64 : 16) == 0 && LOADS >= 1 && KT * CPR % NT == 0 && CHUNK % KT == 0, "index head dim");
};

// Scores of token block [t0, t0 + TT) against keys [k0, k_end) of batch b
// (the keys of one work segment), written to the rows of that token block.
// WIN: window mode (causal == kCausalWindow), a separate instantiation so the
// other modes' register allocation does not carry the window code.
template <int H, int D, bool FP8, bool RELU, bool WIN = false>
__device__ __forceinline__ void idx_segment(const IdxParams &p, unsigned char (&KS)[2][IdxCfg<H, D, FP8>::KT * IdxCfg<H, D, FP8>::KS_STRIDE],
                                            int64_t b, int64_t t0_in, int64_t k0_in, int64_t k_end_in) {
  using C = IdxCfg<H, D, FP8>;
  // segment bounds are wave-uniform: keep them (and everything derived) scalar
  const int64_t t0 = __builtin_amdgcn_readfirstlane((int)t0_in);
  const int64_t k0 = __builtin_amdgcn_readfirstlane((int)k0_in);
  const int64_t k_end = __builtin_amdgcn_readfirstlane((int)k_end_in);
  const int tid = threadIdx.x, lane = lane_id(), w = __builtin_amdgcn_readfirstlane(wave_id());
  const int g32 = lane >> 5, l32 = lane & 31;
  const int64_t t_last = (t0 + C::TT < p.Sq ? t0 + C::TT : p.Sq) - 1;
  float *out_b = p.out + b * p.Sq * p.Sk;
  const int ntile = (int)((k_end - k0 + C::KT - 1) / C::KT);
  __syncthreads();  // the previous segment's waves are done with the key tiles

  // Memory operations of the tile loop are unconditional bounded buffer
  // accesses (loads past the end return 0, stores past the end are dropped),
  // so the compiler's memory waits are counted exactly: refilling the key tile
  // never has to wait for the score stores to reach memory.
  // Key sk of batch b sits at byte sk * row_pitch from the batch's first key.
  const uint32_t row_pitch = (uint32_t)(p.B * C::ROWB);
  const unsigned char *k_b = p.k + b * C::ROWB;
  // this block's score rows [t0, t_last]
  const auto out_rs = make_buffer_rsrc(out_b + t0 * p.Sk, (uint32_t)((t_last - t0 + 1) * p.Sk * 4));

  // ---- key tile loads (thread: LOADS 16-byte chunks of the KT-key tile) ----
  // The resource of tile `it` starts at its first key and ends at the last key
  // row (Sk - 1), so keys past the end read zeros without per-lane checks.
  // Thread tid loads chunk tid % CPR of keys tid / CPR + l * (NT / CPR): one
  // per-thread offset, the l steps in the scalar offset of the load and in the
  // immediate of the LDS store, so the tile loop keeps no per-load addresses
  // live (they had spilled to scratch, and each reload's wait drained the
  // score stores in flight)
  static_assert(C::NT % C::CPR == 0, "whole keys per load round");
  constexpr int KPR = C::NT / C::CPR;  // keys per load round
  const uint32_t loff0 = (uint32_t)(tid / C::CPR) * row_pitch + (uint32_t)(tid % C::CPR) * 16u;
  const int soff0 = (tid / C::CPR) * C::KS_STRIDE + (tid % C::CPR) * 16;
  auto load_tile = [&](int it, i32x4 (&r)[C::LOADS]) {
    const int64_t first = k0 + (int64_t)it * C::KT;
    const int64_t nkeys = p.Sk - first;
    const uint32_t nb = nkeys > 0 ? (uint32_t)((nkeys - 1) * row_pitch + C::ROWB) : 0u;
    const auto rs = make_buffer_rsrc(k_b + (nkeys > 0 ? first : 0) * row_pitch, nb);
#pragma unroll
    for (int l = 0; l < C::LOADS; ++l)
      r[l] = __builtin_bit_cast(
          i32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)loff0, (int)((uint32_t)(l * KPR) * row_pitch), 0));
  };
  auto store_tile = [&](int buf, const i32x4 (&r)[C::LOADS]) {
    unsigned char *dst = &KS[buf][soff0];
#pragma unroll
    for (int l = 0; l < C::LOADS; ++l) *reinterpret_cast<i32x4 *>(dst + l * KPR * C::KS_STRIDE) = r[l];
  };
  i32x4 kreg[C::LOADS];
  load_tile(0, kreg);

  // ---- A operands (q rows) and weights of this wave's 64 (token, head) rows ----
  // e4m3: operands of the 32x32x64 f8f6f4 MFMA, lane (row l32, half g32)
  // holding channels [16 g32, +16) and [32 + 16 g32, +16) of each 64-channel chunk
  typedef typename std::conditional<FP8, i32x8, bf16x8>::type aop_t;
  aop_t A[C::MT][C::KSTEPS];
  const int64_t wave_tok0 = t0 + w * C::TPW;
#pragma unroll
  for (int m = 0; m < C::MT; ++m) {
    const int r = m * 32 + l32;
    const int64_t t = wave_tok0 + r / H;
    const bool ok = t < p.Sq;
    const int64_t qrow = (t * p.B + b) * H + r % H;
#pragma unroll
    for (int k = 0; k < C::KSTEPS; ++k) {
      if constexpr (FP8) {
        i32x4 lo = {0, 0, 0, 0}, hi = {0, 0, 0, 0};
        if (ok) {
          lo = ld_global_16(p.q + qrow * D + 64 * k + 16 * g32);
          hi = ld_global_16(p.q + qrow * D + 64 * k + 32 + 16 * g32);
        }
        A[m][k] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      } else {
        i32x4 v = {0, 0, 0, 0};
        if (ok) v = ld_global_16(p.q + (qrow * D + 16 * k + 8 * g32) * 2);
        A[m][k] = as_bf16x8(v);
      }
    }
  }
  // w of row `lane` (token lane / H, head lane % H); e4m3: times q_scale * k_scale,
  // which commutes with the ReLU because the scales are positive
  float wl = 0.0f;
  {
    const int64_t t = wave_tok0 + lane / H;
    if (t < p.Sq) {
      const int64_t wi = (t * p.B + b) * H + lane % H;
      wl = p.w_f32 ? static_cast<const float *>(p.w)[wi] : bf16_bits_to_f32(static_cast<const uint16_t *>(p.w)[wi]);
    }
    if constexpr (FP8) wl *= p.q_scale[0] * p.k_scale[0];
  }
  float wv[C::MT][16];  // weight of each accumulator row
#pragma unroll
  for (int m = 0; m < C::MT; ++m)
#pragma unroll
    for (int a = 0; a < 16; ++a) wv[m][a] = __shfl(wl, m * 32 + 8 * (a >> 2) + 4 * g32 + (a & 3), 64);

  // Scores of one 32-key sub-tile: part[tl] = sum over the wave's heads of token
  // tl held in this lane's accumulator rows (the other half-wave holds the rest).
  // this lane's B-operand row and column group in a key tile; the sub-tile and
  // k-step parts of the address are immediates of the LDS reads
  const int brow_off = l32 * C::KS_STRIDE + 16 * g32;
  auto subtile = [&](const unsigned char *ks, int sub, float (&part)[C::TPW]) {
#pragma unroll
    for (int tl = 0; tl < C::TPW; ++tl) part[tl] = 0.0f;
#pragma unroll
    for (int m = 0; m < C::MT; ++m) {
      f32x16 acc;
#pragma unroll
      for (int a = 0; a < 16; ++a) acc[a] = 0.0f;
#pragma unroll
      for (int k = 0; k < C::KSTEPS; ++k) {
        const unsigned char *brow = ks + brow_off + sub * 32 * C::KS_STRIDE;  // + 16 g32 folded in
        if constexpr (FP8) {
          const i32x4 lo = *reinterpret_cast<const i32x4 *>(brow + 64 * k);
          const i32x4 hi = *reinterpret_cast<const i32x4 *>(brow + 64 * k + 32);
          const i32x8 bv = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          // unit block scales (E8M0 127 = 2^0): a plain e4m3 product, two k-chunks of 32
          acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(A[m][k], bv, acc, 0, 0, 0, 127, 0, 127);
        } else {
          const i32x4 bv = *reinterpret_cast<const i32x4 *>(brow + 32 * k);  // (16 k + 8 g32) bf16
          acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[m][k], as_bf16x8(bv), acc, 0, 0, 0);
        }
      }
#pragma unroll
      for (int a = 0; a < 16; ++a) {
        const int tl = (m * 32 + 8 * (a >> 2)) / H;
        const float x = RELU ? fmaxf(acc[a], 0.0f) : acc[a];  // one v_max_f32 (IEEE mode off)
        part[tl] = fmaf(x, wv[m][a], part[tl]);
      }
    }
  };

  // Interior sub-tiles (every key below or on the wave's first token, inside
  // Sk, all tokens inside Sq) store without checks: tokens are paired so one
  // permlane32 swap and one add leave token 2j's total in lanes 0-31 and token
  // 2j+1's in lanes 32-63 (each the low half plus the high half), and one
  // full-wave store writes both rows; the sub-tile's key offset rides in the
  // store's scalar offset.
  constexpr int NPAIR = C::TPW >= 2 ? C::TPW / 2 : 1;
  uint32_t soff_lane[NPAIR];
#pragma unroll
  for (int j = 0; j < NPAIR; ++j) {
    const int tl = C::TPW >= 2 ? 2 * j + g32 : 0;
    soff_lane[j] = (uint32_t)(((wave_tok0 + tl - t0) * p.Sk + k0 + l32) * 4);
  }
  const bool wave_in_sq = wave_tok0 + C::TPW - 1 < p.Sq;

  // window mode: this wave's token windows (wave-uniform scalar loads) and
  // their union; sub-tiles outside the union are not computed
  constexpr bool win = WIN;
  int wst[C::TPW], wen[C::TPW];
  bool wpl[C::TPW];  // the row's mask is +0.0 inside its window: not read
  int64_t wmin = 0, wmax = 0;
  // the intersection of the wave's windows, when every one of its rows is
  // plain: key tiles inside it take the interior path (score + 0.0f == score)
  int64_t wisect_lo = 0, wisect_hi = 0;
  if (win) {
    wmin = p.Sk;
    bool all_plain = true;
    wisect_hi = p.Sk;
#pragma unroll
    for (int tl = 0; tl < C::TPW; ++tl) {
      const int64_t t = wave_tok0 + tl;
      wst[tl] = t < p.Sq ? p.starts[b * p.Sq + t] : 0;
      wen[tl] = t < p.Sq ? p.ends[b * p.Sq + t] : 0;
      wpl[tl] = p.row_plain != nullptr && t < p.Sq && p.row_plain[b * p.Sq + t] != 0;
      all_plain = all_plain && wpl[tl];
      wisect_lo = wst[tl] > wisect_lo ? wst[tl] : wisect_lo;
      wisect_hi = wen[tl] < wisect_hi ? wen[tl] : wisect_hi;
      if (wen[tl] > wst[tl]) {
        wmin = wst[tl] < wmin ? wst[tl] : wmin;
        wmax = wen[tl] > wmax ? wen[tl] : wmax;
      }
    }
    if (!all_plain) wisect_hi = wisect_lo;  // no interior tiles
  }
  // additive mask rows of this token block (an empty resource without a mask: loads read 0)
  const float *mask_b = (win && p.mask) ? p.mask + b * p.mask_bstride + t0 * p.Sk : nullptr;
  const auto mask_rs = make_buffer_rsrc(mask_b, mask_b ? (uint32_t)((t_last - t0 + 1) * p.Sk * 4) : 0u);

  store_tile(0, kreg);
  __syncthreads();
  const int64_t wave_tok_last = wave_tok0 + C::TPW - 1;
  for (int it = 0; it < ntile; ++it) {
    load_tile(it + 1, kreg);  // past the last tile: keys beyond Sk read 0, unused
    const unsigned char *ks = KS[it & 1];
    const int64_t tk = k0 + (int64_t)it * C::KT;
    const bool interior = wave_in_sq && tk + C::KT <= k_end &&
                          (win ? (wisect_lo <= tk && tk + C::KT <= wisect_hi)
                               : (!p.causal || tk + C::KT - 1 <= wave_tok0 + p.coff));
    if (interior) {
#pragma unroll
      for (int sub = 0; sub < C::SUBS; ++sub) {
        float part[C::TPW];
        subtile(ks, sub, part);
        const int soff = (int)((uint32_t)(it * C::KT + sub * 32) * 4u);
        if constexpr (C::TPW >= 2) {
#pragma unroll
          for (int j = 0; j < NPAIR; ++j) {
            const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(part[2 * j]),
                                                            __float_as_uint(part[2 * j + 1]), false, false);
            const float v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), out_rs, (int)soff_lane[0 + j], soff, 0);
          }
        } else {
          const float v = sum_halves(part[0]);
          if (g32 == 0) __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), out_rs, (int)soff_lane[0], soff, 0);
        }
      }
    } else {
#pragma unroll
      for (int sub = 0; sub < C::SUBS; ++sub) {
        const int64_t sn = tk + sub * 32;
        // wave-uniform: the sub-tile exists and is not wholly above this wave's
        // diagonal (lower-triangle mode) or outside its windows (window mode)
        const bool active = sn < k_end && !(p.causal == 2 && sn > wave_tok_last + p.coff) &&
                            !(win && (sn + 32 <= wmin || sn >= wmax));
        const int64_t s = sn + l32;
        float mv[C::TPW];  // window mode: the additive mask, loaded ahead of the MFMAs
#pragma unroll
        for (int tl = 0; tl < C::TPW; ++tl) {
          const int64_t t = wave_tok0 + tl;
          const bool ld = win && active && t < p.Sq && s < p.Sk && !wpl[tl];
          mv[tl] = buffer_load_f32(mask_rs, ld ? (int)(((t - t0) * p.Sk + s) * 4) : (int)0xffffffffu, 0);
        }
        float part[C::TPW];
        if (active) {
          subtile(ks, sub, part);
        } else {
#pragma unroll
          for (int tl = 0; tl < C::TPW; ++tl) part[tl] = 0.0f;
        }
        // the stores are issued on every path (inactive ones land past the
        // resource and are dropped), which keeps the memory wait counts exact
#pragma unroll
        for (int tl = 0; tl < C::TPW; ++tl) {
          float v = sum_halves(part[tl]);
          const bool mine = C::TPW == 1 ? (g32 == 0) : ((tl & 1) == g32);
          const int64_t t = wave_tok0 + tl;
          bool above = (p.causal == 1 || p.causal == 2) && s > t + p.coff;
          if (win) {
            above = s < wst[tl] || s >= wen[tl];
            v += mv[tl];
          }
          if (above) v = -INFINITY;  // modes 1 and 3 write it, mode 2 skips the store
          const bool st = (active || (win && sn < k_end)) && mine && t < p.Sq && s < p.Sk && !(above && p.causal == 2);
          const uint32_t off = st ? (uint32_t)(((t - t0) * p.Sk + s) * 4) : 0xffffffffu;
          __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), out_rs, (int)off, 0, 0);
        }
      }
    }
    if (it + 1 < ntile) {
      store_tile((it + 1) & 1, kreg);
      __syncthreads();
    }
  }
}

// -inf into columns [c0, c1) of rows [t0, t_last] of a [., Sk] score matrix,
// row by row; 16-byte stores over the 16-byte-aligned middle of each row.
template <int NT>
__device__ __forceinline__ void fill_neg_inf_rows(float *out_b, int64_t Sk, int64_t t0, int64_t t_last, int64_t c0,
                                                  int64_t c1) {
  if (c1 <= c0) return;
  const f32x4 ninf4 = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
  for (int64_t t = t0; t <= t_last; ++t) {
    float *row = out_b + t * Sk;
    int64_t a = c0;
    while ((reinterpret_cast<uintptr_t>(row + a) & 15) != 0) {  // unaligned head (at most 3 columns)
      if (a >= c1) break;
      if (threadIdx.x == 0) row[a] = -INFINITY;
      ++a;
    }
    const int64_t nv = a < c1 ? (c1 - a) / 4 : 0;
    if ((reinterpret_cast<uintptr_t>(row + a) & 15) == 0) {
      for (int64_t c = threadIdx.x; c < nv; c += NT) reinterpret_cast<f32x4 *>(row + a)[c] = ninf4;
      a += 4 * nv;
    }
    for (int64_t c = a + threadIdx.x; c < c1; c += NT) row[c] = -INFINITY;
  }
}

// Rows of token blocks have different lengths in lower-triangle mode (block tb
// computes keys [0, last token]), so a grid of fixed key chunks leaves some
// compute units with 64 times the work of others.  Lower-triangle mode pairs
// the long block NTB-1-j with the short block j instead: the pair's combined
// row length is the same for every j, and splitting it into `pieces` equal
// ranges of 32-key sub-tiles gives every workgroup the same work.  A piece is
// at most two segments (the end of the long row, the start of the short one).
// Window mode pairs the blocks the same way over their window unions (for a
// causal mask: the lower triangle's balance).  Modes 0 and 1 keep fixed chunks
// of CHUNK keys (all rows as long as Sk).  WIN selects the window-mode
// instantiation (launched for causal == kCausalWindow only).
template <int H, int D, bool FP8, bool RELU, bool WIN>
__global__ void __launch_bounds__((IdxCfg<H, D, FP8>::NT))
__attribute__((amdgpu_waves_per_eu(!WIN && (FP8 || D <= 64) ? 3 : 2)))
indexer_score_kernel(const IdxParams p) {
  using C = IdxCfg<H, D, FP8>;
  __shared__ __attribute__((aligned(16))) unsigned char KS[2][C::KT * C::KS_STRIDE];
  const int64_t b = blockIdx.z;
  if (!WIN && p.causal == 2) {
    const int64_t ntb = (p.Sq + C::TT - 1) / C::TT;
    const int64_t tb_long = ntb - 1 - (int64_t)blockIdx.y, tb_short = blockIdx.y;
    // a block's row: keys [0, min(last token + 1, Sk)), in 32-key sub-tiles
    auto row_keys = [&](int64_t tb) {
      const int64_t t_last = (tb * C::TT + C::TT < p.Sq ? tb * C::TT + C::TT : p.Sq) - 1;
      return t_last + 1 + p.coff < p.Sk ? t_last + 1 + p.coff : p.Sk;
    };
    const int64_t keys_long = row_keys(tb_long), keys_short = tb_short < tb_long ? row_keys(tb_short) : 0;
    const int64_t n_long = (keys_long + 31) / 32, n = n_long + (keys_short + 31) / 32;
    const int64_t pieces = gridDim.x;
    const int64_t lo = (int64_t)blockIdx.x * n / pieces, hi = ((int64_t)blockIdx.x + 1) * n / pieces;
#pragma unroll 1
    for (int sg = 0; sg < 2; ++sg) {
      const int64_t a = sg == 0 ? lo : (lo > n_long ? lo : n_long) - n_long;  // first sub-tile
      const int64_t e = sg == 0 ? (hi < n_long ? hi : n_long) : hi - n_long;  // end sub-tile
      const int64_t keys = sg == 0 ? keys_long : keys_short;
      if (e > a) idx_segment<H, D, FP8, RELU>(p, KS, b, (sg == 0 ? tb_long : tb_short) * C::TT, a * 32,
                                             e * 32 < keys ? e * 32 : keys);
    }
    return;
  }
  if constexpr (WIN) {
    // Window mode, paired like the lower triangle: block ntb-1-j with block j,
    // each computing the 32-key sub-tiles of its token windows' union
    // [lo, hi) (rounded out to 32 keys), the pair's sub-tiles split into equal
    // pieces; every piece also writes -inf into its share of the two blocks'
    // rows outside their unions (rows piece, piece + pieces, ...).
    const int64_t ntb = (p.Sq + C::TT - 1) / C::TT;
    const int64_t tb_long = ntb - 1 - (int64_t)blockIdx.y, tb_short = blockIdx.y;
    const bool has_short = tb_short < tb_long;
    __shared__ int uni[4];  // lo / hi of the long block, then of the short block
    if (threadIdx.x < 64) {
      const int lane = (int)threadIdx.x;
      const int64_t tb = lane < 32 ? tb_long : tb_short;
      const int tl = lane & 31;
      const int64_t t = tb * C::TT + tl;
      const bool ok = tl < C::TT && t < p.Sq && (lane < 32 || has_short);
      int st = ok ? p.starts[b * p.Sq + t] : 0, en = ok ? p.ends[b * p.Sq + t] : 0;
      st = st < 0 ? 0 : st;
      en = en > p.Sk ? (int)p.Sk : en;
      if (en <= st) { st = 0x7fffffff; en = 0; }
      for (int off = 16; off >= 1; off >>= 1) {  // within each half of the wave
        const int so = __shfl_xor(st, off, 64), eo = __shfl_xor(en, off, 64);
        st = so < st ? so : st;
        en = eo > en ? eo : en;
      }
      if (tl == 0) {
        const int lo32 = en > 0 ? st / 32 * 32 : 0;
        int hi32 = en > 0 ? (en + 31) / 32 * 32 : 0;
        hi32 = hi32 > p.Sk ? (int)p.Sk : hi32;
        uni[(lane >> 5) * 2] = lo32;
        uni[(lane >> 5) * 2 + 1] = hi32;
      }
    }
    __syncthreads();
    const int64_t lo_l = uni[0], hi_l = uni[1], lo_s = uni[2], hi_s = has_short ? uni[3] : uni[2];
    const int64_t n_long = (hi_l - lo_l + 31) / 32, n = n_long + (hi_s - lo_s + 31) / 32;
    const int64_t pieces = gridDim.x;
    const int64_t lo = (int64_t)blockIdx.x * n / pieces, hi = ((int64_t)blockIdx.x + 1) * n / pieces;
#pragma unroll 1
    for (int sg = 0; sg < 2; ++sg) {
      const int64_t a = sg == 0 ? lo : (lo > n_long ? lo : n_long) - n_long;
      const int64_t e = sg == 0 ? (hi < n_long ? hi : n_long) : hi - n_long;
      const int64_t k_lo = sg == 0 ? lo_l : lo_s, k_hi = sg == 0 ? hi_l : hi_s;
      if (e > a) {
        const int64_t kb_end = k_lo + e * 32;
        idx_segment<H, D, FP8, RELU, true>(p, KS, b, (sg == 0 ? tb_long : tb_short) * C::TT, k_lo + a * 32,
                                           kb_end < k_hi ? kb_end : k_hi);
      }
    }
    // -inf outside the unions, rows of both blocks shared out among the pair's pieces
    float *out_b = p.out + b * p.Sq * p.Sk;
#pragma unroll 1
    for (int sg = 0; sg < (has_short ? 2 : 1); ++sg) {
      const int64_t t0s = (sg == 0 ? tb_long : tb_short) * C::TT;
      const int64_t t_end = t0s + C::TT < p.Sq ? t0s + C::TT : p.Sq;
      const int64_t k_lo = sg == 0 ? lo_l : lo_s, k_hi = sg == 0 ? hi_l : hi_s;
      for (int64_t t = t0s + blockIdx.x; t < t_end; t += pieces) {
        fill_neg_inf_rows<C::NT>(out_b, p.Sk, t, t, 0, k_lo);
        fill_neg_inf_rows<C::NT>(out_b, p.Sk, t, t, k_hi > k_lo ? k_hi : 0, p.Sk);
      }
    }
    return;
  } else {
  const int64_t t0 = (int64_t)(gridDim.y - 1 - blockIdx.y) * C::TT;
  const int64_t k0 = (int64_t)blockIdx.x * C::CHUNK;
  const int64_t t_last = (t0 + C::TT < p.Sq ? t0 + C::TT : p.Sq) - 1;
  const int64_t chunk_end = k0 + C::CHUNK < p.Sk ? k0 + C::CHUNK : p.Sk;
  const bool outside = p.causal == 1 && k0 > t_last + p.coff;
  if (outside) {
    // chunk wholly above the block's diagonal (mode 1): -inf only
    fill_neg_inf_rows<C::NT>(p.out + b * p.Sq * p.Sk, p.Sk, t0, t_last, k0, chunk_end);
    return;
  }
  idx_segment<H, D, FP8, RELU>(p, KS, b, t0, k0, chunk_end);
  }
}

// Workgroups of `kernel` resident at once on the current device (cached per device).
template <class K>
static int64_t resident_groups(K kernel, int threads) {
  // cached per (device, kernel): kernels of one signature share the type K
  struct Entry { const void *k; int dev; int groups; };
  static Entry cache[256];
  static int used = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  const void *kp = reinterpret_cast<const void *>(kernel);
  for (int i = 0; i < used; ++i)
    if (cache[i].k == kp && cache[i].dev == dev) return cache[i].groups;
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) != hipSuccess)
    return 0;
  const int groups = cus * (per_cu > 0 ? per_cu : 1);
  if (used < 256) cache[used++] = Entry{kp, dev, groups};
  return groups;
}

// Pieces per block pair: the smallest count (1..8) whose grid fills the
// resident workgroup slots within 2% of the best whole-round efficiency.
static int pick_pieces(int64_t groups_per_piece, int64_t slots) {
  if (slots <= 0 || groups_per_piece <= 0) return 1;
  int best_p = 1;
  double best = -1.0;
  for (int pc = 1; pc <= 8; ++pc) {
    const int64_t g = groups_per_piece * pc;
    const double eff = (double)g / (double)(((g + slots - 1) / slots) * slots);
    if (eff > best + 0.02) {
      best = eff;
      best_p = pc;
    }
  }
  return best_p;
}

template <int H, int D, bool FP8, bool RELU>
static int launch_idx_act(const IdxParams &p, hipStream_t st) {
  using C = IdxCfg<H, D, FP8>;
  const int64_t ntb = (p.Sq + C::TT - 1) / C::TT;
  DSA_REQUIRE(ntb < 65536, "dsa_indexer_scores: %lld query tokens exceed the grid (%d per workgroup)",
              (long long)p.Sq, C::TT);
  dim3 grid;
  if (p.causal == 2 || p.causal == kCausalWindow) {
    const int64_t npairs = (ntb + 1) / 2;
    const bool w = p.causal == kCausalWindow;
    const int pieces = pick_pieces(npairs * p.B, w ? resident_groups(indexer_score_kernel<H, D, FP8, RELU, true>, C::NT)
                                                   : resident_groups(indexer_score_kernel<H, D, FP8, RELU, false>, C::NT));
    grid = dim3((unsigned)pieces, (unsigned)npairs, (unsigned)p.B);
  } else {
    grid = dim3((unsigned)((p.Sk + C::CHUNK - 1) / C::CHUNK), (unsigned)ntb, (unsigned)p.B);
  }
  if (p.causal == kCausalWindow)
    hipLaunchKernelGGL((indexer_score_kernel<H, D, FP8, RELU, true>), grid, dim3(C::NT), 0, st, p);
  else
    hipLaunchKernelGGL((indexer_score_kernel<H, D, FP8, RELU, false>), grid, dim3(C::NT), 0, st, p);
  return check_launch("indexer_scores");
}

template <int H, int D, bool FP8>
static int launch_idx(const IdxParams &p, hipStream_t st) {
  return p.relu ? launch_idx_act<H, D, FP8, true>(p, st) : launch_idx_act<H, D, FP8, false>(p, st);
}

}  // namespace dsa

using namespace dsa;

static int indexer_scores_impl(const void *q, const void *w, const void *k, float *scores, int64_t B, int64_t Sq,
                               int64_t Sk, int64_t H, int64_t D, int dtype, int w_dtype, const float *q_scale,
                               const float *k_scale, int causal, const int32_t *starts, const int32_t *ends,
                               const float *mask, int64_t mask_bstride, const int32_t *row_plain, int use_relu,
                               hipStream_t st, const char *fn, int64_t coff = 0) {
  DSA_REQUIRE(B >= 0 && Sq >= 0 && Sk >= 0 && H > 0 && D > 0, "%s: bad dims", fn);
  DSA_REQUIRE(dtype == DSA_DTYPE_BF16 || dtype == DSA_DTYPE_E4M3, "%s: dtype %d", fn, dtype);
  DSA_REQUIRE(w_dtype == DSA_DTYPE_BF16 || w_dtype == DSA_DTYPE_F32, "%s: w dtype %d", fn, w_dtype);
  if (B == 0 || Sq == 0 || Sk == 0) return DSA_OK;
  DSA_REQUIRE(q && w && k && scores, "%s: null tensor pointer", fn);
  DSA_REQUIRE(Sk < (1ll << 31) && B < 65536, "%s: grid too large", fn);
  DSA_REQUIRE(Sk * B * D < (1ll << 31) && Sk < (1ll << 25),
              "%s: k (%lld x %lld x %lld) or score rows too large for 32-bit offsets", fn, (long long)Sk,
              (long long)B, (long long)D);
  const bool f8 = dtype == DSA_DTYPE_E4M3;
  if (f8) DSA_REQUIRE(q_scale && k_scale, "%s: e4m3 input needs q_scale and k_scale", fn);
  IdxParams p;
  p.q = static_cast<const unsigned char *>(q);
  p.w = w;
  p.k = static_cast<const unsigned char *>(k);
  p.out = scores;
  p.q_scale = q_scale;
  p.k_scale = k_scale;
  p.starts = starts;
  p.ends = ends;
  p.mask = mask;
  p.mask_bstride = mask_bstride;
  p.row_plain = row_plain;
  p.B = B;
  p.Sq = Sq;
  p.Sk = Sk;
  p.coff = coff;
  p.w_f32 = w_dtype == DSA_DTYPE_F32;
  p.causal = causal;
  p.relu = use_relu != 0;
#define DSA_IDX_CASE(HH, DD)                                                              \
  if (H == HH && D == DD) return f8 ? launch_idx<HH, DD, true>(p, st) : launch_idx<HH, DD, false>(p, st);
  DSA_IDX_CASE(16, 64)
  DSA_IDX_CASE(32, 64)
  DSA_IDX_CASE(64, 64)
  DSA_IDX_CASE(16, 128)
  DSA_IDX_CASE(32, 128)
  DSA_IDX_CASE(64, 128)
#undef DSA_IDX_CASE
  return set_error(DSA_ERR_UNSUPPORTED, "%s: no kernel for h=%lld d=%lld", fn, (long long)H, (long long)D);
}

extern "C" int dsa_indexer_scores(const void *q, const void *w, const void *k, float *scores, int64_t B,
                                  int64_t Sq, int64_t Sk, int64_t H, int64_t D, int dtype, int w_dtype,
                                  const float *q_scale, const float *k_scale, int causal, int use_relu,
                                  void *stream) {
  DSA_REQUIRE(causal >= 0 && causal <= 2, "dsa_indexer_scores: causal must be 0, 1 or 2");
  return indexer_scores_impl(q, w, k, scores, B, Sq, Sk, H, D, dtype, w_dtype, q_scale, k_scale, causal, nullptr,
                             nullptr, nullptr, 0, nullptr, use_relu, static_cast<hipStream_t>(stream),
                             "dsa_indexer_scores");
}

extern "C" int dsa_indexer_scores_masked(const void *q, const void *w, const void *k, float *scores, int64_t B,
                                         int64_t Sq, int64_t Sk, int64_t H, int64_t D, int dtype, int w_dtype,
                                         const float *q_scale, const float *k_scale, const int32_t *starts,
                                         const int32_t *ends, const float *mask, int64_t mask_bstride,
                                         const int32_t *row_plain, int use_relu, void *stream) {
  DSA_REQUIRE(starts && ends, "dsa_indexer_scores_masked: null window arrays");
  DSA_REQUIRE(mask_bstride >= 0, "dsa_indexer_scores_masked: negative mask batch stride");
  return indexer_scores_impl(q, w, k, scores, B, Sq, Sk, H, D, dtype, w_dtype, q_scale, k_scale, kCausalWindow,
                             starts, ends, mask, mask_bstride, row_plain, use_relu, static_cast<hipStream_t>(stream),
                             "dsa_indexer_scores_masked");
}

// ---------------------------------------------------------------------------
// Streaming indexer + top-k: query rows in chunks through a bounded scratch
// ---------------------------------------------------------------------------
namespace dsa {

// out_scores[b, r0 + t, j] = scratch[b][t][idx] for the chunk's picks (-inf for -1 padding)
// scratch rows are `pitch` scores wide (the chunk's key range)
__global__ void __launch_bounds__(256) gather_topk_scores_kernel(const float *scratch, const int32_t *idx,
                                                                 float *out, int64_t B, int64_t Sq, int64_t rows,
                                                                 int64_t r0, int64_t pitch, int64_t topk) {
  const int64_t e = blockIdx.x * 256ll + threadIdx.x;
  if (e >= B * rows * topk) return;
  const int64_t j = e % topk, t = (e / topk) % rows, b = e / (topk * rows);
  const int64_t o = (b * Sq + r0 + t) * topk + j;
  const int32_t c = idx[o];
  out[o] = (c >= 0 && c < pitch) ? scratch[(b * rows + t) * pitch + c] : -INFINITY;
}

// Scores of a chunk of query rows [r0, r0 + rows) need keys [0, pitch): all Sk
// keys, or with causal rows only up to the chunk's last query position.
static int64_t stream_pitch(int64_t r0, int64_t rows, int64_t Sk, bool causal) {
  return causal && r0 + rows < Sk ? r0 + rows : Sk;
}
// Workspace of a chunk: its [B, rows, pitch] scores, then (rows over 32768
// keys) the top-k's segment passes.
static size_t stream_chunk_bytes(int64_t B, int64_t rows, int64_t pitch, int64_t topk) {
  return (((size_t)(B * rows * pitch * 4) + 255) & ~(size_t)255) + dsa_topk_workspace_size(B * rows, pitch, topk);
}
// Most rows from r0 whose chunk fits the workspace (at least one when a
// full-width row does; the need only grows with rows).
static int64_t stream_next_rows(int64_t B, int64_t Sq, int64_t Sk, int64_t r0, bool causal, int64_t topk,
                                size_t bytes) {
  int64_t lo = 1, hi = Sq - r0;
  while (lo < hi) {
    const int64_t mid = lo + (hi - lo + 1) / 2;
    if (stream_chunk_bytes(B, mid, stream_pitch(r0, mid, Sk, causal), topk) <= bytes) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

}  // namespace dsa

extern "C" size_t dsa_indexer_topk_streaming_workspace_size(int64_t B, int64_t Sq, int64_t Sk, int64_t chunk_rows) {
  if (B <= 0 || Sq <= 0 || Sk <= 0 || chunk_rows <= 0) return 0;
  const int64_t cr = chunk_rows < Sq ? chunk_rows : Sq;
  return (size_t)B * cr * Sk * 4;
}

extern "C" int dsa_indexer_topk_streaming(const void *q, const void *w, const void *k, int32_t *out_idx,
                                          float *out_scores, int64_t B, int64_t Sq, int64_t Sk, int64_t H, int64_t D,
                                          int dtype, int w_dtype, const float *q_scale, const float *k_scale,
                                          int64_t topk, int causal, int use_relu, void *workspace,
                                          size_t workspace_bytes, void *stream) {
  DSA_REQUIRE(B >= 0 && Sq >= 0 && Sk >= 0 && H > 0 && D > 0 && topk > 0,
              "dsa_indexer_topk_streaming: bad dims");
  DSA_REQUIRE(causal == 0 || causal == 1, "dsa_indexer_topk_streaming: causal must be 0 or 1");
  if (B == 0 || Sq == 0) return DSA_OK;
  DSA_REQUIRE(out_idx, "dsa_indexer_topk_streaming: null out_idx");
  if (!workspace || stream_chunk_bytes(B, 1, Sk, topk) > workspace_bytes)
    return set_error(DSA_ERR_WORKSPACE,
                     "dsa_indexer_topk_streaming: workspace %zu bytes holds no score row (need >= %zu per query row)",
                     workspace_bytes, stream_chunk_bytes(B, 1, Sk, topk));
  hipStream_t st = static_cast<hipStream_t>(stream);
  float *scratch = static_cast<float *>(workspace);
  const int64_t elt = dtype == DSA_DTYPE_E4M3 ? 1 : 2;
  const int64_t welt = w_dtype == DSA_DTYPE_F32 ? 4 : 2;
  for (int64_t r0 = 0, rows = 0; r0 < Sq; r0 += rows) {
    // query rows [r0, r0 + rows): q / w start r0 tokens in; causal keys s <= r0 + t,
    // so a causal chunk's scratch rows span only keys [0, r0 + rows) and early
    // chunks take more rows
    rows = stream_next_rows(B, Sq, Sk, r0, causal != 0, topk, workspace_bytes);
    const int64_t pitch = stream_pitch(r0, rows, Sk, causal != 0);
    const size_t sbytes = ((size_t)(B * rows * pitch * 4) + 255) & ~(size_t)255;
    const unsigned char *qc = static_cast<const unsigned char *>(q) + r0 * B * H * D * elt;
    const unsigned char *wc = static_cast<const unsigned char *>(w) + r0 * B * H * welt;
    int rc = indexer_scores_impl(qc, wc, k, scratch, B, rows, pitch, H, D, dtype, w_dtype, q_scale, k_scale,
                                 causal ? 2 : 0, nullptr, nullptr, nullptr, 0, nullptr, use_relu, st,
                                 "dsa_indexer_topk_streaming", causal ? r0 : 0);
    if (rc) return rc;
    // every batch's rows in one top-k launch (outputs Sq * topk apart)
    rc = topk_batched(scratch, rows, B, pitch, pitch, causal, causal ? r0 : 0, topk, out_idx + r0 * topk,
                      Sq * topk, static_cast<unsigned char *>(workspace) + sbytes, workspace_bytes - sbytes, st);
    if (rc) return rc;
    if (out_scores) {
      const int64_t n = B * rows * topk;
      hipLaunchKernelGGL(gather_topk_scores_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, scratch,
                         out_idx, out_scores, B, Sq, rows, r0, pitch, topk);
      rc = check_launch("indexer_topk_streaming(gather)");
      if (rc) return rc;
    }
  }
  return DSA_OK;
}

// ---------------------------------------------------------------------------
// Fused indexer + top-k: the top-k of every query row without writing its
// scores anywhere.  One workgroup walks all keys of a token block (causal:
// the long block ntb-1-j, then the short block j, so every workgroup does the
// same work); each wave keeps, per query row of its tokens, a candidate list
// in LDS, appended in column order as the 32-key sub-tiles are scored (the
// same scoring code as idx_segment, so the scores are bit-identical to the
// dense indexer's).  A row's list takes every key until it would overflow;
// then a selection keeps the row's current top-k (under the top-k contract:
// value descending, NaN as +inf, -0 equal to +0, ties to the lower column)
// and raises the row's threshold to the k-th kept value.  Later keys enter
// only above it: a key equal to it has a higher column than every kept equal
// one and loses the tie.  (A selection short of the last may prune
// instead: it keeps a superset of the top-k, every key at or above a
// threshold with at least k kept keys at or above it, so the same argument
// holds.)  At the end an exact selection leaves the row's top-k.
// ---------------------------------------------------------------------------
namespace dsa {

struct FusedTopkOut {
  int32_t *idx;    // [B, Sq, topk]: ascending columns, -1 padding
  float *scores;   // [B, Sq, topk] or NULL: the selected scores, -inf padding
  int topk;
};

// Candidates held per query row (8 bytes each: raw score bits, column).  The
// list must keep room for a sub-tile's 32 keys after a selection leaves topk.
template <int H> struct FusedCap { static constexpr int value = H == 16 ? 896 : (H == 32 ? 1792 : 3584); };
constexpr int kFusedSlack = 64;

template <int H, int D, bool FP8>
struct FusedCfg {
  using C = IdxCfg<H, D, FP8>;
  static constexpr int CAP = FusedCap<H>::value;
  static constexpr int KS_BYTES = 2 * C::KT * C::KS_STRIDE;
  static constexpr int CAND_BYTES = C::WAVES * C::TPW * CAP * 8;
  static constexpr int HIST_BYTES = C::WAVES * 256 * 4;
  static constexpr int LDS_BYTES = KS_BYTES + CAND_BYTES + HIST_BYTES;
  static_assert(LDS_BYTES <= 160 * 1024, "fused indexer + top-k LDS");
};

// One token block [t0, t0 + TT) of batch b over all of its keys (causal: keys
// s <= t), its rows' top-k written at the end.
template <int H, int D, bool FP8, bool RELU>
__device__ __forceinline__ void idx_block_topk(const IdxParams &p, const FusedTopkOut &o, unsigned char *smem,
                                               int64_t b, int64_t t0_in) {
  using F = FusedCfg<H, D, FP8>;
  using C = IdxCfg<H, D, FP8>;
  constexpr int CAP = F::CAP;
  unsigned char (&KS)[2][C::KT * C::KS_STRIDE] = *reinterpret_cast<unsigned char (*)[2][C::KT * C::KS_STRIDE]>(smem);
  const int64_t t0 = __builtin_amdgcn_readfirstlane((int)t0_in);
  const int tid = threadIdx.x, lane = lane_id(), w = __builtin_amdgcn_readfirstlane(wave_id());
  const int g32 = lane >> 5, l32 = lane & 31;
  uint2 *cand = reinterpret_cast<uint2 *>(smem + F::KS_BYTES) + w * C::TPW * CAP;  // [TPW][CAP] of this wave
  const uint32_t cand_off = (uint32_t)(F::KS_BYTES + w * C::TPW * CAP * 8);        // the same, in fsmem
  const uint32_t hist_off = (uint32_t)(F::KS_BYTES + F::CAND_BYTES + w * 256 * 4);  // this wave's 256 ints
  const int64_t t_last = (t0 + C::TT < p.Sq ? t0 + C::TT : p.Sq) - 1;
  const int64_t kend = p.causal ? (t_last + 1 < p.Sk ? t_last + 1 : p.Sk) : p.Sk;
  const int ntile = (int)((kend + C::KT - 1) / C::KT);
  const int topk = o.topk;
  __syncthreads();  // the previous block's waves are done with the key tiles

  const uint32_t row_pitch = (uint32_t)(p.B * C::ROWB);
  const unsigned char *k_b = p.k + b * C::ROWB;
  static_assert(C::NT % C::CPR == 0, "whole keys per load round");
  constexpr int KPR = C::NT / C::CPR;
  const uint32_t loff0 = (uint32_t)(tid / C::CPR) * row_pitch + (uint32_t)(tid % C::CPR) * 16u;
  const int soff0 = (tid / C::CPR) * C::KS_STRIDE + (tid % C::CPR) * 16;
  auto load_tile = [&](int it, i32x4 (&r)[C::LOADS]) {
    const int64_t first = (int64_t)it * C::KT;
    const int64_t nkeys = p.Sk - first;
    const uint32_t nb = nkeys > 0 ? (uint32_t)((nkeys - 1) * row_pitch + C::ROWB) : 0u;
    const auto rs = make_buffer_rsrc(k_b + (nkeys > 0 ? first : 0) * row_pitch, nb);
#pragma unroll
    for (int l = 0; l < C::LOADS; ++l)
      r[l] = __builtin_bit_cast(
          i32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)loff0, (int)((uint32_t)(l * KPR) * row_pitch), 0));
  };
  auto store_tile = [&](int buf, const i32x4 (&r)[C::LOADS]) {
    unsigned char *dst = &KS[buf][soff0];
#pragma unroll
    for (int l = 0; l < C::LOADS; ++l) *reinterpret_cast<i32x4 *>(dst + l * KPR * C::KS_STRIDE) = r[l];
  };
  i32x4 kreg[C::LOADS];
  if (ntile > 0) load_tile(0, kreg);

  // A operands and weights of this wave's rows (as idx_segment)
  typedef typename std::conditional<FP8, i32x8, bf16x8>::type aop_t;
  aop_t A[C::MT][C::KSTEPS];
  const int64_t wave_tok0 = t0 + w * C::TPW;
#pragma unroll
  for (int m = 0; m < C::MT; ++m) {
    const int r = m * 32 + l32;
    const int64_t t = wave_tok0 + r / H;
    const bool ok = t < p.Sq;
    const int64_t qrow = (t * p.B + b) * H + r % H;
#pragma unroll
    for (int k = 0; k < C::KSTEPS; ++k) {
      if constexpr (FP8) {
        i32x4 lo = {0, 0, 0, 0}, hi = {0, 0, 0, 0};
        if (ok) {
          lo = ld_global_16(p.q + qrow * D + 64 * k + 16 * g32);
          hi = ld_global_16(p.q + qrow * D + 64 * k + 32 + 16 * g32);
        }
        A[m][k] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      } else {
        i32x4 v = {0, 0, 0, 0};
        if (ok) v = ld_global_16(p.q + (qrow * D + 16 * k + 8 * g32) * 2);
        A[m][k] = as_bf16x8(v);
      }
    }
  }
  float wl = 0.0f;
  {
    const int64_t t = wave_tok0 + lane / H;
    if (t < p.Sq) {
      const int64_t wi = (t * p.B + b) * H + lane % H;
      wl = p.w_f32 ? static_cast<const float *>(p.w)[wi] : bf16_bits_to_f32(static_cast<const uint16_t *>(p.w)[wi]);
    }
    if constexpr (FP8) wl *= p.q_scale[0] * p.k_scale[0];
  }
  float wv[C::MT][16];
#pragma unroll
  for (int m = 0; m < C::MT; ++m)
#pragma unroll
    for (int a = 0; a < 16; ++a) wv[m][a] = __shfl(wl, m * 32 + 8 * (a >> 2) + 4 * g32 + (a & 3), 64);

  const int brow_off = l32 * C::KS_STRIDE + 16 * g32;
  auto subtile = [&](const unsigned char *ks, int sub, float (&part)[C::TPW]) {
#pragma unroll
    for (int tl = 0; tl < C::TPW; ++tl) part[tl] = 0.0f;
#pragma unroll
    for (int m = 0; m < C::MT; ++m) {
      f32x16 acc;
#pragma unroll
      for (int a = 0; a < 16; ++a) acc[a] = 0.0f;
#pragma unroll
      for (int k = 0; k < C::KSTEPS; ++k) {
        const unsigned char *brow = ks + brow_off + sub * 32 * C::KS_STRIDE;
        if constexpr (FP8) {
          const i32x4 lo = *reinterpret_cast<const i32x4 *>(brow + 64 * k);
          const i32x4 hi = *reinterpret_cast<const i32x4 *>(brow + 64 * k + 32);
          const i32x8 bv = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(A[m][k], bv, acc, 0, 0, 0, 127, 0, 127);
        } else {
          const i32x4 bv = *reinterpret_cast<const i32x4 *>(brow + 32 * k);
          acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[m][k], as_bf16x8(bv), acc, 0, 0, 0);
        }
      }
#pragma unroll
      for (int a = 0; a < 16; ++a) {
        const int tl = (m * 32 + 8 * (a >> 2)) / H;
        const float x = RELU ? fmaxf(acc[a], 0.0f) : acc[a];
        part[tl] = fmaf(x, wv[m][a], part[tl]);
      }
    }
  };

  // per query row of the wave (wave-uniform): list length, threshold key, and
  // whether the list still takes every key (no selection yet)
  int cnt[C::TPW], thr[C::TPW], opn[C::TPW];
#pragma unroll
  for (int tl = 0; tl < C::TPW; ++tl) {
    cnt[tl] = 0;
    thr[tl] = 0;
    opn[tl] = 1;
  }
  // select_row keeps row tl's current top-k (exact), or prunes its list to a
  // superset of it with a raised threshold (wave-uniform call).
  // Pruning selections (1/32 of the surplus over the top-k may stay) short of
  // the final one save the exact ranking's share of a call: measured 11%
  // faster at 16 heads (cfg3), 6% at 64 (cfg5), 4% at 32 (1/8 and 1/16 of the
  // surplus: 1-3% less gain).  Only where the kept list always leaves the
  // slack free.
  constexpr int PRUNE = 32;
  const int prune = topk + (CAP - topk) / PRUNE <= CAP - kFusedSlack ? PRUNE : 0;
  auto select_row = [&](int tl, bool exact) {
    const uint2 kk = cand_keep_top<CAP / 64>(cand_off + (uint32_t)(tl * CAP * 8), cnt[tl], topk, hist_off,
                                             exact ? 0 : prune);
    // (the count wave-uniform, so the list tests stay scalar branches)
    cnt[tl] = __builtin_amdgcn_readfirstlane((int)kk.y);
    thr[tl] = (int)kk.x;
    opn[tl] = 0;
  };
  // the scores of this lane's row tl at key s (valid: a candidate of the row)
  constexpr int NPAIR = C::TPW >= 2 ? C::TPW / 2 : 1;
  auto emit = [&](int j, float v, int64_t s) {
    const int tl = C::TPW >= 2 ? 2 * j + g32 : 0;
    const int t_lo = C::TPW >= 2 ? 2 * j : 0, t_hi = C::TPW >= 2 ? 2 * j + 1 : 0;
    const int64_t t = wave_tok0 + tl;
    const int64_t lim = p.causal ? (t + 1 < p.Sk ? t + 1 : p.Sk) : p.Sk;
    const bool valid = t < p.Sq && s < lim && (C::TPW >= 2 || g32 == 0);
    const uint32_t key = score_okey(__float_as_uint(v));
    bool in = valid && ((g32 ? opn[t_hi] : opn[t_lo]) != 0 || key > (uint32_t)(g32 ? thr[t_hi] : thr[t_lo]));
    uint64_t bm = __ballot(in);
    int n0 = __popc((uint32_t)bm), n1 = __popc((uint32_t)(bm >> 32));
    if (cnt[t_lo] + n0 > CAP || (C::TPW >= 2 && cnt[t_hi] + n1 > CAP)) {  // rare, wave-uniform
      if (cnt[t_lo] + n0 > CAP) select_row(t_lo, false);
      if (C::TPW >= 2 && cnt[t_hi] + n1 > CAP) select_row(t_hi, false);
      in = valid && ((g32 ? opn[t_hi] : opn[t_lo]) != 0 || key > (uint32_t)(g32 ? thr[t_hi] : thr[t_lo]));
      bm = __ballot(in);
      n0 = __popc((uint32_t)bm);
      n1 = __popc((uint32_t)(bm >> 32));
    }
    if (in) {
      const uint32_t half = g32 ? (uint32_t)(bm >> 32) : (uint32_t)bm;
      const int pos = (g32 ? cnt[t_hi] : cnt[t_lo]) + __popc(half & ((1u << l32) - 1u));
      cand[tl * CAP + pos] = make_uint2(__float_as_uint(v), (uint32_t)s);
    }
    cnt[t_lo] += n0;
    if (C::TPW >= 2) cnt[t_hi] += n1;
  };

  if (ntile > 0) store_tile(0, kreg);
  __syncthreads();
  const int64_t wave_tok_last = wave_tok0 + C::TPW - 1;
  for (int it = 0; it < ntile; ++it) {
    load_tile(it + 1, kreg);  // past the last tile: keys beyond Sk read 0, unused
    const unsigned char *ks = KS[it & 1];
#pragma unroll 1
    for (int sub = 0; sub < C::SUBS; ++sub) {
      const int64_t sn = (int64_t)it * C::KT + sub * 32;
      // wave-uniform: the sub-tile exists and is not wholly above the wave's diagonal
      if (sn >= kend || (p.causal && sn > wave_tok_last)) break;
      float part[C::TPW];
      subtile(ks, sub, part);
      const int64_t s = sn + l32;
      if constexpr (C::TPW >= 2) {
#pragma unroll
        for (int j = 0; j < NPAIR; ++j) {
          // token 2j's total in lanes 0-31, token 2j+1's in lanes 32-63 (as idx_segment)
          const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(part[2 * j]),
                                                          __float_as_uint(part[2 * j + 1]), false, false);
          emit(j, __uint_as_float(r[0]) + __uint_as_float(r[1]), s);
        }
      } else {
        emit(0, sum_halves(part[0]), s);
      }
    }
    if (it + 1 < ntile) {
      store_tile((it + 1) & 1, kreg);
      __syncthreads();
    }
  }

  // each row: its list's top-k, in column order
#pragma unroll
  for (int tl = 0; tl < C::TPW; ++tl) {
    if (cnt[tl] > topk) select_row(tl, true);
    wave_lds_sync();
    const int64_t t = wave_tok0 + tl;
    if (t < p.Sq) {
      int32_t *oi = o.idx + (b * p.Sq + t) * topk;
      float *os = o.scores ? o.scores + (b * p.Sq + t) * topk : nullptr;
      const uint2 *c = cand + tl * CAP;
      for (int e = lane; e < topk; e += 64) {
        const bool has = e < cnt[tl];
        const uint2 v = has ? c[e] : make_uint2(0u, 0u);
        oi[e] = has ? (int32_t)v.y : -1;
        if (os) os[e] = has ? __uint_as_float(v.x) : -INFINITY;
      }
    }
  }
}

template <int H, int D, bool FP8, bool RELU>
__global__ void __launch_bounds__(256) indexer_topk_fused_kernel(const IdxParams p, const FusedTopkOut o) {
  using C = IdxCfg<H, D, FP8>;
  const int64_t b = blockIdx.y;
  if (p.causal) {
    const int64_t ntb = (p.Sq + C::TT - 1) / C::TT;
    const int64_t tb_long = ntb - 1 - (int64_t)blockIdx.x, tb_short = blockIdx.x;
    idx_block_topk<H, D, FP8, RELU>(p, o, fsmem, b, tb_long * C::TT);
    if (tb_short < tb_long) idx_block_topk<H, D, FP8, RELU>(p, o, fsmem, b, tb_short * C::TT);
  } else {
    idx_block_topk<H, D, FP8, RELU>(p, o, fsmem, b, (int64_t)blockIdx.x * C::TT);
  }
}

template <int H, int D, bool FP8, bool RELU>
static int launch_fused_act(const IdxParams &p, const FusedTopkOut &o, hipStream_t st) {
  using C = IdxCfg<H, D, FP8>;
  using F = FusedCfg<H, D, FP8>;
  const int64_t ntb = (p.Sq + C::TT - 1) / C::TT;
  DSA_REQUIRE(ntb < (1ll << 31), "dsa_indexer_topk_fused: too many query tokens");
  const auto kern = indexer_topk_fused_kernel<H, D, FP8, RELU>;
  const hipError_t e = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           F::LDS_BYTES);
  if (e != hipSuccess) return set_error(DSA_ERR_HIP, "dsa_indexer_topk_fused: LDS attribute: %s", hipGetErrorString(e));
  const dim3 grid((unsigned)(p.causal ? (ntb + 1) / 2 : ntb), (unsigned)p.B);
  hipLaunchKernelGGL(kern, grid, dim3(C::NT), F::LDS_BYTES, st, p, o);
  return check_launch("dsa_indexer_topk_fused");
}

template <int H, int D, bool FP8>
static int launch_fused(const IdxParams &p, const FusedTopkOut &o, hipStream_t st) {
  return p.relu ? launch_fused_act<H, D, FP8, true>(p, o, st) : launch_fused_act<H, D, FP8, false>(p, o, st);
}

}  // namespace dsa

extern "C" int64_t dsa_indexer_topk_fused_max_topk(int64_t H, int64_t D) {
  if (!(D == 64 || D == 128)) return 0;
  if (H == 16) return FusedCap<16>::value - kFusedSlack;
  if (H == 32) return FusedCap<32>::value - kFusedSlack;
  if (H == 64) return FusedCap<64>::value - kFusedSlack;
  return 0;
}

extern "C" int dsa_indexer_topk_fused(const void *q, const void *w, const void *k, int32_t *out_idx, float *out_scores,
                                      int64_t B, int64_t Sq, int64_t Sk, int64_t H, int64_t D, int dtype,
                                      int w_dtype, const float *q_scale, const float *k_scale, int64_t topk,
                                      int causal, int use_relu, void *stream) {
  DSA_REQUIRE(B >= 0 && Sq >= 0 && Sk >= 0 && H > 0 && D > 0 && topk > 0, "dsa_indexer_topk_fused: bad dims");
  DSA_REQUIRE(causal == 0 || causal == 1, "dsa_indexer_topk_fused: causal must be 0 or 1");
  DSA_REQUIRE(dtype == DSA_DTYPE_BF16 || dtype == DSA_DTYPE_E4M3, "dsa_indexer_topk_fused: dtype %d", dtype);
  DSA_REQUIRE(w_dtype == DSA_DTYPE_BF16 || w_dtype == DSA_DTYPE_F32, "dsa_indexer_topk_fused: w dtype %d", w_dtype);
  const int64_t maxk = dsa_indexer_topk_fused_max_topk(H, D);
  if (maxk == 0 || topk > maxk)
    return set_error(DSA_ERR_UNSUPPORTED, "dsa_indexer_topk_fused: h=%lld d=%lld topk=%lld (at most %lld)",
                     (long long)H, (long long)D, (long long)topk, (long long)maxk);
  if (B == 0 || Sq == 0) return DSA_OK;
  DSA_REQUIRE(q && w && (k || Sk == 0) && out_idx, "dsa_indexer_topk_fused: null tensor pointer");
  DSA_REQUIRE(Sk < (1ll << 25) && B < 65536 && Sk * B * D < (1ll << 31),
              "dsa_indexer_topk_fused: k (%lld x %lld x %lld) too large for 32-bit offsets", (long long)Sk,
              (long long)B, (long long)D);
  const bool f8 = dtype == DSA_DTYPE_E4M3;
  if (f8) DSA_REQUIRE(q_scale && k_scale, "dsa_indexer_topk_fused: e4m3 input needs q_scale and k_scale");
  IdxParams p;
  memset(&p, 0, sizeof(p));
  p.q = static_cast<const unsigned char *>(q);
  p.w = w;
  p.k = static_cast<const unsigned char *>(k);
  p.q_scale = q_scale;
  p.k_scale = k_scale;
  p.B = B;
  p.Sq = Sq;
  p.Sk = Sk;
  p.w_f32 = w_dtype == DSA_DTYPE_F32;
  p.causal = causal;
  p.relu = use_relu != 0;
  FusedTopkOut o{out_idx, out_scores, (int)topk};
  hipStream_t st = static_cast<hipStream_t>(stream);
#define DSA_FUSED_CASE(HH, DD) \
  if (H == HH && D == DD) return f8 ? launch_fused<HH, DD, true>(p, o, st) : launch_fused<HH, DD, false>(p, o, st);
  DSA_FUSED_CASE(16, 64)
  DSA_FUSED_CASE(32, 64)
  DSA_FUSED_CASE(64, 64)
  DSA_FUSED_CASE(16, 128)
  DSA_FUSED_CASE(32, 128)
  DSA_FUSED_CASE(64, 128)
#undef DSA_FUSED_CASE
  return set_error(DSA_ERR_UNSUPPORTED, "dsa_indexer_topk_fused: no kernel for h=%lld d=%lld", (long long)H,
                   (long long)D);
}
