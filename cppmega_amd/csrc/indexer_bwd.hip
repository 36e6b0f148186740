// Backward of the DSA indexer scores on gfx950 MFMA (bf16).
//
// Forward: score[b, t, s] = sum_h w[t, b, h] * act(L[b, t, h, s]),
//          L = q[t, b, h, :] . k[s, b, :]    (act = ReLU or identity).
// Given G = d loss / d score [B, Sq, Sk] (fp32):
//   dw[t, b, h]    = sum_s G[b, t, s] * act(L)
//   dq[t, b, h, :] = w[t, b, h] * sum_s G[b, t, s] * act'(L) * k[s, b, :]
//   dk[s, b, :]    = sum_{t, h} G[b, t, s] * w[t, b, h] * act'(L) * q[t, b, h, :]
// (act'(L) = [L > 0] for ReLU, 1 otherwise).  These are the gradients autograd
// takes through the reference's per-head loop (cppmega/megatron/dsa_indexer_fused_patch.py:71-133:
// fp32 bmm, ReLU, times the head weight, summed over heads), which Megatron
// relies on when the indexer is trained by its KL loss.
//
// Two MFMA kernels recompute L, so the [b, t, h, s] logits never exist:
//   * indexer_bwd_q_kernel, query-major: a wave keeps 64 (token, head) rows of q
//     in registers and streams LDS key tiles; L^T = K Q^T leaves one row per lane
//     (and 16 keys in its registers), so dw is a per-lane running sum and the
//     weight factors out of dq: dq^T[d][row] += K^T[d][key] M[key][row] with
//     M = G * act'(L) rounded to bf16, scaled by w[row] once at the end.
//   * indexer_bwd_k_kernel, key-major: a wave keeps 64 keys in registers and
//     streams LDS tiles of q rows of one token chunk; L = Q K^T leaves one key
//     per lane, M = G * w * act'(L) (bf16) and dk^T[d][key] += Q^T[d][row] M[row][key];
//     each (key block, token chunk) writes an fp32 partial, and dk_reduce_kernel
//     sums the chunks in chunk order.
// Both orders are fixed by the shapes, so results are bitwise reproducible.
// causal != 0 restricts every sum to s <= t (G above the diagonal is ignored).
// Row windows (starts / ends, one [start, end) per (batch, query row)) restrict
// them further to start <= s < end: the window-mode forward writes -inf there
// whatever the raw score, so G outside the windows carries no gradient, and
// key tiles outside every window of a workgroup's rows are not computed.  The
// key-major kernel then marks, per (batch, token chunk, key block), whether it
// wrote a partial, and the reduction sums only those.
#include <type_traits>

#include "dsa_common.hpp"

namespace dsa {

struct IdxBwdParams {
  const float *g;            // [B, Sq, Sk]
  const unsigned char *q;    // [Sq, B, H, D] bf16
  const void *w;             // [Sq, B, H] f32 or bf16
  const unsigned char *k;    // [Sk, B, D] bf16
  uint16_t *dq;              // [Sq, B, H, D] bf16
  void *dw;                  // [Sq, B, H] (w's dtype)
  float *dk_part;            // [B][nch][Sk][D] f32
  uint16_t *dk;              // [Sk, B, D] bf16
  int64_t B, Sq, Sk;
  int w_f32, causal;
  int gvec;                  // G rows 16-byte aligned (Sk % 4 == 0): 16-byte G loads
  int nch, tc;               // token chunks of the key-major kernel and their length
  const int32_t *starts;     // [B, Sq] row windows [start, end), or NULL (no windows)
  const int32_t *ends;
  int32_t *kflags;           // windows: [B][nch][nkb], 1 where the key-major kernel wrote a partial
  int nkb;                   // key blocks of the key-major kernel
};

// Key range [lo, hi) of row t of batch b: the causal limit and the row window.
__device__ __forceinline__ void row_keys(const IdxBwdParams &p, int64_t b, int64_t t, int &lo, int &hi) {
  const int sk = (int)p.Sk;
  lo = 0;
  hi = p.causal ? (t + 1 < p.Sk ? (int)t + 1 : sk) : sk;
  if (p.ends != nullptr) {
    const int st = p.starts[b * p.Sq + t], en = p.ends[b * p.Sq + t];
    lo = st > 0 ? st : 0;
    hi = en < hi ? en : hi;
  }
  if (hi < lo) hi = lo;
}

template <int H, int D>
struct IdxBwdCfg {
  // 32-row tiles per wave (q kernel) / 32-key tiles per wave (k kernel): two at
  // d = 64, one at d = 128 (the accumulators of two would not fit 256 VGPRs)
  static constexpr int MT = D == 64 ? 2 : 1;
  static constexpr int RPW = MT * 32;          // (token, head) rows per wave (q kernel)
  static constexpr int WAVES = 4;
  static constexpr int NT = 64 * WAVES;
  static constexpr int TT = RPW * WAVES / H;   // tokens per workgroup (q kernel)
  static constexpr int ROWB = D * 2;           // bytes per bf16 row
  static constexpr int KT = 16384 / ROWB;      // rows per LDS tile (16 KiB)
  static constexpr int SUBS = KT / 32;
  static constexpr int STRIDE = ROWB + 32;     // LDS row stride: 32-byte pad for the transposed reads
  static constexpr int KSTEPS = D / 16;
  static constexpr int DT = D / 32;            // 32-wide d tiles
  static constexpr int CPR = ROWB / 16;        // 16-byte chunks per row
  static constexpr int LOADS = KT * CPR / NT;  // 16-byte loads per thread per tile
  static constexpr int KB = WAVES * MT * 32;   // keys per workgroup (k kernel)
  // G staged in LDS with each tile, one tile ahead: q kernel [TT tokens][KT keys],
  // k kernel [KT / H tokens][KB keys] (f32), in 16-byte pieces per thread
  static constexpr int GQ_PIECES = TT * KT / 4;
  static constexpr int GQ_PER_T = (GQ_PIECES + NT - 1) / NT;
  static constexpr int TPT = KT / H > 0 ? KT / H : 1;  // tokens per k-kernel row tile
  static constexpr int GK_PIECES = TPT * KB / 4;
  static constexpr int GK_PER_T = (GK_PIECES + NT - 1) / NT;
  static_assert(H == 16 || H == 32 || H == 64, "index heads must be 16, 32 or 64");
  static_assert((D == 64 || D == 128) && LOADS >= 1 && KT * CPR % NT == 0, "index head dim");
  static_assert(TT >= 1 && (RPW * WAVES) % H == 0, "whole tokens per workgroup");
};

__device__ __forceinline__ float ld_w(const IdxBwdParams &p, int64_t i) {
  return p.w_f32 ? static_cast<const float *>(p.w)[i] : bf16_bits_to_f32(static_cast<const uint16_t *>(p.w)[i]);
}

// ---------------------------------------------------------------------------
// dq, dw: one workgroup per (token block, batch), longest rows first.
// WIN: row windows (p.starts / p.ends), an instantiation of its own so that the
// causal / full kernel carries no window bounds in its per-element mask.
// ---------------------------------------------------------------------------
template <int H, int D, bool RELU, bool WIN>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
indexer_bwd_q_kernel(const IdxBwdParams p) {
  using C = IdxBwdCfg<H, D>;
  __shared__ __attribute__((aligned(16))) unsigned char KS[2][C::KT * C::STRIDE];
  __shared__ __attribute__((aligned(16))) float GS[2][C::TT * C::KT];
  // Items (token block, batch) in decreasing row length.  The first half of the
  // grid takes them longest first and the second half shortest first, so the
  // two workgroups that share a compute unit (grid positions k and k + n/2 when
  // the dispatcher fills one slot per unit, then the next) have complementary
  // lengths.
  const int64_t ntb = (p.Sq + C::TT - 1) / C::TT;
  const int64_t n_items = ntb * p.B;
  const int64_t half = (n_items + 1) / 2;
  const int64_t wg = blockIdx.x;
  const int64_t item = wg < half ? wg : n_items - 1 - (wg - half);
  const int64_t b = item % p.B;
  const int64_t t0 = (ntb - 1 - item / p.B) * C::TT;
  const int tid = threadIdx.x, lane = lane_id(), w = __builtin_amdgcn_readfirstlane(wave_id());
  const int g32 = lane >> 5, l32 = lane & 31;
  const int64_t t_last = (t0 + C::TT < p.Sq ? t0 + C::TT : p.Sq) - 1;
  int64_t kend = p.causal ? (t_last + 1 < p.Sk ? t_last + 1 : p.Sk) : p.Sk;
  int64_t kbeg = 0;  // keys below every row's window start are skipped
  if constexpr (WIN) {
    // the union of the workgroup's row ranges (TT <= 64 tokens: one per lane, in every wave)
    int lo = 0x7fffffff, hi = 0;
    if (lane < C::TT && t0 + lane <= t_last) {
      int a, e;
      row_keys(p, b, t0 + lane, a, e);
      if (e > a) { lo = a; hi = e; }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const int lo2 = __shfl_xor(lo, off, 64), hi2 = __shfl_xor(hi, off, 64);
      lo = lo2 < lo ? lo2 : lo;
      hi = hi2 > hi ? hi2 : hi;
    }
    kend = __builtin_amdgcn_readfirstlane(hi);
    kbeg = hi > 0 ? __builtin_amdgcn_readfirstlane(lo) : 0;
  }
  const int it0 = (int)(kbeg / C::KT);
  const int ntile = (int)((kend + C::KT - 1) / C::KT);
  const int64_t wave_row0 = t0 * H + w * C::RPW;      // (token, head) rows t * H + h
  const int64_t wave_tok_last = (wave_row0 + C::RPW - 1) / H;
  int64_t wave_kend = p.causal ? (wave_tok_last + 1 < p.Sk ? wave_tok_last + 1 : p.Sk) : p.Sk;
  // keys [wave_klo, wave_khi) lie in every row's range of the wave (causal: below its
  // first token + 1; windows: the intersection of the rows' windows, set below)
  const int64_t wave_tok0 = wave_row0 / H;
  int64_t wave_klo = 0;
  int64_t wave_khi = p.causal ? (wave_tok0 + 1 < p.Sk ? wave_tok0 + 1 : p.Sk) : p.Sk;

  // key tiles: rows [first, first + KT) of batch b through a resource ending at the last key
  const uint32_t row_pitch = (uint32_t)(p.B * C::ROWB);
  const unsigned char *k_b = p.k + b * C::ROWB;
  uint32_t loff[C::LOADS];
#pragma unroll
  for (int l = 0; l < C::LOADS; ++l) {
    const int u = tid + C::NT * l;
    loff[l] = (uint32_t)(u / C::CPR) * row_pitch + (uint32_t)(u % C::CPR) * 16u;
  }
  // G rows of this workgroup's tokens through one resource (past it: zeros)
  const float *g_b = p.g + (b * p.Sq + t0) * p.Sk;
  const int sk32 = (int)p.Sk;
  const auto g_rs = make_buffer_rsrc(g_b, (uint32_t)((t_last - t0 + 1) * p.Sk * 4));
  auto load_tile = [&](int it, i32x4 (&r)[C::LOADS], f32x4 (&gr)[C::GQ_PER_T]) {
    const int64_t first = (int64_t)it * C::KT;
    const int64_t nkeys = p.Sk - first;
    const uint32_t nb = nkeys > 0 ? (uint32_t)((nkeys - 1) * row_pitch + C::ROWB) : 0u;
    const auto rs = make_buffer_rsrc(k_b + (nkeys > 0 ? first : 0) * row_pitch, nb);
#pragma unroll
    for (int l = 0; l < C::LOADS; ++l)
      r[l] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)loff[l], 0, 0));
    // G[token t0 + tl][keys first + 4c .. + 3]; keys past Sk are masked where G is used
#pragma unroll
    for (int l = 0; l < C::GQ_PER_T; ++l) {
      const int u = tid + C::NT * l;
      const int tl = u / (C::KT / 4), c = u % (C::KT / 4);
      const bool in = u < C::GQ_PIECES;
      const uint32_t off = in ? (uint32_t)(((int64_t)tl * p.Sk + first + 4 * c) * 4) : 0xffffffffu;
      if (p.gvec) {
        gr[l] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(g_rs, (int)off, 0, 0));
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) gr[l][j] = buffer_load_f32(g_rs, in ? (int)(off + 4 * j) : (int)0xffffffffu, 0);
      }
    }
  };
  auto store_tile = [&](int buf, const i32x4 (&r)[C::LOADS], const f32x4 (&gr)[C::GQ_PER_T]) {
#pragma unroll
    for (int l = 0; l < C::LOADS; ++l) {
      const int u = tid + C::NT * l;
      *reinterpret_cast<i32x4 *>(&KS[buf][(u / C::CPR) * C::STRIDE + (u % C::CPR) * 16]) = r[l];
    }
#pragma unroll
    for (int l = 0; l < C::GQ_PER_T; ++l) {
      const int u = tid + C::NT * l;
      if (u < C::GQ_PIECES) *reinterpret_cast<f32x4 *>(&GS[buf][4 * u]) = gr[l];
    }
  };
  i32x4 kreg[C::LOADS];
  f32x4 greg[C::GQ_PER_T];
  load_tile(it0, kreg, greg);

  // q rows of the wave as MFMA B operands (row = lane l32 of tile m; d = 16k + 8 g32 + e)
  bf16x8 QB[C::MT][C::KSTEPS];
  float wl[C::MT];
  int64_t tok[C::MT];
#pragma unroll
  for (int m = 0; m < C::MT; ++m) {
    const int64_t r = wave_row0 + m * 32 + l32;
    tok[m] = r / H;
    const bool ok = tok[m] < p.Sq;
    const int64_t qrow = (tok[m] * p.B + b) * H + r % H;
    wl[m] = ok ? ld_w(p, qrow) : 0.0f;
#pragma unroll
    for (int k = 0; k < C::KSTEPS; ++k) {
      i32x4 v = {0, 0, 0, 0};
      if (ok) v = ld_global_16(p.q + (qrow * D + 16 * k + 8 * g32) * 2);
      QB[m][k] = as_bf16x8(v);
    }
  }
  // keys klo[m] <= s < klim[m] are in the row's range (causal: s <= t; windows)
  int klim[C::MT], klo[C::MT];
  int wave_kbeg = 0;
#pragma unroll
  for (int m = 0; m < C::MT; ++m) {
    if constexpr (WIN) {
      int a = 0, e = 0;
      if (tok[m] < p.Sq) row_keys(p, b, tok[m], a, e);
      klo[m] = a;
      klim[m] = e;
    } else {
      klo[m] = 0;
      klim[m] = p.causal ? (tok[m] + 1 < p.Sk ? (int)tok[m] + 1 : sk32) : sk32;
    }
  }
  if constexpr (WIN) {
    // the union of the wave's row ranges (sub-tiles outside it are skipped) and
    // their intersection (sub-tiles inside it need no key test)
    int lo = 0x7fffffff, hi = 0, ilo = 0, ihi = 0x7fffffff;
#pragma unroll
    for (int m = 0; m < C::MT; ++m) {
      if (klim[m] > klo[m]) {
        lo = klo[m] < lo ? klo[m] : lo;
        hi = klim[m] > hi ? klim[m] : hi;
      }
      ilo = klo[m] > ilo ? klo[m] : ilo;
      ihi = klim[m] < ihi ? klim[m] : ihi;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const int lo2 = __shfl_xor(lo, off, 64), hi2 = __shfl_xor(hi, off, 64);
      const int ilo2 = __shfl_xor(ilo, off, 64), ihi2 = __shfl_xor(ihi, off, 64);
      lo = lo2 < lo ? lo2 : lo;
      hi = hi2 > hi ? hi2 : hi;
      ilo = ilo2 > ilo ? ilo2 : ilo;
      ihi = ihi2 < ihi ? ihi2 : ihi;
    }
    wave_kend = __builtin_amdgcn_readfirstlane(hi);
    wave_kbeg = hi > 0 ? __builtin_amdgcn_readfirstlane(lo) : 0;
    wave_klo = __builtin_amdgcn_readfirstlane(ilo);
    wave_khi = __builtin_amdgcn_readfirstlane(ihi);  // below wave_klo: no interior sub-tile
  }
  f32x16 dqa[C::MT][C::DT];
  float dwa[C::MT];
#pragma unroll
  for (int m = 0; m < C::MT; ++m) {
    dwa[m] = 0.0f;
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
      for (int a = 0; a < 16; ++a) dqa[m][dt][a] = 0.0f;
  }

  store_tile(0, kreg, greg);
  __syncthreads();
  for (int it = it0; it < ntile; ++it) {
    load_tile(it + 1, kreg, greg);  // past the last tile: zeros, unused
    const unsigned char *ks = KS[(it - it0) & 1];
    const float *gs = GS[(it - it0) & 1];
#pragma unroll 1
    for (int sub = 0; sub < C::SUBS; ++sub) {
      const int64_t sn = (int64_t)it * C::KT + sub * 32;
      if (sn >= wave_kend) break;  // wave-uniform
      if (WIN && sn + 32 <= wave_kbeg) continue;
      // G of the lane's row token at keys sn + 8i + 4 g32 + (0..3), from the staged tile
      f32x4 gv[C::MT][4];
#pragma unroll
      for (int m = 0; m < C::MT; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          gv[m][i] = *reinterpret_cast<const f32x4 *>(gs + (tok[m] - t0) * C::KT + sub * 32 + 8 * i + 4 * g32);
      // L^T[key][row] = K Q^T (M = key, N = row)
      f32x16 acc[C::MT];
#pragma unroll
      for (int m = 0; m < C::MT; ++m)
#pragma unroll
        for (int a = 0; a < 16; ++a) acc[m][a] = 0.0f;
#pragma unroll
      for (int k = 0; k < C::KSTEPS; ++k) {
        const i32x4 kr = *reinterpret_cast<const i32x4 *>(ks + (sub * 32 + l32) * C::STRIDE + (16 * k + 8 * g32) * 2);
#pragma unroll
        for (int m = 0; m < C::MT; ++m)
          acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(kr), QB[m][k], acc[m], 0, 0, 0);
      }
      // M = G act'(L) (0 off the causal window and past Sk), dw += M L; M -> bf16 B operands.
      // 32-bit keys and non-short-circuit predicates: one select per element, no branches.
      // A sub-tile inside every row range of the wave (the causal interior, or the
      // intersection of the row windows) needs no key test.
      const int s0 = (int)sn + 4 * g32;
      bf16x8 MB[C::MT][2];
      auto form_m = [&](auto interior) {
        constexpr bool IN = decltype(interior)::value;
#pragma unroll
        for (int m = 0; m < C::MT; ++m) {
          uint32_t mw[8];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float mv[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int s = s0 + 8 * i + j;
              const float L = acc[m][4 * i + j];
              const bool ok = (IN | ((s < klim[m]) & (!WIN | (s >= klo[m])))) & (!RELU | (L > 0.0f));
              const float v = ok ? gv[m][i][j] : 0.0f;
              dwa[m] = fmaf(v, L, dwa[m]);
              mv[j] = v;
            }
            mw[2 * i] = pack_bf16x2(mv[0], mv[1]);
            mw[2 * i + 1] = pack_bf16x2(mv[2], mv[3]);
          }
#pragma unroll
          for (int kc = 0; kc < 2; ++kc)
            MB[m][kc] = as_bf16x8(i32x4{(int)mw[4 * kc], (int)mw[4 * kc + 1], (int)mw[4 * kc + 2], (int)mw[4 * kc + 3]});
        }
      };
      if (sn >= wave_klo && sn + 32 <= wave_khi) form_m(std::true_type{});
      else form_m(std::false_type{});
      // dq^T[d][row] += K^T[d][key] M[key][row]: keys of k-step kc in the accumulator order
#pragma unroll
      for (int kc = 0; kc < 2; ++kc)
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) {
          const i32x4 av = tr_operand(ks, C::STRIDE, dt * 32, sub * 32 + 16 * kc, 8, 4);
#pragma unroll
          for (int m = 0; m < C::MT; ++m)
            dqa[m][dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(av), MB[m][kc], dqa[m][dt], 0, 0, 0);
        }
    }
    if (it + 1 < ntile) {
      // the buffer stored into was last read in iteration it - 1, before that iteration's barrier
      store_tile((it + 1 - it0) & 1, kreg, greg);
      __syncthreads();
    }
  }

  // dq = w * dq^T (lane: row l32 of tile m, d = dt*32 + 8i + 4 g32 + j), dw = both halves' sums
#pragma unroll
  for (int m = 0; m < C::MT; ++m) {
    const bool ok = tok[m] < p.Sq;
    const int64_t r = wave_row0 + m * 32 + l32;
    const int64_t qrow = (tok[m] * p.B + b) * H + r % H;
    const float dwv = sum_halves(dwa[m]);
    if (ok) {
      uint16_t *drow = p.dq + qrow * D;
#pragma unroll
      for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const f32x16 &a = dqa[m][dt];
          const i32x2 pk = {(int)pack_bf16x2(a[4 * i] * wl[m], a[4 * i + 1] * wl[m]),
                            (int)pack_bf16x2(a[4 * i + 2] * wl[m], a[4 * i + 3] * wl[m])};
          *reinterpret_cast<i32x2 *>(drow + dt * 32 + 8 * i + 4 * g32) = pk;
        }
      if (g32 == 0) {
        if (p.w_f32) static_cast<float *>(p.dw)[qrow] = dwv;
        else static_cast<uint16_t *>(p.dw)[qrow] = (uint16_t)f32_to_bf16_bits(dwv);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// dk: one workgroup per (key block of KB keys, token chunk, batch)
// ---------------------------------------------------------------------------
// First token chunk whose tokens can reach key block kb (causal); every chunk otherwise.
__device__ __forceinline__ int first_chunk(const IdxBwdParams &p, int64_t kb, int kbk) {
  if (!p.causal) return 0;
  const int64_t c = kb * kbk / p.tc;
  return (int)(c < p.nch ? c : p.nch);
}

// WIN: row windows (p.starts / p.ends).  The windowed kernel is its own
// instantiation, so the causal / full kernel's code is unchanged by them.  With
// windows, G is zeroed outside each token's window as the tile is staged in
// LDS (so the inner loop needs no window test), and a per-tile bitmask of the
// 32-row sub-tiles whose token windows meet each wave's keys, built with the
// tile, skips the others.
template <int H, int D, bool RELU, bool WIN>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
indexer_bwd_k_kernel(const IdxBwdParams p) {
  using C = IdxBwdCfg<H, D>;
  __shared__ __attribute__((aligned(16))) unsigned char QS[2][C::KT * C::STRIDE];
  __shared__ float WS[2][C::KT];
  __shared__ __attribute__((aligned(16))) float GSk[2][C::TPT * C::KB];
  constexpr int NSW = C::SUBS * C::WAVES;          // (sub-tile, wave) pairs of a row tile
  __shared__ int SKIPM[2][WIN ? NSW : 1];          // WIN: 1 where the sub-tile meets the wave's keys
  const int64_t kb = blockIdx.x, b = blockIdx.z;
  const int c = blockIdx.y;
  if (!WIN && c < first_chunk(p, kb, C::KB)) return;  // no token of the chunk reaches these keys
  const int tid = threadIdx.x, lane = lane_id(), w = __builtin_amdgcn_readfirstlane(wave_id());
  const int g32 = lane >> 5, l32 = lane & 31;
  const int64_t key0 = kb * C::KB + w * (C::MT * 32);  // this wave's first key
  const int64_t tc0 = (int64_t)c * p.tc;
  int64_t tc1 = (tc0 + p.tc < p.Sq ? tc0 + p.tc : p.Sq);
  // rows (token, head) of the chunk, from the first token that can reach this workgroup's keys
  int64_t tstart = tc0;
  if (!WIN && p.causal && kb * C::KB > tstart) tstart = kb * C::KB;
  const int kblk0i = (int)(kb * C::KB);
  if constexpr (WIN) {
    // the chunk's first and last token whose key range meets [kb * KB, kb * KB + KB)
    __shared__ int tr[2][C::WAVES];
    const int kb1 = kblk0i + C::KB;
    int tmin = 0x7fffffff, tmax = -1;
    for (int64_t t = tc0 + tid; t < tc1; t += C::NT) {
      int a, e;
      row_keys(p, b, t, a, e);
      if (e > a && a < kb1 && e > kblk0i) {
        tmin = (int)t < tmin ? (int)t : tmin;
        tmax = (int)t;
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const int a2 = __shfl_xor(tmin, off, 64), b2 = __shfl_xor(tmax, off, 64);
      tmin = a2 < tmin ? a2 : tmin;
      tmax = b2 > tmax ? b2 : tmax;
    }
    if (lane == 0) {
      tr[0][w] = tmin;
      tr[1][w] = tmax;
    }
    __syncthreads();
#pragma unroll
    for (int v = 0; v < C::WAVES; ++v) {
      tmin = tr[0][v] < tmin ? tr[0][v] : tmin;
      tmax = tr[1][v] > tmax ? tr[1][v] : tmax;
    }
    const int touched = tmax >= 0 ? 1 : 0;
    if (tid == 0) p.kflags[((b * p.nch + c) * p.nkb) + kb] = touched;
    if (!touched) return;  // block-uniform
    tstart = tmin;
    tc1 = (int64_t)tmax + 1;
  }
  const int64_t row0 = tstart * H, row1 = tc1 * H;
  const int ntile = row1 > row0 ? (int)((row1 - row0 + C::KT - 1) / C::KT) : 0;

  // the wave's keys as MFMA B operands (key = n*32 + l32, d = 16k + 8 g32 + e)
  bf16x8 KBr[C::MT][C::KSTEPS];
#pragma unroll
  for (int n = 0; n < C::MT; ++n) {
    const int64_t key = key0 + n * 32 + l32;
#pragma unroll
    for (int k = 0; k < C::KSTEPS; ++k) {
      i32x4 v = {0, 0, 0, 0};
      if (key < p.Sk) v = ld_global_16(p.k + ((key * p.B + b) * D + 16 * k + 8 * g32) * 2);
      KBr[n][k] = as_bf16x8(v);
    }
  }
  // q rows r (global row index over (token, head) = t * H + h) of batch b: q[(t*B + b)*H + h]
  auto qaddr = [&](int64_t r) { return p.q + (((r / H) * p.B + b) * H + r % H) * (int64_t)C::ROWB; };
  // G of batch b through one resource (past it: zeros); a row tile's tokens x this workgroup's keys
  const float *g_b = p.g + b * p.Sq * p.Sk;
  const auto g_rs = make_buffer_rsrc(g_b, (uint32_t)(p.Sq * p.Sk * 4));
  const int64_t kblk0 = kb * C::KB;
  auto load_tile = [&](int it, i32x4 (&r)[C::LOADS], float &wv, f32x4 (&gr)[C::GK_PER_T], int &meets) {
#pragma unroll
    for (int l = 0; l < C::LOADS; ++l) {
      const int u = tid + C::NT * l;
      const int64_t row = row0 + (int64_t)it * C::KT + u / C::CPR;
      r[l] = row < row1 ? ld_global_16(qaddr(row) + (u % C::CPR) * 16) : i32x4{0, 0, 0, 0};
    }
    const int64_t row = row0 + (int64_t)it * C::KT + tid;
    wv = (tid < C::KT && row < row1) ? ld_w(p, ((row / H) * p.B + b) * H + row % H) : 0.0f;
    const int64_t tok0 = (row0 + (int64_t)it * C::KT) / H;  // the tile's first token
#pragma unroll
    for (int l = 0; l < C::GK_PER_T; ++l) {
      const int u = tid + C::NT * l;
      const int tl = u / (C::KB / 4), c = u % (C::KB / 4);
      const bool in = u < C::GK_PIECES;
      const uint32_t off = in ? (uint32_t)(((tok0 + tl) * p.Sk + kblk0 + 4 * c) * 4) : 0xffffffffu;
      if (p.gvec) {
        gr[l] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(g_rs, (int)off, 0, 0));
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) gr[l][j] = buffer_load_f32(g_rs, in ? (int)(off + 4 * j) : (int)0xffffffffu, 0);
      }
      if constexpr (WIN) {  // G outside the token's window carries no gradient
        int a = 0, e = 0;
        if (in && tok0 + tl < tc1) row_keys(p, b, tok0 + tl, a, e);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int key = kblk0i + 4 * c + j;
          gr[l][j] = (key >= a && key < e) ? gr[l][j] : 0.0f;
        }
      }
    }
    meets = 0;
    if constexpr (WIN) {  // (sub-tile rs, wave v) = tid: does a token window of rows rs*32.. meet v's keys
      if (tid < NSW) {
        const int rs = tid / C::WAVES, v = tid % C::WAVES;
        const int64_t k0v = kblk0 + v * (C::MT * 32);
        constexpr int TPS = 32 / H > 0 ? 32 / H : 1;
#pragma unroll
        for (int ti = 0; ti < TPS; ++ti) {
          const int64_t t = (row0 + (int64_t)it * C::KT + rs * 32) / H + ti;
          int a = 0, e = 0;
          if (t < tc1) row_keys(p, b, t, a, e);
          meets |= (e > a && a < k0v + C::MT * 32 && e > k0v) ? 1 : 0;
        }
      }
    }
  };
  auto store_tile = [&](int buf, const i32x4 (&r)[C::LOADS], float wv, const f32x4 (&gr)[C::GK_PER_T], int meets) {
#pragma unroll
    for (int l = 0; l < C::LOADS; ++l) {
      const int u = tid + C::NT * l;
      *reinterpret_cast<i32x4 *>(&QS[buf][(u / C::CPR) * C::STRIDE + (u % C::CPR) * 16]) = r[l];
    }
    if (tid < C::KT) WS[buf][tid] = wv;
    if constexpr (WIN) {
      if (tid < NSW) SKIPM[buf][tid] = meets;
    }
#pragma unroll
    for (int l = 0; l < C::GK_PER_T; ++l) {
      const int u = tid + C::NT * l;
      if (u < C::GK_PIECES) *reinterpret_cast<f32x4 *>(&GSk[buf][4 * u]) = gr[l];
    }
  };

  f32x16 dka[C::MT][C::DT];
#pragma unroll
  for (int n = 0; n < C::MT; ++n)
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
      for (int a = 0; a < 16; ++a) dka[n][dt][a] = 0.0f;

  i32x4 qreg[C::LOADS];
  float wreg = 0.0f;
  f32x4 greg[C::GK_PER_T];
  int mreg = 0;
  if (ntile > 0) {
    load_tile(0, qreg, wreg, greg, mreg);
    store_tile(0, qreg, wreg, greg, mreg);
  }
  __syncthreads();
  for (int it = 0; it < ntile; ++it) {
    if (it + 1 < ntile) load_tile(it + 1, qreg, wreg, greg, mreg);
    const unsigned char *qs = QS[it & 1];
    const float *ws = WS[it & 1];
    const float *gsk = GSk[it & 1];
    // WIN: this wave's sub-tiles that meet its keys, one scalar bitmask per tile
    uint32_t subm = 0xffffffffu;
    if constexpr (WIN) {
      subm = 0;
#pragma unroll
      for (int rs = 0; rs < C::SUBS; ++rs)
        subm |= (uint32_t)__builtin_amdgcn_readfirstlane(SKIPM[it & 1][rs * C::WAVES + w]) << rs;
    }
#pragma unroll 1
    for (int rs = 0; rs < C::SUBS; ++rs) {
      const int64_t rb = row0 + (int64_t)it * C::KT + rs * 32;  // first row of the sub-tile
      if (rb >= row1) break;
      // the sub-tile's last token is below this wave's first key: nothing (causal)
      if (!WIN && p.causal && (rb + 31) / H < key0) continue;
      if (WIN && ((subm >> rs) & 1u) == 0) continue;  // no token window meets this wave's keys
      // G[t][key] for the (at most two) tokens of rows rb .. rb + 31
      constexpr int TPS = 32 / H > 0 ? 32 / H : 1;  // tokens per 32-row sub-tile
      float gv[C::MT][TPS];
#pragma unroll
      for (int n = 0; n < C::MT; ++n)
#pragma unroll
        for (int ti = 0; ti < TPS; ++ti) {
          const int lt = (rs * 32) / H + ti;  // token within the row tile
          const int64_t key = key0 + n * 32 + l32;
          const float gsv = gsk[lt * C::KB + (int)(key - kblk0)];
          gv[n][ti] = key < p.Sk ? gsv : 0.0f;
        }
      // L[row][key] = Q K^T (M = row, N = key)
      f32x16 acc[C::MT];
#pragma unroll
      for (int n = 0; n < C::MT; ++n)
#pragma unroll
        for (int a = 0; a < 16; ++a) acc[n][a] = 0.0f;
#pragma unroll
      for (int k = 0; k < C::KSTEPS; ++k) {
        const i32x4 qr = *reinterpret_cast<const i32x4 *>(qs + (rs * 32 + l32) * C::STRIDE + (16 * k + 8 * g32) * 2);
#pragma unroll
        for (int n = 0; n < C::MT; ++n)
          acc[n] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(qr), KBr[n][k], acc[n], 0, 0, 0);
      }
      // M[row][key] = G w act'(L), rows 8i + 4 g32 + j of the sub-tile
      f32x4 wv4[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) wv4[i] = *reinterpret_cast<const f32x4 *>(ws + rs * 32 + 8 * i + 4 * g32);
      // rows 8i + 4 g32 + j of the sub-tile belong to token rb / H + (H == 16 ? i / 2 : 0):
      // a sub-tile starts on a 32-row boundary (row0 is a multiple of 32 rows)
      const int tb = (int)(rb / H);
      bf16x8 MB[C::MT][2];
#pragma unroll
      for (int n = 0; n < C::MT; ++n) {
        const int key = (int)(key0 + n * 32 + l32);
        uint32_t mw[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int ti = H == 16 ? (i >> 1) : 0;
          const bool in_win = WIN | !p.causal | (key <= tb + ti);  // WIN: G is already 0 outside
          const float gw = gv[n][ti];
          float mv[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float L = acc[n][4 * i + j];
            const bool ok = in_win & (!RELU | (L > 0.0f));
            mv[j] = ok ? gw * wv4[i][j] : 0.0f;
          }
          mw[2 * i] = pack_bf16x2(mv[0], mv[1]);
          mw[2 * i + 1] = pack_bf16x2(mv[2], mv[3]);
        }
#pragma unroll
        for (int kc = 0; kc < 2; ++kc)
          MB[n][kc] = as_bf16x8(i32x4{(int)mw[4 * kc], (int)mw[4 * kc + 1], (int)mw[4 * kc + 2], (int)mw[4 * kc + 3]});
      }
      // dk^T[d][key] += Q^T[d][row] M[row][key]: rows of k-step kc in the accumulator order
#pragma unroll
      for (int kc = 0; kc < 2; ++kc)
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) {
          const i32x4 av = tr_operand(qs, C::STRIDE, dt * 32, rs * 32 + 16 * kc, 8, 4);
#pragma unroll
          for (int n = 0; n < C::MT; ++n)
            dka[n][dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(av), MB[n][kc], dka[n][dt], 0, 0, 0);
        }
    }
    if (it + 1 < ntile) {
      store_tile((it + 1) & 1, qreg, wreg, greg, mreg);
      __syncthreads();
    }
  }
  // partial dk of (chunk c): lane = key n*32 + l32, d = dt*32 + 8i + 4 g32 + (0..3)
  float *part = p.dk_part + ((b * p.nch + c) * p.Sk) * D;
#pragma unroll
  for (int n = 0; n < C::MT; ++n) {
    const int64_t key = key0 + n * 32 + l32;
    if (key >= p.Sk) continue;
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *reinterpret_cast<f32x4 *>(part + key * D + dt * 32 + 8 * i + 4 * g32) =
            f32x4{dka[n][dt][4 * i], dka[n][dt][4 * i + 1], dka[n][dt][4 * i + 2], dka[n][dt][4 * i + 3]};
  }
}

// dk[s, b, :] = bf16(sum over the chunks that reached key s, in chunk order)
template <int D, int KBK>
__global__ void __launch_bounds__(256) indexer_bwd_dk_reduce_kernel(const IdxBwdParams p) {
  const int64_t e = blockIdx.x * 256ll + threadIdx.x;  // (b, s, d) with d fastest
  if (e >= p.B * p.Sk * D) return;
  const int64_t d = e % D, s = (e / D) % p.Sk, b = e / (D * p.Sk);
  float acc = 0.0f;
  if (p.kflags != nullptr) {  // windows: the chunks that wrote a partial for this key block
    // D is a multiple of 64, so a wave's 64 consecutive elements share one
    // (batch, key): the flags are wave-uniform scalar loads
    static_assert(D % 64 == 0, "a wave's elements share one key");
    const int64_t kblk = __builtin_amdgcn_readfirstlane((int)(s / KBK));
    const int64_t bb = __builtin_amdgcn_readfirstlane((int)b);
    const int32_t *fl = p.kflags + bb * p.nch * p.nkb + kblk;
    for (int c = 0; c < p.nch; ++c)
      if (fl[c * p.nkb]) acc += p.dk_part[((b * p.nch + c) * p.Sk + s) * D + d];
  } else {
    const int c0 = first_chunk(p, s / KBK, KBK);
    for (int c = c0; c < p.nch; ++c) acc += p.dk_part[((b * p.nch + c) * p.Sk + s) * D + d];
  }
  p.dk[(s * p.B + b) * D + d] = (uint16_t)f32_to_bf16_bits(acc);
}

// Token chunks of the key-major kernel: chunks of >= 128 tokens, at most 32 of
// them (the fp32 dk partials are nch x the size of dk).
static void bwd_chunks(int64_t Sq, int *nch, int *tc) {
  int n = (int)((Sq + 127) / 128);
  if (n > 32) n = 32;
  if (n < 1) n = 1;
  int64_t len = (Sq + n - 1) / n;
  len = (len + 15) / 16 * 16;
  *nch = (int)((Sq + len - 1) / len);
  if (*nch < 1) *nch = 1;
  *tc = (int)len;
}

template <int H, int D, bool RELU>
static int launch_idx_bwd(IdxBwdParams p, hipStream_t st) {
  using C = IdxBwdCfg<H, D>;
  const int64_t ntb = (p.Sq + C::TT - 1) / C::TT;
  DSA_REQUIRE(ntb * p.B < (1ll << 31), "dsa_indexer_scores_backward: grid too large");
  const int64_t nkb = (p.Sk + C::KB - 1) / C::KB;
  p.nkb = (int)nkb;
  if (p.ends != nullptr)
    hipLaunchKernelGGL((indexer_bwd_q_kernel<H, D, RELU, true>), dim3((unsigned)(ntb * p.B)), dim3(C::NT), 0, st, p);
  else
    hipLaunchKernelGGL((indexer_bwd_q_kernel<H, D, RELU, false>), dim3((unsigned)(ntb * p.B)), dim3(C::NT), 0, st, p);
  int rc = check_launch("indexer_scores_backward(dq)");
  if (rc) return rc;
  if (p.ends != nullptr)
    hipLaunchKernelGGL((indexer_bwd_k_kernel<H, D, RELU, true>), dim3((unsigned)nkb, (unsigned)p.nch, (unsigned)p.B),
                       dim3(C::NT), 0, st, p);
  else
    hipLaunchKernelGGL((indexer_bwd_k_kernel<H, D, RELU, false>), dim3((unsigned)nkb, (unsigned)p.nch, (unsigned)p.B),
                       dim3(C::NT), 0, st, p);
  rc = check_launch("indexer_scores_backward(dk)");
  if (rc) return rc;
  const int64_t n = p.B * p.Sk * D;
  hipLaunchKernelGGL((indexer_bwd_dk_reduce_kernel<D, C::KB>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                     p);
  return check_launch("indexer_scores_backward(dk reduce)");
}

template <int H, int D>
static int launch_idx_bwd_act(const IdxBwdParams &p, bool relu, hipStream_t st) {
  return relu ? launch_idx_bwd<H, D, true>(p, st) : launch_idx_bwd<H, D, false>(p, st);
}

}  // namespace dsa

using namespace dsa;

extern "C" size_t dsa_indexer_scores_backward_workspace_size(int64_t B, int64_t Sq, int64_t Sk, int64_t H,
                                                             int64_t D) {
  (void)H;
  if (B <= 0 || Sq <= 0 || Sk <= 0 || D <= 0) return 0;
  int nch = 1, tc = 1;
  bwd_chunks(Sq, &nch, &tc);
  // fp32 dk partials per token chunk, then the windows' per-(chunk, key block)
  // flags (key blocks of at least 128 keys)
  const size_t part = ((size_t)B * nch * Sk * D * sizeof(float) + 255) & ~(size_t)255;
  return part + (size_t)B * nch * ((Sk + 127) / 128) * sizeof(int32_t);
}

extern "C" int dsa_indexer_scores_backward(const float *grad_scores, const void *q, const void *w, const void *k,
                                           void *dq, void *dw, void *dk, int64_t B, int64_t Sq, int64_t Sk,
                                           int64_t H, int64_t D, int dtype, int w_dtype, int causal, int use_relu,
                                           const int32_t *starts, const int32_t *ends, void *workspace,
                                           size_t workspace_bytes, void *stream) {
  DSA_REQUIRE(B >= 0 && Sq >= 0 && Sk >= 0 && H > 0 && D > 0, "dsa_indexer_scores_backward: bad dims");
  DSA_REQUIRE(dtype == DSA_DTYPE_BF16, "dsa_indexer_scores_backward: q / k must be bf16 (dtype %d)", dtype);
  DSA_REQUIRE(w_dtype == DSA_DTYPE_BF16 || w_dtype == DSA_DTYPE_F32, "dsa_indexer_scores_backward: w dtype %d",
              w_dtype);
  DSA_REQUIRE(causal == 0 || causal == 1, "dsa_indexer_scores_backward: causal must be 0 or 1");
  DSA_REQUIRE((starts == nullptr) == (ends == nullptr), "dsa_indexer_scores_backward: give both starts and ends");
  if (B == 0 || Sq == 0 || Sk == 0) return DSA_OK;
  DSA_REQUIRE(grad_scores && q && w && k && dq && dw && dk, "dsa_indexer_scores_backward: null tensor pointer");
  DSA_REQUIRE(Sq * Sk < (1ll << 30) && Sk < (1ll << 25) && B < 65536,
              "dsa_indexer_scores_backward: %lld x %lld scores too large for 32-bit offsets", (long long)Sq,
              (long long)Sk);
  const size_t need = dsa_indexer_scores_backward_workspace_size(B, Sq, Sk, H, D);
  if (!workspace || workspace_bytes < need)
    return set_error(DSA_ERR_WORKSPACE, "dsa_indexer_scores_backward: workspace %zu < required %zu", workspace_bytes,
                     need);
  IdxBwdParams p;
  p.g = grad_scores;
  p.q = static_cast<const unsigned char *>(q);
  p.w = w;
  p.k = static_cast<const unsigned char *>(k);
  p.dq = static_cast<uint16_t *>(dq);
  p.dw = dw;
  p.dk_part = static_cast<float *>(workspace);
  p.dk = static_cast<uint16_t *>(dk);
  p.B = B;
  p.Sq = Sq;
  p.Sk = Sk;
  p.w_f32 = w_dtype == DSA_DTYPE_F32;
  p.causal = causal;
  p.gvec = (Sk % 4 == 0) && (reinterpret_cast<uintptr_t>(grad_scores) & 15u) == 0;
  bwd_chunks(Sq, &p.nch, &p.tc);
  p.starts = starts;
  p.ends = ends;
  p.kflags = starts ? reinterpret_cast<int32_t *>(static_cast<unsigned char *>(workspace) +
                                                  (((size_t)B * p.nch * Sk * D * sizeof(float) + 255) & ~(size_t)255))
                    : nullptr;
  p.nkb = 0;  // set per kernel configuration by the launcher
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool relu = use_relu != 0;
#define DSA_IDXB_CASE(HH, DD) \
  if (H == HH && D == DD) return launch_idx_bwd_act<HH, DD>(p, relu, st);
  DSA_IDXB_CASE(16, 64)
  DSA_IDXB_CASE(32, 64)
  DSA_IDXB_CASE(64, 64)
  DSA_IDXB_CASE(16, 128)
  DSA_IDXB_CASE(32, 128)
  DSA_IDXB_CASE(64, 128)
#undef DSA_IDXB_CASE
  return set_error(DSA_ERR_UNSUPPORTED, "dsa_indexer_scores_backward: no kernel for h=%lld d=%lld", (long long)H,
                   (long long)D);
}
