// DSA indexer KL loss on gfx950: the KL divergence between the head-averaged
// causal attention distribution and the indexer's softmax, without ever
// materialising the [b, np, sq, sk] attention probabilities.
//
// Reference: compute_dsa_indexer_loss_splitk
// (cppmega/megatron/dsa_splitk_indexer_loss.py:328-468), a two-stage Triton
// kernel (stage 1 :57-186 accumulates per-head softmax statistics, stage 2
// :194-322 recomputes q.k, averages the normalised probabilities over heads
// and reduces the KL per position), checked by its test against a clone of
// Megatron's compute_dsa_indexer_loss (tests/test_dsa_splitk_indexer_loss.py:29-83):
//
//   a_h[t, s] = scale * query[t, h] . key[s, h]  (+ sparse top-k mask) (s <= t)
//   P[t, s]   = mean_h softmax_s a_h[t, :]
//   Q[t, s]   = softmax_s (index_scores[t, :] + sparse top-k mask) over all s
//   loss      = coeff * mean_t sum_s P (ln(P + 1e-10) - ln(Q + 1e-10))
//
// Five stream-ordered kernels, all deterministic (no atomics outside LDS):
//  1. kl_index_stats_kernel  one wave per (b, t): the log2 normaliser
//     gamma = max + log2(sum exp2(x - max)) of x = index_scores * log2(e) over
//     the row (sparse: over the row's top-k set, built as a bitmask in LDS and
//     written out for the other kernels);
//  2. kl_attn_stats_kernel   per (b, head, pair of 256-token blocks): the log2
//     normaliser beta_h[t] of c * q.k (c = scale * log2(e)) over s <= t, on
//     MFMA 32x32x16 bf16 with S^T = K . Q^T (keys on M, tokens on N, so a lane
//     holds 16 keys of one token and row reductions stay in-lane); key chunks
//     are double-buffered in LDS and shared by the 8 waves; a long and a short
//     token block share one workgroup so every workgroup does equal work;
//  3. kl_pass_kernel         per (b, 128-token block, key chunk): for every head
//     recompute c * q.k, accumulate exp2(c * q.k - beta_h) in registers (the
//     head sum of P), then form the KL terms of the chunk against
//     Q = exp2(index * log2(e) - gamma) and write one partial sum per token;
//  4. kl_rows_kernel         row loss = sum of its chunk partials in chunk order
//     (NaN when the row has no admissible attention column or a NaN index
//     normaliser, as the reference's softmax gives);
//  5. kl_mean_kernel         one workgroup: coeff * mean of the row losses in a
//     fixed summation order.
//
// Gradient with respect to index_scores (dsa_indexer_kl_loss_backward; the
// loss's only path back to the indexer, which Megatron obtains by autograd
// through compute_dsa_indexer_loss).  With Q = softmax(z) over the row's
// columns and P the detached target,
//   dL/dz_s = g * coeff / (B * Sq) * (Q_s * R - P_s * Q_s / (Q_s + 1e-10)),
//   R       = sum_j P_j * Q_j / (Q_j + 1e-10)
// (0 where Q_s = 0: -inf scores and, sparse, columns outside the top-k set;
// NaN over a row whose loss is NaN).  Kernels 1-3 run as above, except that
// the pass kernel writes P into the gradient buffer (s <= t) and one partial
// R per key chunk instead of the KL terms; then
//  6. kl_grad_kernel         one workgroup per row: R in chunk order, then the
//     whole row of the gradient in place over P (16-byte loads and stores).
#include "dsa_common.hpp"

namespace dsa {
namespace kl {

constexpr int kNT = 256;      // threads per workgroup of the small kernels
constexpr int kMaxW = 1024;   // mask words per row in LDS (sparse: Sk <= 32768)
constexpr float kLn2 = 0.69314718055994531f;
constexpr float kEps = 1e-10f;

template <int D, int NW>
struct Cfg {
  static constexpr int NT = 64 * NW;               // threads per workgroup
  static constexpr int TB = 32 * NW;               // tokens per workgroup (32 per wave)
  static constexpr int KC = D <= 128 ? 128 : 64;   // keys per LDS chunk
  static constexpr int ROWB = D * 2;               // bytes per bf16 key row
  static constexpr int STRIDE = ROWB + 16;         // LDS row pitch (bank spread)
  static constexpr int SUBS = KC / 32;             // 32-key sub-tiles per chunk
  static constexpr int KSTEPS = D / 16;            // MFMA k-steps per q.k
  static constexpr int CPR = ROWB / 16;            // 16-byte pieces per key row
  static constexpr int LOADS = KC * CPR / NT;      // 16-byte loads per thread per chunk
  static_assert(D % 32 == 0 && D <= 256 && KC * CPR % NT == 0, "head dim");
};

struct Params {
  const float *index_scores;      // [B, Sq, Sk]
  const void *topk;               // [B, Sq, K] int32 or int64 (sparse only)
  const unsigned char *query;     // [Sq, B, H, D] bf16
  const unsigned char *key;       // [Sk, B, G, D] bf16
  uint32_t *mask;                 // [B, Sq, W]   top-k bitmask (sparse only)
  float *gamma;                   // [B, Sq]      index normaliser (log2 units)
  float *beta;                    // [B, H, Sq]   attention normaliser (log2 units)
  float *partial;                 // [B, NC, Sq]  KL partial sums per key chunk
  float *rows;                    // [B, Sq]      per-position KL
  float *loss;                    // [1]
  float *partial_r;               // [B, NC, Sq]  gradient: R partial sums per key chunk
  float *grad;                    // [B, Sq, Sk]  gradient: P (pass kernel), then dL/dz
  const float *grad_loss;         // [1]          upstream gradient of the loss
  int64_t B, Sq, Sk, H, G, K, W, NC;
  int64_t NI;                     // KL work items per batch (block, chunk pairs)
  int topk_i64;
  int sparse;
  float c;                        // softmax_scale * log2(e)
  float coeff;
};

// Online log2-sum-exp2 pair: (m, d) represents d * 2^m.  m starts at the
// finite kNegBig so that merging two empty pairs never forms inf - inf.
__device__ __forceinline__ void lse_merge(float &m, float &d, float mo, float dd) {
  const float nm = fmaxf(m, mo);
  d = d * exp2_fast(m - nm) + dd * exp2_fast(mo - nm);
  m = nm;
}

// ---------------------------------------------------------------------------
// 1. index normaliser (and the sparse top-k bitmask)
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(kNT) kl_index_stats_kernel(Params p) {
  __shared__ uint32_t bits[4][kMaxW];
  const int w = wave_id(), lane = lane_id();
  const int64_t row = (int64_t)blockIdx.x * 4 + w;  // b * Sq + t
  if (row >= p.B * p.Sq) return;                      // wave-uniform
  const float *I = p.index_scores + row * p.Sk;
  float m = kNegBig, d = 0.0f;
  if (p.sparse) {
    uint32_t *bw = bits[w];
    for (int i = lane; i < p.W; i += 64) bw[i] = 0u;
    wave_lds_sync();
    for (int64_t j = lane; j < p.K; j += 64) {
      const int64_t s = p.topk_i64 ? static_cast<const int64_t *>(p.topk)[row * p.K + j]
                                   : (int64_t) static_cast<const int32_t *>(p.topk)[row * p.K + j];
      if (s >= 0 && s < p.Sk) atomicOr(&bw[s >> 5], 1u << (s & 31));
    }
    wave_lds_sync();
    for (int i = lane; i < p.W; i += 64) {
      uint32_t word = bw[i];
      p.mask[row * p.W + i] = word;
      while (word) {  // each set column once (duplicates in the top-k list count once)
        const int bpos = __builtin_ctz(word);
        word &= word - 1u;
        lse_merge(m, d, I[i * 32 + bpos] * kLog2e, 1.0f);
      }
    }
  } else {
    const uint32_t nbytes = (uint32_t)(p.Sk * 4);
    const auto rs = make_buffer_rsrc(I, nbytes);
    const bool vec = (p.Sk & 3) == 0;  // 16-byte aligned rows
    for (int64_t s0 = 4 * lane; s0 < p.Sk; s0 += 256) {
      f32x4 v;
      if (vec) {
        v = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(s0 * 4), 0, 0));
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = buffer_load_f32(rs, (int)((s0 + j) * 4), 0);
      }
      float x[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) x[j] = s0 + j < p.Sk ? v[j] * kLog2e : -INFINITY;
      const float nm = fmaxf(m, fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])));
      d = d * exp2_fast(m - nm) + exp2_fast(x[0] - nm) + exp2_fast(x[1] - nm) + exp2_fast(x[2] - nm) +
          exp2_fast(x[3] - nm);
      m = nm;
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float mo = __shfl_xor(m, off, 64), dd = __shfl_xor(d, off, 64);
    lse_merge(m, d, mo, dd);
  }
  // no finite-weight column (all -inf, or an empty top-k set): the reference's
  // softmax is NaN; an inf or NaN score makes d NaN, which propagates
  if (lane == 0) p.gamma[row] = d > 0.0f ? m + __builtin_amdgcn_logf(d) : __builtin_nanf("");
}

// ---------------------------------------------------------------------------
// Shared pieces of the two MFMA kernels
// ---------------------------------------------------------------------------
// B operand (q^T, N = token) of head h for token t: lane half g holds
// elements 16k + 8g .. +8 of the row at k-step k (zero past Sq).
template <int D>
__device__ __forceinline__ void load_q_operand(const Params &p, int64_t b, int64_t h, int64_t t,
                                               bf16x8 (&Q)[Cfg<D, 4>::KSTEPS]) {
  const int g = lane_id() >> 5;
  const bool ok = t < p.Sq;
  const unsigned char *row = p.query + (((ok ? t : 0) * p.B + b) * p.H + h) * (int64_t)(D * 2);
#pragma unroll
  for (int k = 0; k < Cfg<D, 4>::KSTEPS; ++k) {
    i32x4 v = {0, 0, 0, 0};
    if (ok) v = ld_global_16(row + (16 * k + 8 * g) * 2);
    Q[k] = as_bf16x8(v);
  }
}

// Cooperative loads of key chunk [k0, k0 + KC) of (b, group grp) into
// registers; rows at or past Sk read zeros (bounded buffer resource).
template <int D, int NW>
struct ChunkLoader {
  using C = Cfg<D, NW>;
  uint32_t off[C::LOADS];
  uint32_t pitch;
  __device__ ChunkLoader(const Params &p) {
    pitch = (uint32_t)(p.B * p.G * C::ROWB);
#pragma unroll
    for (int l = 0; l < C::LOADS; ++l) {
      const int u = threadIdx.x + C::NT * l;
      off[l] = (uint32_t)(u / C::CPR) * pitch + (uint32_t)(u % C::CPR) * 16u;
    }
  }
  __device__ void load(const Params &p, int64_t b, int64_t grp, int64_t k0, i32x4 (&r)[C::LOADS]) const {
    const int64_t nkeys = p.Sk - k0;
    const uint32_t nb = nkeys > 0 ? (uint32_t)((nkeys - 1) * pitch + C::ROWB) : 0u;
    const unsigned char *base = p.key + ((nkeys > 0 ? k0 : 0) * p.B + b) * p.G * C::ROWB + grp * C::ROWB;
    const auto rs = make_buffer_rsrc(base, nb);
#pragma unroll
    for (int l = 0; l < C::LOADS; ++l)
      r[l] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)off[l], 0, 0));
  }
  __device__ static void store(unsigned char *ks, const i32x4 (&r)[C::LOADS]) {
#pragma unroll
    for (int l = 0; l < C::LOADS; ++l) {
      const int u = threadIdx.x + C::NT * l;
      *reinterpret_cast<i32x4 *>(ks + (u / C::CPR) * C::STRIDE + (u % C::CPR) * 16) = r[l];
    }
  }
};

// S^T of sub-tile `sub` (32 keys) of the LDS chunk against the wave's 32
// tokens: acc[4i + j] = q(token lane & 31) . k(key 32 sub + 8i + 4g + j).
template <int D>
__device__ __forceinline__ f32x16 qk_subtile(const unsigned char *ks, int sub, const bf16x8 (&Q)[Cfg<D, 4>::KSTEPS]) {
  using C = Cfg<D, 4>;
  const int lane = lane_id();
  const unsigned char *arow = ks + (sub * 32 + (lane & 31)) * C::STRIDE + (lane >> 5) * 16;
  f32x16 acc;
#pragma unroll
  for (int a = 0; a < 16; ++a) acc[a] = 0.0f;
#pragma unroll
  for (int k = 0; k < C::KSTEPS; ++k) {
    const i32x4 av = *reinterpret_cast<const i32x4 *>(arow + 32 * k);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(av), Q[k], acc, 0, 0, 0);
  }
  return acc;
}

// Top-k bitmask word of token t covering keys [key0, key0 + 32) (key0 a
// multiple of 32); all ones in dense mode.
__device__ __forceinline__ uint32_t mask_word(const Params &p, int64_t b, int64_t t, int64_t key0) {
  if (!p.sparse) return 0xffffffffu;
  return t < p.Sq ? p.mask[(b * p.Sq + t) * p.W + (key0 >> 5)] : 0u;
}

// Admissible-column bits of accumulator register a = 4i + j (key
// key0 + 8i + 4g + j) for token t: s <= t, s < Sk, t < Sq and, sparse, in the
// top-k set (bit of `word`).  Word-level: clear the bits past the last
// admissible key, then gather the lane half's four 4-bit groups.
__device__ __forceinline__ uint32_t valid_bits(const Params &p, uint32_t word, int64_t t, int64_t key0) {
  const int g = lane_id() >> 5;
  const int64_t last = (t < p.Sk - 1 ? t : p.Sk - 1) - key0;  // last admissible m
  const uint32_t keep = t >= p.Sq || last < 0 ? 0u : (last >= 31 ? 0xffffffffu : (2u << last) - 1u);
  const uint32_t w = (word & keep) >> (4 * g);
  return (w & 0xfu) | ((w >> 4) & 0xf0u) | ((w >> 8) & 0xf00u) | ((w >> 12) & 0xf000u);
}

// acc if bit a of vb is set, -inf otherwise (sign-extended bit field as a
// select mask: one bfe + one bfi).
__device__ __forceinline__ float keep_or_neginf(float acc, uint32_t vb, int a) {
  const uint32_t m = (uint32_t)(((int32_t)(vb << (31 - a))) >> 31);
  return __uint_as_float((m & __float_as_uint(acc)) | (~m & 0xff800000u));
}

// Chunks of KC keys that token block blk (TB tokens) needs: keys up to
// min(last token of the block, Sk - 1).
__device__ __forceinline__ int64_t block_chunks(const Params &p, int64_t blk, int64_t TB, int64_t KC) {
  const int64_t lt = (TB * (blk + 1) < p.Sq ? TB * (blk + 1) : p.Sq) - 1;
  return (lt < p.Sk - 1 ? lt : p.Sk - 1) / KC + 1;
}

// ---------------------------------------------------------------------------
// 2. attention normalisers beta_h[t] (log2 units of c * q.k)
// ---------------------------------------------------------------------------
template <int D, int NW>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(NW == 8 ? 4 : 2)))
kl_attn_stats_kernel(Params p) {
  using C = Cfg<D, NW>;
  constexpr int kTB = C::TB;
  __shared__ __attribute__((aligned(16))) unsigned char KS[2][C::KC * C::STRIDE];
  const int w = wave_id(), lane = lane_id(), g = lane >> 5;
  const int64_t NB = (p.Sq + kTB - 1) / kTB, NP = (NB + 1) / 2;
  const int64_t bid = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t pair = bid % NP, bh = bid / NP, h = bh % p.H, b = bh / p.H;
  const int64_t grp = h / (p.H / p.G);
  ChunkLoader<D, NW> ld(p);

  for (int half = 0; half < 2; ++half) {
    const int64_t blk = half == 0 ? NB - 1 - pair : pair;  // the long block first
    if (half == 1 && blk == NB - 1 - pair) break;          // odd NB: middle block once
    const int64_t t0 = blk * kTB, wt0 = t0 + 32 * w, t = wt0 + (lane & 31);
    const int64_t wt_last = wt0 + 31;
    const int64_t kend = p.Sk < t0 + kTB ? p.Sk : t0 + kTB;  // keys s <= last token of the block
    const int nch = (int)((kend + C::KC - 1) / C::KC);
    bf16x8 Q[C::KSTEPS];
    load_q_operand<D>(p, b, h, t, Q);
    float m = kNegBig, d = 0.0f;
    i32x4 kr[C::LOADS];
    __syncthreads();  // the previous block's waves are done with the LDS chunks
    ld.load(p, b, grp, 0, kr);
    ChunkLoader<D, NW>::store(KS[0], kr);
    __syncthreads();
    // sparse: the chunk's top-k mask words are loaded one chunk ahead
    uint32_t mw[C::SUBS];
#pragma unroll
    for (int sub = 0; sub < C::SUBS; ++sub) mw[sub] = mask_word(p, b, t, 32 * sub);
    for (int ci = 0; ci < nch; ++ci) {
      if (ci + 1 < nch) ld.load(p, b, grp, (int64_t)(ci + 1) * C::KC, kr);
      uint32_t mwn[C::SUBS];
#pragma unroll
      for (int sub = 0; sub < C::SUBS; ++sub)
        mwn[sub] = ci + 1 < nch ? mask_word(p, b, t, (int64_t)(ci + 1) * C::KC + 32 * sub) : 0u;
      const unsigned char *ks = KS[ci & 1];
#pragma unroll
      for (int sub = 0; sub < C::SUBS; ++sub) {
        const int64_t key0 = (int64_t)ci * C::KC + 32 * sub;
        if (key0 > wt_last || key0 >= p.Sk) continue;  // wave-uniform: wholly above the diagonal
        const f32x16 acc = qk_subtile<D>(ks, sub, Q);
        const bool need_mask = p.sparse || key0 + 31 > wt0 || key0 + 31 >= p.Sk || wt_last >= p.Sq;
        // c > 0: max(c * acc) = c * max(acc), and exp2(c * acc - nm) is one fma
        float x[16];
        if (need_mask) {
          const uint32_t vb = valid_bits(p, mw[sub], t, key0);
#pragma unroll
          for (int a = 0; a < 16; ++a) x[a] = keep_or_neginf(acc[a], vb, a);
        } else {
#pragma unroll
          for (int a = 0; a < 16; ++a) x[a] = acc[a];
        }
        float lm = x[0];
#pragma unroll
        for (int a = 1; a < 16; ++a) lm = fmaxf(lm, x[a]);
        const float nm = fmaxf(m, lm * p.c);
        float s = 0.0f;
#pragma unroll
        for (int a = 0; a < 16; ++a) s += exp2_fast(fmaf(x[a], p.c, -nm));
        d = d * exp2_fast(m - nm) + s;
        m = nm;
      }
#pragma unroll
      for (int sub = 0; sub < C::SUBS; ++sub) mw[sub] = mwn[sub];
      if (ci + 1 < nch) {
        ChunkLoader<D, NW>::store(KS[(ci + 1) & 1], kr);
        __syncthreads();
      }
    }
    // the two lane halves hold the same token's other keys
    const float mo = __shfl_xor(m, 32, 64), dd = __shfl_xor(d, 32, 64);
    lse_merge(m, d, mo, dd);
    if (g == 0 && t < p.Sq)
      p.beta[(b * p.H + h) * p.Sq + t] = d > 0.0f ? m + __builtin_amdgcn_logf(d) : -INFINITY;
  }
}

// ---------------------------------------------------------------------------
// 3. KL partial sums per (token, key chunk)
// ---------------------------------------------------------------------------
template <int D, int NW, bool GRAD = false>
__global__ void __launch_bounds__(64 * NW) kl_pass_kernel(Params p) {
  using C = Cfg<D, NW>;
  constexpr int kTB = C::TB;
  __shared__ __attribute__((aligned(16))) unsigned char KS[2][C::KC * C::STRIDE];
  const int w = wave_id(), lane = lane_id(), g = lane >> 5;
  // Work items are the (b, block, chunk) pairs at or below the diagonal:
  // first every block's full chunks, block-major, then the cheaper diagonal
  // chunks (one per block), so a last partial round of the grid is short
  // work.  The grid is padded to a multiple of 8 so that each XCD takes one
  // contiguous, equal share (consecutive items share a token block's q rows
  // in that XCD's L2).
  const int64_t NB = (p.Sq + kTB - 1) / kTB;
  const int64_t bid = xcd_remap(blockIdx.x, gridDim.x);
  if (bid >= p.B * p.NI) return;
  const int64_t nfull = p.NI - NB;  // items per batch before the diagonal ones
  int64_t b, blk = 0, ci;
  if (bid < p.B * nfull) {
    b = bid / nfull;
    int64_t rem = bid % nfull;
    for (;; ++blk) {  // scalar walk over the blocks' full-chunk counts (NB steps at most)
      const int64_t n = block_chunks(p, blk, kTB, C::KC) - 1;
      if (rem < n) break;
      rem -= n;
    }
    ci = rem;
  } else {
    const int64_t r = bid - p.B * nfull;
    b = r / NB;
    blk = r % NB;
    ci = block_chunks(p, blk, kTB, C::KC) - 1;
  }
  const int64_t t0 = blk * kTB, k0 = ci * C::KC;
  const int64_t wt0 = t0 + 32 * w, t = wt0 + (lane & 31), wt_last = wt0 + 31;
  const int64_t hpg = p.H / p.G;
  ChunkLoader<D, NW> ld(p);

  // admissible bits of this lane's 16 keys per sub-tile (same for every head)
  uint32_t vb[C::SUBS];
  bool sub_on[C::SUBS];
#pragma unroll
  for (int sub = 0; sub < C::SUBS; ++sub) {
    const int64_t key0 = k0 + 32 * sub;
    sub_on[sub] = key0 <= wt_last && key0 < p.Sk && wt0 < p.Sq;  // wave-uniform
    vb[sub] = sub_on[sub] ? valid_bits(p, mask_word(p, b, t, key0), t, key0) : 0u;
  }

  float P[C::SUBS][16];
#pragma unroll
  for (int sub = 0; sub < C::SUBS; ++sub)
#pragma unroll
    for (int a = 0; a < 16; ++a) P[sub][a] = 0.0f;

  i32x4 kr[C::LOADS];
  ld.load(p, b, 0, k0, kr);
  ChunkLoader<D, NW>::store(KS[0], kr);
  __syncthreads();
  // the next head's q operand and normaliser are loaded one head ahead
  const float *beta_bt = p.beta + b * p.H * p.Sq + (t < p.Sq ? t : 0);
  bf16x8 Qn[C::KSTEPS];
  load_q_operand<D>(p, b, 0, t, Qn);
  float bn = beta_bt[0];
  for (int64_t h = 0; h < p.H; ++h) {
    const int64_t grp = h / hpg;
    const bool last_of_grp = h % hpg == hpg - 1;
    if (h % hpg == 0 && grp + 1 < p.G) ld.load(p, b, grp + 1, k0, kr);
    bf16x8 Q[C::KSTEPS];
#pragma unroll
    for (int k = 0; k < C::KSTEPS; ++k) Q[k] = Qn[k];
    const float bh = bn;
    if (h + 1 < p.H) {
      load_q_operand<D>(p, b, h + 1, t, Qn);
      bn = beta_bt[(h + 1) * p.Sq];
    }
    const unsigned char *ks = KS[grp & 1];
#pragma unroll
    for (int sub = 0; sub < C::SUBS; ++sub) {
      if (!sub_on[sub]) continue;
      const f32x16 acc = qk_subtile<D>(ks, sub, Q);
#pragma unroll
      for (int a = 0; a < 16; ++a) P[sub][a] += exp2_fast(fmaf(acc[a], p.c, -bh));
    }
    if (last_of_grp && grp + 1 < p.G) {
      // the other buffer was last read for group grp - 1, before the previous barrier
      ChunkLoader<D, NW>::store(KS[(grp + 1) & 1], kr);
      __syncthreads();
    }
  }

  // KL terms of the chunk: P = (head sum) / H on admissible columns, 0 elsewhere
  const float inv_h = 1.0f / (float)p.H;
  const float gam = t < p.Sq ? p.gamma[b * p.Sq + t] : 0.0f;
  const float *irow = p.index_scores + b * p.Sq * p.Sk;
  const auto irs = make_buffer_rsrc(irow, (uint32_t)(p.Sq * p.Sk * 4));
  const bool vec = (p.Sk & 3) == 0;  // rows 16-byte aligned: one b128 load per 4 keys
  float kl = 0.0f;
  float *grow = GRAD ? p.grad + (b * p.Sq + (t < p.Sq ? t : 0)) * p.Sk : nullptr;
#pragma unroll
  for (int sub = 0; sub < C::SUBS; ++sub) {
    if (!sub_on[sub]) continue;
    const int64_t key0 = k0 + 32 * sub;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // keys key0 + 8i + 4g + (0..3) of this lane's row; reads past the row
      // (or past Sq) only feed inadmissible columns
      const int64_t s0 = key0 + 8 * i + 4 * g;
      f32x4 iv;
      if (vec) {
        const uint32_t off = t < p.Sq ? (uint32_t)((t * p.Sk + s0) * 4) : 0xfffffff0u;
        iv = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(irs, (int)off, 0, 0));
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int64_t s = s0 + j;
          const uint32_t off = (t < p.Sq && s < p.Sk) ? (uint32_t)((t * p.Sk + s) * 4) : 0xfffffff0u;
          iv[j] = buffer_load_f32(irs, (int)off, 0);
        }
      }
      if constexpr (GRAD) {
        // P on this lane's four keys (0 off the admissible set), and R's terms
        f32x4 pv;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int a = 4 * i + j;
          const bool on = (vb[sub] >> a) & 1u;
          const float pr = on ? P[sub][a] * inv_h : 0.0f;
          const float q = exp2_fast(fmaf(iv[j], kLog2e, -gam));
          pv[j] = pr;
          if (on) kl += pr * (q / (q + kEps));
        }
        if (t < p.Sq && s0 < p.Sk) {
          if (vec) {
            *reinterpret_cast<f32x4 *>(grow + s0) = pv;
          } else {
#pragma unroll
            for (int j = 0; j < 4; ++j)
              if (s0 + j < p.Sk) grow[s0 + j] = pv[j];
          }
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int a = 4 * i + j;
          if ((vb[sub] >> a) & 1u) {
            const float pr = P[sub][a] * inv_h;
            const float q = exp2_fast(fmaf(iv[j], kLog2e, -gam));
            kl += pr * (__builtin_amdgcn_logf(pr + kEps) - __builtin_amdgcn_logf(q + kEps));
          }
        }
      }
    }
  }
  if constexpr (GRAD) {
    kl = sum_halves(kl);
    if (g == 0 && t < p.Sq) p.partial_r[(b * p.NC + ci) * p.Sq + t] = kl;
  } else {
    kl = sum_halves(kl) * kLn2;
    if (g == 0 && t < p.Sq) p.partial[(b * p.NC + ci) * p.Sq + t] = kl;
  }
}

// ---------------------------------------------------------------------------
// 4. row losses, 5. mean
// ---------------------------------------------------------------------------
template <int D>
__global__ void __launch_bounds__(kNT) kl_rows_kernel(Params p) {
  const int64_t row = (int64_t)blockIdx.x * kNT + threadIdx.x;
  if (row >= p.B * p.Sq) return;
  const int64_t b = row / p.Sq, t = row % p.Sq;
  const int64_t last_k = t < p.Sk - 1 ? t : p.Sk - 1;
  const int64_t cmax = last_k / Cfg<D, 4>::KC;
  float s = 0.0f;
  for (int64_t c = 0; c <= cmax; ++c) s += p.partial[(b * p.NC + c) * p.Sq + t];
  const bool no_target = !(p.beta[b * p.H * p.Sq + t] > -INFINITY);
  const float gam = p.gamma[row];
  if (no_target || gam != gam) s = __builtin_nanf("");
  p.rows[row] = s;
}

// 6. gradient row: dL/dz over P in place (one workgroup per (b, t) row)
template <int D>
__global__ void __launch_bounds__(kNT) kl_grad_kernel(Params p) {
  const int64_t row = blockIdx.x;
  const int64_t b = row / p.Sq, t = row % p.Sq;
  const int64_t last_k = t < p.Sk - 1 ? t : p.Sk - 1;  // P is written for s <= last_k
  const int64_t cmax = last_k / Cfg<D, 4>::KC;
  float R = 0.0f;
  for (int64_t c = 0; c <= cmax; ++c) R += p.partial_r[(b * p.NC + c) * p.Sq + t];
  const bool no_target = !(p.beta[b * p.H * p.Sq + t] > -INFINITY);
  const float gam = p.gamma[row];
  const bool nan_row = no_target || gam != gam;
  const float gs = p.grad_loss[0] * p.coeff / (float)(p.B * p.Sq);
  const float *zrow = p.index_scores + row * p.Sk;
  float *grow = p.grad + row * p.Sk;
  const uint32_t *mrow = p.sparse ? p.mask + row * p.W : nullptr;
  const bool vec = (p.Sk & 3) == 0;
  for (int64_t s0 = 4 * (int64_t)threadIdx.x; s0 < p.Sk; s0 += 4 * kNT) {
    f32x4 z, pr, out;
    if (vec) {
      z = *reinterpret_cast<const f32x4 *>(zrow + s0);
      pr = s0 <= last_k ? *reinterpret_cast<const f32x4 *>(grow + s0) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        z[j] = s0 + j < p.Sk ? zrow[s0 + j] : 0.0f;
        pr[j] = s0 + j <= last_k ? grow[s0 + j] : 0.0f;
      }
    }
    const uint32_t mw = mrow ? mrow[s0 >> 5] >> (s0 & 31) : 0xfu;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float q = ((mw >> j) & 1u) ? exp2_fast(fmaf(z[j], kLog2e, -gam)) : 0.0f;
      const float pj = s0 + j <= last_k ? pr[j] : 0.0f;
      out[j] = nan_row ? __builtin_nanf("") : gs * (q * R - pj * (q / (q + kEps)));
    }
    if (vec) {
      *reinterpret_cast<f32x4 *>(grow + s0) = out;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (s0 + j < p.Sk) grow[s0 + j] = out[j];
    }
  }
}

__global__ void __launch_bounds__(1024) kl_mean_kernel(Params p) {
  __shared__ float red[1024];
  const int64_t n = p.B * p.Sq;
  float s = 0.0f;
  for (int64_t i = threadIdx.x; i < n; i += 1024) s += p.rows[i];
  red[threadIdx.x] = s;
  __syncthreads();
  for (int off = 512; off >= 1; off >>= 1) {
    if ((int)threadIdx.x < off) red[threadIdx.x] += red[threadIdx.x + off];
    __syncthreads();
  }
  if (threadIdx.x == 0) p.loss[0] = red[0] / (float)n * p.coeff;
}

// ---------------------------------------------------------------------------
// host
// ---------------------------------------------------------------------------
struct Layout {
  size_t mask, gamma, beta, partial, rows, partial_r, total;
};

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static Layout layout(int64_t B, int64_t Sq, int64_t Sk, int64_t H, int64_t D, int sparse) {
  const int64_t KC = D <= 128 ? 128 : 64;
  const int64_t W = (Sk + 31) / 32, NC = (Sk + KC - 1) / KC;
  Layout L;
  size_t o = 0;
  L.mask = o;    o += align256(sparse ? (size_t)(B * Sq * W) * 4 : 0);
  L.gamma = o;   o += align256((size_t)(B * Sq) * 4);
  L.beta = o;    o += align256((size_t)(B * H * Sq) * 4);
  L.partial = o; o += align256((size_t)(B * NC * Sq) * 4);
  L.rows = o;    o += align256((size_t)(B * Sq) * 4);
  L.partial_r = o; o += align256((size_t)(B * NC * Sq) * 4);
  L.total = o;
  return L;
}

template <int D, int NWS, int NWP, bool GRAD>
static int launch_mfma(const Params &p, hipStream_t st) {
  using CS = Cfg<D, NWS>;
  using CP = Cfg<D, NWP>;
  const int64_t NBS = (p.Sq + CS::TB - 1) / CS::TB, NP = (NBS + 1) / 2;
  hipLaunchKernelGGL((kl_attn_stats_kernel<D, NWS>), dim3((unsigned)(p.B * p.H * NP)), dim3(CS::NT), 0, st, p);
  int rc = check_launch("kl_attn_stats_kernel");
  if (rc) return rc;
  const int64_t NBP = (p.Sq + CP::TB - 1) / CP::TB;
  Params q = p;
  q.NI = 0;
  for (int64_t j = 0; j < NBP; ++j) {
    const int64_t lt = (CP::TB * (j + 1) < p.Sq ? CP::TB * (j + 1) : p.Sq) - 1;
    q.NI += (lt < p.Sk - 1 ? lt : p.Sk - 1) / CP::KC + 1;
  }
  const int64_t items = (p.B * q.NI + 7) / 8 * 8;
  hipLaunchKernelGGL((kl_pass_kernel<D, NWP, GRAD>), dim3((unsigned)items), dim3(CP::NT), 0, st, q);
  rc = check_launch("kl_pass_kernel");
  if (rc) return rc;
  if constexpr (GRAD) {
    hipLaunchKernelGGL(kl_grad_kernel<D>, dim3((unsigned)(p.B * p.Sq)), dim3(kNT), 0, st, p);
    return check_launch("kl_grad_kernel");
  }
  hipLaunchKernelGGL(kl_rows_kernel<D>, dim3((unsigned)((p.B * p.Sq + kNT - 1) / kNT)), dim3(kNT), 0, st, p);
  return check_launch("kl_rows_kernel");
}

// Checks and Params shared by the loss and its gradient (kernels 1-3).
static int kl_setup(const char *fn, const float *index_scores, const void *topk_indices, int topk_dtype,
                    int64_t topk, const void *query, const void *key, int64_t B, int64_t Sq, int64_t Sk,
                    int64_t H, int64_t G, int64_t D, float softmax_scale, float loss_coeff, int sparse,
                    void *workspace, size_t workspace_bytes, Params &p) {
  DSA_REQUIRE(index_scores && query && key, "%s: null pointer", fn);
  DSA_REQUIRE(B > 0 && Sq > 0 && Sk > 0 && H > 0 && G > 0, "%s: empty shape B=%lld Sq=%lld Sk=%lld H=%lld G=%lld",
              fn, (long long)B, (long long)Sq, (long long)Sk, (long long)H, (long long)G);
  DSA_REQUIRE(H % G == 0, "%s: H=%lld is not a multiple of the key heads G=%lld", fn, (long long)H, (long long)G);
  DSA_REQUIRE(softmax_scale > 0.0f && softmax_scale < INFINITY, "%s: softmax_scale %g must be positive", fn,
              (double)softmax_scale);
  DSA_REQUIRE(D == 64 || D == 128 || D == 192 || D == 256, "%s: head dim %lld not in {64,128,192,256}", fn,
              (long long)D);
  DSA_REQUIRE(B * Sq * Sk < ((int64_t)1 << 29), "%s: B*Sq*Sk=%lld index scores exceed 2 GiB", fn,
              (long long)(B * Sq * Sk));
  DSA_REQUIRE(Sk * B * G * D * 2 < ((int64_t)1 << 31), "%s: key tensor exceeds 2 GiB", fn);
  if (sparse) {
    DSA_REQUIRE(topk_indices && topk > 0, "%s: sparse mode needs top-k indices", fn);
    DSA_REQUIRE(topk_dtype == DSA_DTYPE_I32 || topk_dtype == DSA_DTYPE_I64, "%s: top-k dtype %d is not int32/int64",
                fn, topk_dtype);
    DSA_REQUIRE(Sk <= 32 * kMaxW, "%s: sparse mode supports Sk <= %d (got %lld)", fn, 32 * kMaxW, (long long)Sk);
  }
  const Layout L = layout(B, Sq, Sk, H, D, sparse);
  if (!workspace || workspace_bytes < L.total)
    return set_error(DSA_ERR_WORKSPACE, "%s: workspace %zu bytes < %zu required", fn,
                     workspace ? workspace_bytes : (size_t)0, L.total);
  unsigned char *ws = static_cast<unsigned char *>(workspace);
  p = Params{};
  p.index_scores = index_scores;
  p.topk = topk_indices;
  p.query = static_cast<const unsigned char *>(query);
  p.key = static_cast<const unsigned char *>(key);
  p.mask = reinterpret_cast<uint32_t *>(ws + L.mask);
  p.gamma = reinterpret_cast<float *>(ws + L.gamma);
  p.beta = reinterpret_cast<float *>(ws + L.beta);
  p.partial = reinterpret_cast<float *>(ws + L.partial);
  p.rows = reinterpret_cast<float *>(ws + L.rows);
  p.partial_r = reinterpret_cast<float *>(ws + L.partial_r);
  p.B = B; p.Sq = Sq; p.Sk = Sk; p.H = H; p.G = G; p.K = sparse ? topk : 0;
  p.W = (Sk + 31) / 32;
  p.NC = (Sk + (D <= 128 ? 128 : 64) - 1) / (D <= 128 ? 128 : 64);
  p.topk_i64 = topk_dtype == DSA_DTYPE_I64;
  p.sparse = sparse ? 1 : 0;
  p.c = softmax_scale * kLog2e;
  p.coeff = loss_coeff;
  return DSA_OK;
}

template <bool GRAD>
static int kl_launch(const Params &p, int64_t D, hipStream_t st) {
  hipLaunchKernelGGL(kl_index_stats_kernel, dim3((unsigned)((p.B * p.Sq + 3) / 4)), dim3(kNT), 0, st, p);
  int rc = check_launch("kl_index_stats_kernel");
  if (rc) return rc;
  switch (D) {
    case 64: return launch_mfma<64, 8, 4, GRAD>(p, st);
    case 128: return launch_mfma<128, 8, 4, GRAD>(p, st);
    case 192: return launch_mfma<192, 8, 4, GRAD>(p, st);
    default: return launch_mfma<256, 8, 4, GRAD>(p, st);
  }
}

}  // namespace kl
}  // namespace dsa

extern "C" size_t dsa_indexer_kl_loss_workspace_size(int64_t B, int64_t Sq, int64_t Sk, int64_t H, int64_t D,
                                                      int sparse) {
  if (B <= 0 || Sq <= 0 || Sk <= 0 || H <= 0 || D <= 0) return 0;
  return dsa::kl::layout(B, Sq, Sk, H, D, sparse).total;
}

extern "C" int dsa_indexer_kl_loss(const float *index_scores, const void *topk_indices, int topk_dtype,
                                   int64_t topk, const void *query, const void *key, float *loss,
                                   float *row_loss, int64_t B, int64_t Sq, int64_t Sk, int64_t H, int64_t G,
                                   int64_t D, float softmax_scale, float loss_coeff, int sparse,
                                   void *workspace, size_t workspace_bytes, void *stream) {
  using namespace dsa;
  using namespace dsa::kl;
  DSA_REQUIRE(loss, "dsa_indexer_kl_loss: null loss pointer");
  Params p;
  int rc = kl_setup("dsa_indexer_kl_loss", index_scores, topk_indices, topk_dtype, topk, query, key, B, Sq, Sk, H, G,
                    D, softmax_scale, loss_coeff, sparse, workspace, workspace_bytes, p);
  if (rc) return rc;
  if (row_loss) p.rows = row_loss;
  p.loss = loss;
  hipStream_t st = static_cast<hipStream_t>(stream);
  rc = kl_launch<false>(p, D, st);
  if (rc) return rc;
  hipLaunchKernelGGL(kl_mean_kernel, dim3(1), dim3(1024), 0, st, p);
  return check_launch("kl_mean_kernel");
}

extern "C" int dsa_indexer_kl_loss_backward(const float *index_scores, const void *topk_indices, int topk_dtype,
                                            int64_t topk, const void *query, const void *key,
                                            const float *grad_loss, float *grad_index_scores, int64_t B, int64_t Sq,
                                            int64_t Sk, int64_t H, int64_t G, int64_t D, float softmax_scale,
                                            float loss_coeff, int sparse, void *workspace, size_t workspace_bytes,
                                            void *stream) {
  using namespace dsa;
  using namespace dsa::kl;
  DSA_REQUIRE(grad_loss && grad_index_scores, "dsa_indexer_kl_loss_backward: null gradient pointer");
  DSA_REQUIRE(grad_index_scores != index_scores, "dsa_indexer_kl_loss_backward: the gradient may not overwrite the scores");
  Params p;
  int rc = kl_setup("dsa_indexer_kl_loss_backward", index_scores, topk_indices, topk_dtype, topk, query, key, B, Sq,
                    Sk, H, G, D, softmax_scale, loss_coeff, sparse, workspace, workspace_bytes, p);
  if (rc) return rc;
  p.grad = grad_index_scores;
  p.grad_loss = grad_loss;
  return kl_launch<true>(p, D, static_cast<hipStream_t>(stream));
}
