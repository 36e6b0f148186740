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
// Tile: one workgroup = 256 (token, head) rows x 128 keys; each wave owns 64
// rows (2 M-subtiles, A operands in registers) and reads the key tile (B
// operands) from LDS.  Causal: tiles whose first key lies beyond their last
// token do no MFMA work (mode 1 fills -inf, mode 2 skips them).
#include <type_traits>

#include "dsa_common.hpp"

namespace dsa {

struct IdxParams {
  const unsigned char *q;
  const void *w;
  const unsigned char *k;
  float *out;
  const float *q_scale;
  const float *k_scale;
  int64_t B, Sq, Sk;
  int w_f32;
  int causal;
  int relu;
};

template <int H, int D, bool FP8>
struct IdxCfg {
  static constexpr int ELT = FP8 ? 1 : 2;
  static constexpr int ROWS = 256;
  static constexpr int TT = ROWS / H;       // tokens per workgroup
  static constexpr int TPW = 64 / H;        // tokens per wave
  static constexpr int TN = 128;            // keys per workgroup
  static constexpr int KS_STRIDE = D * ELT + 16;
  static constexpr int KSTEPS = D / 16;
  static_assert(H == 16 || H == 32 || H == 64, "index heads must be 16, 32 or 64");
  static_assert(D % 16 == 0 && D * ELT % 16 == 0, "index head dim");
};

template <int H, int D, bool FP8>
__global__ void __launch_bounds__(256) indexer_score_kernel(const IdxParams p) {
  using C = IdxCfg<H, D, FP8>;
  __shared__ __attribute__((aligned(16))) unsigned char KS[C::TN * C::KS_STRIDE];
  const int tid = threadIdx.x, lane = lane_id(), w = wave_id();
  const int g32 = lane >> 5, l32 = lane & 31;
  const int64_t b = blockIdx.z;
  const int64_t t0 = (int64_t)blockIdx.y * C::TT;
  const int64_t s0 = (int64_t)blockIdx.x * C::TN;
  const int64_t t_last = (t0 + C::TT < p.Sq ? t0 + C::TT : p.Sq) - 1;
  float *out_b = p.out + b * p.Sq * p.Sk;

  if (p.causal && s0 > t_last) {
    if (p.causal == 1) {
      for (int i = tid; i < C::TT * C::TN; i += 256) {
        const int64_t t = t0 + i / C::TN, s = s0 + i % C::TN;
        if (t < p.Sq && s < p.Sk) out_b[t * p.Sk + s] = -INFINITY;
      }
    }
    return;
  }

  // ---- stage the key tile: KS[key][d] ----
  constexpr int CPR = D * C::ELT / 16;  // 16-byte chunks per key row
  for (int i = tid; i < C::TN * CPR; i += 256) {
    const int key = i / CPR, c = i % CPR;
    const int64_t s = s0 + key;
    i32x4 v = {0, 0, 0, 0};
    if (s < p.Sk) v = ld_global_16(p.k + ((s * p.B + b) * D) * C::ELT + c * 16);
    *reinterpret_cast<i32x4 *>(KS + key * C::KS_STRIDE + c * 16) = v;
  }

  // ---- A operands (q rows) and per-row weights ----
  typedef typename std::conditional<FP8, long, bf16x8>::type aop_t;
  aop_t A[2][C::KSTEPS];
  float wv[2][16];
  const int64_t wave_tok0 = t0 + w * C::TPW;
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    const int r = m * 32 + l32;  // A-operand row of this lane
    const int64_t t = wave_tok0 + r / H;
    const int h = r % H;
    const bool ok = t < p.Sq;
    const int64_t qrow = (t * p.B + b) * H + h;
#pragma unroll
    for (int k = 0; k < C::KSTEPS; ++k) {
      if constexpr (FP8) {
        A[m][k] = ok ? *reinterpret_cast<const long *>(p.q + qrow * D + 16 * k + 8 * g32) : 0l;
      } else {
        i32x4 v = {0, 0, 0, 0};
        if (ok) v = ld_global_16(p.q + (qrow * D + 16 * k + 8 * g32) * 2);
        A[m][k] = as_bf16x8(v);
      }
    }
#pragma unroll
    for (int a = 0; a < 16; ++a) {
      const int rr = m * 32 + 8 * (a >> 2) + 4 * g32 + (a & 3);  // accumulator row
      const int64_t tt = wave_tok0 + rr / H;
      const int hh = rr % H;
      float wval = 0.0f;
      if (tt < p.Sq) {
        const int64_t wi = (tt * p.B + b) * H + hh;
        wval = p.w_f32 ? static_cast<const float *>(p.w)[wi]
                       : bf16_bits_to_f32(static_cast<const uint16_t *>(p.w)[wi]);
      }
      wv[m][a] = wval;
    }
  }
  float qk = 1.0f;
  if constexpr (FP8) qk = p.q_scale[0] * p.k_scale[0];
  __syncthreads();

  const int64_t wave_tok_last = wave_tok0 + C::TPW - 1;
#pragma unroll 1
  for (int n = 0; n < C::TN / 32; ++n) {
    const int64_t sn = s0 + n * 32;
    if (sn >= p.Sk) break;
    const int64_t s = sn + l32;
    if (p.causal && sn > wave_tok_last) {
      if (p.causal == 1) {
#pragma unroll
        for (int tl = 0; tl < C::TPW; ++tl) {
          const int64_t t = wave_tok0 + tl;
          if ((tl & 1) == g32 && t < p.Sq && s < p.Sk) out_b[t * p.Sk + s] = -INFINITY;
        }
      }
      continue;
    }
    float part[C::TPW];
#pragma unroll
    for (int tl = 0; tl < C::TPW; ++tl) part[tl] = 0.0f;
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      f32x16 acc;
#pragma unroll
      for (int a = 0; a < 16; ++a) acc[a] = 0.0f;
#pragma unroll
      for (int k = 0; k < C::KSTEPS; ++k) {
        if constexpr (FP8) {
          const long bv = *reinterpret_cast<const long *>(KS + (n * 32 + l32) * C::KS_STRIDE + 16 * k + 8 * g32);
          acc = __builtin_amdgcn_mfma_f32_32x32x16_fp8_fp8(A[m][k], bv, acc, 0, 0, 0);
        } else {
          const i32x4 bv = *reinterpret_cast<const i32x4 *>(KS + (n * 32 + l32) * C::KS_STRIDE + (16 * k + 8 * g32) * 2);
          acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[m][k], as_bf16x8(bv), acc, 0, 0, 0);
        }
      }
#pragma unroll
      for (int a = 0; a < 16; ++a) {
        const int tl = (m * 32 + 8 * (a >> 2)) / H;
        float x = acc[a];
        if constexpr (FP8) x *= qk;
        if (p.relu) x = fmaxf(x, 0.0f);
        part[tl] += x * wv[m][a];
      }
    }
#pragma unroll
    for (int tl = 0; tl < C::TPW; ++tl) part[tl] += xor32(part[tl]);
#pragma unroll
    for (int tl = 0; tl < C::TPW; ++tl) {
      const bool mine = C::TPW == 1 ? (g32 == 0) : ((tl & 1) == g32);
      const int64_t t = wave_tok0 + tl;
      if (mine && t < p.Sq && s < p.Sk) {
        if (p.causal && s > t) {
          if (p.causal == 1) out_b[t * p.Sk + s] = -INFINITY;
        } else {
          out_b[t * p.Sk + s] = part[tl];
        }
      }
    }
  }
}

template <int H, int D, bool FP8>
static int launch_idx(const IdxParams &p, hipStream_t st) {
  using C = IdxCfg<H, D, FP8>;
  const dim3 grid((unsigned)((p.Sk + C::TN - 1) / C::TN), (unsigned)((p.Sq + C::TT - 1) / C::TT), (unsigned)p.B);
  hipLaunchKernelGGL((indexer_score_kernel<H, D, FP8>), grid, dim3(256), 0, st, p);
  return check_launch("indexer_scores");
}

}  // namespace dsa

using namespace dsa;

extern "C" int dsa_indexer_scores(const void *q, const void *w, const void *k, float *scores, int64_t B,
                                  int64_t Sq, int64_t Sk, int64_t H, int64_t D, int dtype, int w_dtype,
                                  const float *q_scale, const float *k_scale, int causal, int use_relu,
                                  void *stream) {
  DSA_REQUIRE(B >= 0 && Sq >= 0 && Sk >= 0 && H > 0 && D > 0, "dsa_indexer_scores: bad dims");
  DSA_REQUIRE(dtype == DSA_DTYPE_BF16 || dtype == DSA_DTYPE_E4M3, "dsa_indexer_scores: dtype %d", dtype);
  DSA_REQUIRE(w_dtype == DSA_DTYPE_BF16 || w_dtype == DSA_DTYPE_F32, "dsa_indexer_scores: w dtype %d", w_dtype);
  DSA_REQUIRE(causal >= 0 && causal <= 2, "dsa_indexer_scores: causal must be 0, 1 or 2");
  if (B == 0 || Sq == 0 || Sk == 0) return DSA_OK;
  DSA_REQUIRE(q && w && k && scores, "dsa_indexer_scores: null tensor pointer");
  DSA_REQUIRE(Sk < (1ll << 31) && (Sq + 255) / 16 < 65536 && B < 65536, "dsa_indexer_scores: grid too large");
  const bool f8 = dtype == DSA_DTYPE_E4M3;
  if (f8) DSA_REQUIRE(q_scale && k_scale, "dsa_indexer_scores: e4m3 input needs q_scale and k_scale");
  IdxParams p;
  p.q = static_cast<const unsigned char *>(q);
  p.w = w;
  p.k = static_cast<const unsigned char *>(k);
  p.out = scores;
  p.q_scale = q_scale;
  p.k_scale = k_scale;
  p.B = B;
  p.Sq = Sq;
  p.Sk = Sk;
  p.w_f32 = w_dtype == DSA_DTYPE_F32;
  p.causal = causal;
  p.relu = use_relu != 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
#define DSA_IDX_CASE(HH, DD)                                                              \
  if (H == HH && D == DD) return f8 ? launch_idx<HH, DD, true>(p, st) : launch_idx<HH, DD, false>(p, st);
  DSA_IDX_CASE(16, 64)
  DSA_IDX_CASE(32, 64)
  DSA_IDX_CASE(64, 64)
  DSA_IDX_CASE(16, 128)
  DSA_IDX_CASE(32, 128)
  DSA_IDX_CASE(64, 128)
#undef DSA_IDX_CASE
  return set_error(DSA_ERR_UNSUPPORTED, "dsa_indexer_scores: no kernel for h=%lld d=%lld", (long long)H,
                   (long long)D);
}
