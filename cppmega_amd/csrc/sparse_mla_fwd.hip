// SparseMLA forward for gfx950 (bf16 and OCP-e4m3 tensorwise).
//
// Reference semantics: cppmega/megatron/sparse_mla_ops/tilelang_sparse_mla_fwd.py:137-290
// (bf16) and tilelang_sparse_mla_fwd_fp8.py:187-393 (fp8).  For every query
// token the selected latent-KV rows are gathered, S = scale * Q K^T is formed
// over d_qk, an online exp2 softmax runs over the slots, P is rounded to bf16
// and O = P V is accumulated in fp32 over the d_v prefix; LSE is emitted in
// log2 units.
//
// Work decomposition (one workgroup = 256 threads = 4 waves per token and kv
// group): heads are processed in tiles of 32 (the N dimension of a
// 32x32x16 MFMA).  With one head tile the 4 waves split the top-k slots
// between them (flash-decoding inside the workgroup) and merge their
// (max, sum, O) states through LDS at the end; with more tiles the waves take
// different tiles.  Each wave walks its slots in blocks of 32:
//   1. gather: 16-byte row-chunk loads (16 lanes cover one 256-byte row) of
//      the 32 selected rows into a per-wave LDS tile, K row-major and the
//      V prefix transposed (Vt[d][slot]) so both MFMA operands read 16 or 8
//      contiguous bytes per lane;
//   2. S^T[slot][head] = K Q^T with Q held in registers as the B operand;
//      the accumulator gives each lane one head and 16 slots, so the softmax
//      row reduction is 15 in-lane ops plus one cross-half exchange;
//   3. P (fp32 -> bf16) is re-used directly from the accumulator registers as
//      the B operand of O^T[d][head] += Vt P^T (slot order permuted
//      identically in the A operand read from Vt).
#include "dsa_common.hpp"

namespace dsa {

struct FwdParams {
  const unsigned char *q;
  const unsigned char *kv;
  const int32_t *idx;
  uint16_t *out;
  float *lse;
  const float *q_scale;
  const float *kv_scale;
  int64_t S, S_kv, H, G, topk;
  int hpg;          // heads per kv group
  int ntiles;       // ceil(hpg / 32)
  int tiles_per_wg; // head tiles one workgroup covers
  int splits;       // waves sharing one head tile (split over slots)
  int wg_per_tok;   // ceil(ntiles / tiles_per_wg)
  float sl2;        // sm_scale * log2(e)
};

template <int D_QK, int D_V, bool FP8>
struct FwdCfg {
  static constexpr int ELT = FP8 ? 1 : 2;
  static constexpr int CH = 16 / ELT;            // elements per 16-byte chunk
  static constexpr int NCH = D_QK / CH;          // chunks per row
  static constexpr int NCH_V = D_V / CH;         // chunks of the V prefix
  static constexpr int KL_STRIDE = D_QK * ELT + 16;
  static constexpr int VT_STRIDE = 32 * 2 + 8;
  static constexpr int KL_BYTES = 32 * KL_STRIDE;
  static constexpr int VT_BYTES = D_V * VT_STRIDE;
  static constexpr int SC_BYTES = FP8 ? 32 * 4 : 0;
  static constexpr int DT = D_V / 32;
  static constexpr int MERGE_BYTES = DT * 16 * 64 * 4 + 2 * 64 * 4;
  static constexpr int RAW = KL_BYTES + VT_BYTES + SC_BYTES;
  static constexpr int WAVE_BYTES = ((RAW > MERGE_BYTES ? RAW : MERGE_BYTES) + 15) / 16 * 16;
  static constexpr int KSTEPS = D_QK / 16;
  static constexpr int UNITS = 8 * NCH;          // (4 rows x 1 chunk) per 32-row block
  static constexpr int UPL = (UNITS + 63) / 64;
  static_assert(D_V % 32 == 0 && D_QK % 16 == 0 && D_V <= D_QK, "unsupported head dims");
  static_assert(NCH_V * CH == D_V, "d_v must be a whole number of 16-byte chunks");
};

template <bool FP8>
struct QOperand;
template <>
struct QOperand<false> { typedef bf16x8 type; };
template <>
struct QOperand<true> { typedef long type; };

template <int D_QK, int D_V, bool FP8>
__global__ void __launch_bounds__(256)
sparse_mla_fwd_kernel(const FwdParams p) {
  using C = FwdCfg<D_QK, D_V, FP8>;
  typedef typename QOperand<FP8>::type qop_t;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

  const int lane = lane_id(), w = wave_id();
  const int g32 = lane >> 5, l32 = lane & 31;

  const int64_t bid = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t tg = bid % p.wg_per_tok;
  int64_t rest = bid / p.wg_per_tok;
  const int64_t g = rest % p.G;
  rest /= p.G;
  const int64_t tok = rest;                       // b * S + s
  const int64_t b = tok / p.S;

  const int tile_local = w / p.splits, split = w % p.splits;
  const int tile = (int)tg * p.tiles_per_wg + tile_local;
  const bool active = tile_local < p.tiles_per_wg && tile < p.ntiles;

  unsigned char *wsm = smem + w * C::WAVE_BYTES;
  unsigned char *Kl = wsm;
  unsigned char *Vt = wsm + C::KL_BYTES;
  float *Ksc = reinterpret_cast<float *>(wsm + C::KL_BYTES + C::VT_BYTES);

  const int h_local = tile * 32 + l32;
  const bool head_ok = active && h_local < p.hpg;
  const int64_t qrow = tok * p.H + g * p.hpg + h_local;
  const int32_t *idx_row = p.idx + (tok * p.G + g) * p.topk;
  const int64_t kv_row0 = b * p.S_kv;

  // Q as the B operand: lane = head, 8 (bf16) or 8 (fp8) consecutive d per k-step.
  qop_t qreg[C::KSTEPS];
#pragma unroll
  for (int k = 0; k < C::KSTEPS; ++k) {
    if constexpr (FP8) {
      qreg[k] = head_ok ? *reinterpret_cast<const long *>(p.q + qrow * D_QK + 16 * k + 8 * g32) : 0l;
    } else {
      i32x4 v = {0, 0, 0, 0};
      if (head_ok) v = ld_global_16(p.q + (qrow * D_QK + 16 * k + 8 * g32) * 2);
      qreg[k] = as_bf16x8(v);
    }
  }
  float qsc = 1.0f;
  if constexpr (FP8) qsc = p.q_scale[tok];
  const float tscale = p.sl2 * qsc;

  float m_run = kNegBig, l_run = 0.0f;
  f32x16 oacc[C::DT];
#pragma unroll
  for (int t = 0; t < C::DT; ++t)
#pragma unroll
    for (int a = 0; a < 16; ++a) oacc[t][a] = 0.0f;

  const int nblk = (int)((p.topk + 31) / 32);
  if (active) {
    for (int blk = split; blk < nblk; blk += p.splits) {
      const int slot0 = blk * 32;
      int my_idx = -1;
      {
        const int sl = slot0 + l32;
        if (sl < p.topk) {
          const int v = idx_row[sl];
          if (v >= 0 && v < p.S_kv) my_idx = v;
        }
      }
      const uint64_t vmask = __ballot(my_idx >= 0);

      // ---- gather 32 rows into LDS (K row-major, V transposed) ----
#pragma unroll
      for (int uu = 0; uu < C::UPL; ++uu) {
        const int u = lane + 64 * uu;
        const int c = u % C::NCH;
        const int quad = (u / C::NCH) & 7;
        int ri[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) ri[r] = __shfl(my_idx, quad * 4 + r, 64);
        if (u < C::UNITS) {
          i32x4 v[4];
          float sc[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            v[r] = i32x4{0, 0, 0, 0};
            sc[r] = 0.0f;
            if (ri[r] >= 0) {
              const int64_t row = (kv_row0 + ri[r]) * p.G + g;
              v[r] = ld_global_16(p.kv + row * (D_QK * C::ELT) + c * 16);
              if constexpr (FP8) sc[r] = p.kv_scale[kv_row0 + ri[r]];
            }
          }
#pragma unroll
          for (int r = 0; r < 4; ++r)
            *reinterpret_cast<i32x4 *>(Kl + (quad * 4 + r) * C::KL_STRIDE + c * 16) = v[r];
          if (c < C::NCH_V) {
            if constexpr (FP8) {
#pragma unroll
              for (int e = 0; e < 16; ++e) {
                float f[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                  const uint32_t word = (uint32_t)v[r][e >> 2];
                  f[r] = e4m3_to_f32((word >> (8 * (e & 3))) & 0xffu) * sc[r];
                }
                i32x2 pk = {(int)pack_bf16x2(f[0], f[1]), (int)pack_bf16x2(f[2], f[3])};
                *reinterpret_cast<i32x2 *>(Vt + (c * 16 + e) * C::VT_STRIDE + quad * 8) = pk;
              }
            } else {
#pragma unroll
              for (int e = 0; e < 8; ++e) {
                uint32_t h[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                  const uint32_t word = (uint32_t)v[r][e >> 1];
                  h[r] = (e & 1) ? (word >> 16) : (word & 0xffffu);
                }
                i32x2 pk = {(int)(h[0] | (h[1] << 16)), (int)(h[2] | (h[3] << 16))};
                *reinterpret_cast<i32x2 *>(Vt + (c * 8 + e) * C::VT_STRIDE + quad * 8) = pk;
              }
            }
          }
          if constexpr (FP8) {
            if (c == 0) {
#pragma unroll
              for (int r = 0; r < 4; ++r) Ksc[quad * 4 + r] = sc[r];
            }
          }
        }
      }
      wave_lds_sync();

      // ---- S^T = K Q^T  (M = slot, N = head, K = d) ----
      f32x16 sacc;
#pragma unroll
      for (int a = 0; a < 16; ++a) sacc[a] = 0.0f;
#pragma unroll
      for (int k = 0; k < C::KSTEPS; ++k) {
        if constexpr (FP8) {
          const long a = *reinterpret_cast<const long *>(Kl + l32 * C::KL_STRIDE + 16 * k + 8 * g32);
          sacc = __builtin_amdgcn_mfma_f32_32x32x16_fp8_fp8(a, qreg[k], sacc, 0, 0, 0);
        } else {
          const i32x4 a = *reinterpret_cast<const i32x4 *>(Kl + l32 * C::KL_STRIDE + (16 * k + 8 * g32) * 2);
          sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), qreg[k], sacc, 0, 0, 0);
        }
      }

      // ---- online softmax over this block's 32 slots (log2 domain) ----
      float t[16];
      float mloc = kNegBig;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float ksc4[4] = {1.0f, 1.0f, 1.0f, 1.0f};
        if constexpr (FP8) {
          const f32x4 s4 = *reinterpret_cast<const f32x4 *>(Ksc + 8 * i + 4 * g32);
          ksc4[0] = s4[0]; ksc4[1] = s4[1]; ksc4[2] = s4[2]; ksc4[3] = s4[3];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int slot = 8 * i + 4 * g32 + j;
          const bool valid = (vmask >> slot) & 1ull;
          const float v = sacc[4 * i + j] * tscale * ksc4[j];
          t[4 * i + j] = valid ? v : -INFINITY;
          mloc = fmaxf(mloc, t[4 * i + j]);
        }
      }
      mloc = fmaxf(mloc, xor32(mloc));
      const float m_new = fmaxf(m_run, mloc);
      const float alpha = exp2f(m_run - m_new);
      float lsum = 0.0f;
#pragma unroll
      for (int a = 0; a < 16; ++a) {
        t[a] = exp2f(t[a] - m_new);
        lsum += t[a];
      }
      lsum += xor32(lsum);
      l_run = l_run * alpha + lsum;
      m_run = m_new;
#pragma unroll
      for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
        for (int a = 0; a < 16; ++a) oacc[dt][a] *= alpha;

      // ---- O^T[d][head] += Vt[d][slot] P^T[slot][head] ----
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        i32x4 pb;
#pragma unroll
        for (int e = 0; e < 4; ++e) pb[e] = (int)pack_bf16x2(t[8 * kc + 2 * e], t[8 * kc + 2 * e + 1]);
        const bf16x8 bop = as_bf16x8(pb);
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) {
          const unsigned char *vrow = Vt + (dt * 32 + l32) * C::VT_STRIDE;
          const i32x2 lo = *reinterpret_cast<const i32x2 *>(vrow + (16 * kc + 4 * g32) * 2);
          const i32x2 hi = *reinterpret_cast<const i32x2 *>(vrow + (16 * kc + 8 + 4 * g32) * 2);
          const i32x4 av = {lo[0], lo[1], hi[0], hi[1]};
          oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(av), bop, oacc[dt], 0, 0, 0);
        }
      }
      wave_lds_sync();
    }
  }

  // ---- merge the split states of each head tile ----
  __syncthreads();
  float *Ob = reinterpret_cast<float *>(wsm);
  float *ML = Ob + C::DT * 16 * 64;
  if (active) {
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
      for (int a = 0; a < 16; ++a) Ob[(dt * 16 + a) * 64 + lane] = oacc[dt][a];
    ML[lane] = m_run;
    ML[64 + lane] = l_run;
  }
  __syncthreads();
  if (active && split == 0 && head_ok) {
    float mw[4], fw[4];
    float M = kNegBig;
    for (int s2 = 0; s2 < p.splits; ++s2) {
      const float *MLs = reinterpret_cast<const float *>(smem + (w + s2) * C::WAVE_BYTES) + C::DT * 16 * 64;
      mw[s2] = MLs[lane];
      M = fmaxf(M, mw[s2]);
    }
    float L = 0.0f;
    for (int s2 = 0; s2 < p.splits; ++s2) {
      const float *MLs = reinterpret_cast<const float *>(smem + (w + s2) * C::WAVE_BYTES) + C::DT * 16 * 64;
      fw[s2] = exp2f(mw[s2] - M);
      L += MLs[64 + lane] * fw[s2];
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    uint16_t *orow = p.out + qrow * D_V;
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float acc = 0.0f;
          for (int s2 = 0; s2 < p.splits; ++s2) {
            const float *Os = reinterpret_cast<const float *>(smem + (w + s2) * C::WAVE_BYTES);
            acc += Os[(dt * 16 + 4 * i + j) * 64 + lane] * fw[s2];
          }
          o[j] = acc * inv;
        }
        const i32x2 pk = {(int)pack_bf16x2(o[0], o[1]), (int)pack_bf16x2(o[2], o[3])};
        *reinterpret_cast<i32x2 *>(orow + dt * 32 + 8 * i + 4 * g32) = pk;
      }
    }
    if (g32 == 0) p.lse[qrow] = L > 0.0f ? log2f(L) + M : -INFINITY;
  }
}

template <int D_QK, int D_V, bool FP8>
static int launch_fwd(const FwdParams &p, int64_t nblocks, hipStream_t st) {
  using C = FwdCfg<D_QK, D_V, FP8>;
  const size_t lds = 4 * (size_t)C::WAVE_BYTES;
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute((const void *)sparse_mla_fwd_kernel<D_QK, D_V, FP8>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return set_error(DSA_ERR_HIP, "sparse_mla_fwd: LDS attribute: %s", hipGetErrorString(e));
  }
  hipLaunchKernelGGL((sparse_mla_fwd_kernel<D_QK, D_V, FP8>), dim3((unsigned)nblocks), dim3(256), lds, st, p);
  return check_launch("sparse_mla_fwd");
}

// Fill a head-tile decomposition shared by the forward and backward kernels.
void plan_head_tiles(int64_t hpg, int *ntiles, int *tiles_per_wg, int *splits, int *wg_per_tok) {
  const int nt = (int)((hpg + 31) / 32);
  const int tw = nt >= 4 ? 4 : nt;
  *ntiles = nt;
  *tiles_per_wg = tw;
  *splits = 4 / tw;
  *wg_per_tok = (nt + tw - 1) / tw;
}

}  // namespace dsa

using namespace dsa;

extern "C" int dsa_sparse_mla_fwd(const void *q, const void *kv, const int32_t *indices, void *out,
                                  float *lse2, int64_t B, int64_t S, int64_t S_kv, int64_t H,
                                  int64_t G, int64_t D_qk, int64_t D_v, int64_t topk, float sm_scale,
                                  int dtype, const float *q_scale, const float *kv_scale,
                                  void *stream) {
  DSA_REQUIRE(B >= 0 && S >= 0 && S_kv > 0 && H > 0 && G > 0 && topk > 0,
              "dsa_sparse_mla_fwd: bad dims B=%lld S=%lld S_kv=%lld H=%lld G=%lld topk=%lld",
              (long long)B, (long long)S, (long long)S_kv, (long long)H, (long long)G, (long long)topk);
  DSA_REQUIRE(H % G == 0, "dsa_sparse_mla_fwd: H=%lld not divisible by G=%lld", (long long)H, (long long)G);
  DSA_REQUIRE(D_v > 0 && D_v <= D_qk, "dsa_sparse_mla_fwd: need 0 < d_v <= d_qk (got %lld, %lld)",
              (long long)D_v, (long long)D_qk);
  DSA_REQUIRE(dtype == DSA_DTYPE_BF16 || dtype == DSA_DTYPE_E4M3, "dsa_sparse_mla_fwd: dtype %d", dtype);
  DSA_REQUIRE(S_kv < (1ll << 31) && topk < (1ll << 31), "dsa_sparse_mla_fwd: S_kv/topk too large");
  if (B == 0 || S == 0) return DSA_OK;
  DSA_REQUIRE(q && kv && indices && out && lse2, "dsa_sparse_mla_fwd: null tensor pointer");
  if (dtype == DSA_DTYPE_E4M3)
    DSA_REQUIRE(q_scale && kv_scale, "dsa_sparse_mla_fwd: e4m3 input needs q_scale and kv_scale");
  FwdParams p;
  p.q = static_cast<const unsigned char *>(q);
  p.kv = static_cast<const unsigned char *>(kv);
  p.idx = indices;
  p.out = static_cast<uint16_t *>(out);
  p.lse = lse2;
  p.q_scale = q_scale;
  p.kv_scale = kv_scale;
  p.S = S;
  p.S_kv = S_kv;
  p.H = H;
  p.G = G;
  p.topk = topk;
  p.hpg = (int)(H / G);
  plan_head_tiles(p.hpg, &p.ntiles, &p.tiles_per_wg, &p.splits, &p.wg_per_tok);
  p.sl2 = sm_scale * kLog2e;
  const int64_t nblocks = B * S * G * p.wg_per_tok;
  DSA_REQUIRE(nblocks < (1ll << 31), "dsa_sparse_mla_fwd: grid too large");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool f8 = dtype == DSA_DTYPE_E4M3;
  if (D_qk == 128 && D_v == 64) return f8 ? launch_fwd<128, 64, true>(p, nblocks, st) : launch_fwd<128, 64, false>(p, nblocks, st);
  if (D_qk == 128 && D_v == 128) return f8 ? launch_fwd<128, 128, true>(p, nblocks, st) : launch_fwd<128, 128, false>(p, nblocks, st);
  if (D_qk == 192 && D_v == 128) return f8 ? launch_fwd<192, 128, true>(p, nblocks, st) : launch_fwd<192, 128, false>(p, nblocks, st);
  if (D_qk == 64 && D_v == 32 && !f8) return launch_fwd<64, 32, false>(p, nblocks, st);
  return set_error(DSA_ERR_UNSUPPORTED, "dsa_sparse_mla_fwd: no kernel for d_qk=%lld d_v=%lld dtype=%d",
                   (long long)D_qk, (long long)D_v, dtype);
}
