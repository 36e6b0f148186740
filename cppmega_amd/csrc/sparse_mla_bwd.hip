// SparseMLA backward for gfx950 (bf16 and OCP-e4m3 tensorwise), deterministic.
//
// Reference semantics: cppmega/megatron/sparse_mla_ops/tilelang_sparse_mla_bwd.py:123-167
// (Delta), :204-419 (P recompute, dP, dS, dQ, dKV scatter) and :170-201 (fp32 ->
// bf16 dKV), plus tilelang_sparse_mla_bwd_fp8.py:199-489 for the e4m3 form
// (QK^T on e4m3 codes, bf16-dequantised Q / KV for the other GEMMs).
//
// The reference scatters dKV with fp32 atomics (non-deterministic).  Here the
// backward runs as
//   1. csr_count / scan / csr_fill: an inverse index kv-row -> list of
//      (token, slot) entries (counting sort over the int32 indices);
//   2. bwd_main (query-major, one workgroup per token and kv group): Delta,
//      P = exp2(s * scale' - LSE2), dP = dO V^T, dS = P (dP - Delta) scale,
//      dQ = dS K written directly, and the per-(token, slot) dKV row
//      c = dS^T Q + P^T dO written as fp32 to a workspace;
//   3. dkv_reduce (kv-major, one workgroup per kv row): the row's entries are
//      sorted ascending and their fp32 rows summed in that fixed order (four
//      contiguous quarters combined in a fixed tree), then cast to bf16.
// Every addition therefore happens in an order fixed by the indices alone, so
// repeated calls are bitwise identical.
//
// bwd_main MFMA orientation (32x32x16, wave = 32 heads x 32 slots per block):
//   S = Q K^T and dP = dO V^T with M = head, N = slot: each lane then owns one
//   slot and 16 heads, which is exactly the A-operand layout (M = slot,
//   K = head) of c = dS Q + P dO, so dS / P feed that GEMM from registers.
//   dQ = dS K contracts over slots, so dS is transposed once through LDS
//   (dS_t[head][slot]) and K is also kept transposed (Kt[d][slot]).
#include "dsa_common.hpp"

namespace dsa {

void plan_head_tiles(int64_t hpg, int *ntiles, int *tiles_per_wg, int *splits, int *wg_per_tok);

struct BwdParams {
  const unsigned char *q;
  const unsigned char *kv;
  const uint16_t *o;
  const uint16_t *dO;
  const int32_t *idx;
  const float *lse;
  const float *delta;  // optional precomputed Delta [B,S,H]
  uint16_t *dq;
  const float *q_scale;
  const float *kv_scale;
  float *partials;
  int64_t S, S_kv, H, G, topk;
  int hpg, ntiles, tiles_per_wg, splits, wg_per_tok;
  float sl2;    // sm_scale * log2(e)
  float scale;  // sm_scale
};

template <int D_QK, int D_V, bool FP8>
struct BwdCfg {
  static constexpr int ELT = FP8 ? 1 : 2;
  static constexpr int CH = 16 / ELT;
  static constexpr int NCH = D_QK / CH;
  static constexpr int NCH_V = D_V / CH;
  static constexpr int KL_STRIDE = D_QK * ELT + 16;   // raw K rows (bf16 or e4m3)
  static constexpr int KD_STRIDE = D_V * 2 + 16;      // e4m3 only: dequantised V rows (bf16)
  static constexpr int KT_STRIDE = 32 * 2 + 16;       // Kt[d][slot] bf16
  static constexpr int DS_STRIDE = 32 * 2 + 16;       // dS_t[head][slot] bf16
  static constexpr int QT_STRIDE = 32 * 2 + 8;        // prologue: Qt[d][head], dOt[d][head]
  static constexpr int KL_BYTES = 32 * KL_STRIDE;
  static constexpr int KD_BYTES = FP8 ? 32 * KD_STRIDE : 0;
  static constexpr int KT_BYTES = D_QK * KT_STRIDE;
  static constexpr int DS_BYTES = 32 * DS_STRIDE;
  static constexpr int SC_BYTES = FP8 ? 32 * 4 : 0;
  static constexpr int LD_BYTES = 64 * 4;             // lse2 (eff) and Delta per head
  static constexpr int OFF_KD = KL_BYTES;
  static constexpr int OFF_KT = OFF_KD + KD_BYTES;
  static constexpr int OFF_DS = OFF_KT + KT_BYTES;
  static constexpr int OFF_SC = OFF_DS + DS_BYTES;
  static constexpr int OFF_LD = OFF_SC + SC_BYTES;
  static constexpr int RAW = OFF_LD + LD_BYTES;
  static constexpr int DQT = D_QK / 32;
  static constexpr int DVT = D_V / 32;
  static constexpr int MERGE_BYTES = DQT * 16 * 64 * 4;
  static constexpr int PRO_BYTES = (D_QK + D_V) * QT_STRIDE;
  static constexpr int WAVE_BYTES = ((RAW > MERGE_BYTES ? RAW : MERGE_BYTES) + 15) / 16 * 16;
  static constexpr int KSTEPS = D_QK / 16;
  static constexpr int VSTEPS = D_V / 16;
  static constexpr int UNITS = 8 * NCH;
  static constexpr int UPL = (UNITS + 63) / 64;
  static_assert(PRO_BYTES <= OFF_LD, "prologue tiles must fit below the lse/delta slot");
  static_assert(D_V % 32 == 0 && D_QK % 32 == 0 && D_V <= D_QK, "unsupported head dims");
  static_assert(NCH_V * CH == D_V, "d_v must be a whole number of 16-byte chunks");
};

template <bool FP8>
struct QOp;
template <>
struct QOp<false> { typedef bf16x8 type; };
template <>
struct QOp<true> { typedef long type; };

template <int D_QK, int D_V, bool FP8>
__global__ void __launch_bounds__(256)
sparse_mla_bwd_main_kernel(const BwdParams p) {
  using C = BwdCfg<D_QK, D_V, FP8>;
  typedef typename QOp<FP8>::type qop_t;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

  const int lane = lane_id(), w = wave_id();
  const int g32 = lane >> 5, l32 = lane & 31;

  const int64_t bid = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t tg = bid % p.wg_per_tok;
  int64_t rest = bid / p.wg_per_tok;
  const int64_t g = rest % p.G;
  const int64_t tok = rest / p.G;
  const int64_t b = tok / p.S;

  const int tile_local = w / p.splits, split = w % p.splits;
  const int tile = (int)tg * p.tiles_per_wg + tile_local;
  const bool active = tile_local < p.tiles_per_wg && tile < p.ntiles;

  unsigned char *wsm = smem + w * C::WAVE_BYTES;
  unsigned char *Kl = wsm;
  unsigned char *Kd = wsm + C::OFF_KD;
  unsigned char *Kt = wsm + C::OFF_KT;
  unsigned char *DSt = wsm + C::OFF_DS;
  float *Ksc = reinterpret_cast<float *>(wsm + C::OFF_SC);
  float *LD = reinterpret_cast<float *>(wsm + C::OFF_LD);

  const int h_local = tile * 32 + l32;      // head owned by this lane in the A-operand role
  const bool head_ok = active && h_local < p.hpg;
  const int64_t qrow = tok * p.H + g * p.hpg + h_local;
  const int64_t entry0 = (tok * p.G + g) * p.topk;  // entry (= key) of slot 0
  const int32_t *idx_row = p.idx + entry0;
  const int64_t kv_row0 = b * p.S_kv;

  float qsc = 1.0f;
  if constexpr (FP8) qsc = p.q_scale[tok];

  // ---------------- prologue ----------------
  qop_t qA[C::KSTEPS];
  bf16x8 doA[C::VSTEPS];
  float delta_part = 0.0f;
#pragma unroll
  for (int k = 0; k < C::KSTEPS; ++k) {
    if constexpr (FP8) {
      qA[k] = head_ok ? *reinterpret_cast<const long *>(p.q + qrow * D_QK + 16 * k + 8 * g32) : 0l;
    } else {
      i32x4 v = {0, 0, 0, 0};
      if (head_ok) v = ld_global_16(p.q + (qrow * D_QK + 16 * k + 8 * g32) * 2);
      qA[k] = as_bf16x8(v);
    }
  }
#pragma unroll
  for (int k = 0; k < C::VSTEPS; ++k) {
    i32x4 dv = {0, 0, 0, 0}, ov = {0, 0, 0, 0};
    if (head_ok) {
      dv = ld_global_16(p.dO + qrow * D_V + 16 * k + 8 * g32);
      ov = ld_global_16(p.o + qrow * D_V + 16 * k + 8 * g32);
    }
    doA[k] = as_bf16x8(dv);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t du = (uint32_t)dv[e], ou = (uint32_t)ov[e];
      delta_part += bf16_bits_to_f32(ou & 0xffffu) * bf16_bits_to_f32(du & 0xffffu);
      delta_part += bf16_bits_to_f32(ou >> 16) * bf16_bits_to_f32(du >> 16);
    }
  }
  float delta_h = delta_part + xor32(delta_part);
  if (p.delta != nullptr && head_ok) delta_h = p.delta[qrow];
  float lse_h = INFINITY;  // padded heads: P = exp2(x - inf) = 0
  if (head_ok) {
    const float l = p.lse[qrow];
    lse_h = (l == -INFINITY) ? INFINITY : l;  // all-masked row: zero gradient
  }

  // Transposed Q (dequantised for e4m3) and dO tiles -> B operands of c = dS Q + P dO.
  bf16x8 qB[2][C::DQT];
  bf16x8 doB[2][C::DVT];
  if (active) {
    unsigned char *Qt = wsm;
    unsigned char *dOt = wsm + D_QK * C::QT_STRIDE;
#pragma unroll
    for (int k = 0; k < C::KSTEPS; ++k) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        uint32_t hbits;
        if constexpr (FP8) {
          const uint32_t code = (uint32_t)((unsigned long)qA[k] >> (8 * e)) & 0xffu;
          hbits = f32_to_bf16_bits(e4m3_to_f32(code) * qsc);
        } else {
          const i32x4 v = __builtin_bit_cast(i32x4, qA[k]);
          const uint32_t word = (uint32_t)v[e >> 1];
          hbits = (e & 1) ? (word >> 16) : (word & 0xffffu);
        }
        *reinterpret_cast<uint16_t *>(Qt + (16 * k + 8 * g32 + e) * C::QT_STRIDE + l32 * 2) = (uint16_t)hbits;
      }
    }
#pragma unroll
    for (int k = 0; k < C::VSTEPS; ++k) {
      const i32x4 v = __builtin_bit_cast(i32x4, doA[k]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t word = (uint32_t)v[e >> 1];
        const uint32_t hbits = (e & 1) ? (word >> 16) : (word & 0xffffu);
        *reinterpret_cast<uint16_t *>(dOt + (16 * k + 8 * g32 + e) * C::QT_STRIDE + l32 * 2) = (uint16_t)hbits;
      }
    }
    if (g32 == 0) {
      LD[l32] = lse_h;
      LD[32 + l32] = delta_h;
    }
    wave_lds_sync();
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
#pragma unroll
      for (int dt = 0; dt < C::DQT; ++dt) {
        const unsigned char *row = Qt + (dt * 32 + l32) * C::QT_STRIDE;
        const i32x2 lo = *reinterpret_cast<const i32x2 *>(row + (16 * kc + 4 * g32) * 2);
        const i32x2 hi = *reinterpret_cast<const i32x2 *>(row + (16 * kc + 8 + 4 * g32) * 2);
        qB[kc][dt] = as_bf16x8(i32x4{lo[0], lo[1], hi[0], hi[1]});
      }
#pragma unroll
      for (int dt = 0; dt < C::DVT; ++dt) {
        const unsigned char *row = dOt + (dt * 32 + l32) * C::QT_STRIDE;
        const i32x2 lo = *reinterpret_cast<const i32x2 *>(row + (16 * kc + 4 * g32) * 2);
        const i32x2 hi = *reinterpret_cast<const i32x2 *>(row + (16 * kc + 8 + 4 * g32) * 2);
        doB[kc][dt] = as_bf16x8(i32x4{lo[0], lo[1], hi[0], hi[1]});
      }
    }
    wave_lds_sync();
  }

  f32x16 dqacc[C::DQT];
#pragma unroll
  for (int t = 0; t < C::DQT; ++t)
#pragma unroll
    for (int a = 0; a < 16; ++a) dqacc[t][a] = 0.0f;

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
      // ---- gather: K rows (raw), Kt (bf16, dequantised), Kd (e4m3: bf16 V rows) ----
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
          if constexpr (FP8) {
            uint32_t hb[4][16];
#pragma unroll
            for (int e = 0; e < 16; ++e) {
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const uint32_t word = (uint32_t)v[r][e >> 2];
                hb[r][e] = f32_to_bf16_bits(e4m3_to_f32((word >> (8 * (e & 3))) & 0xffu) * sc[r]);
              }
              const i32x2 pk = {(int)(hb[0][e] | (hb[1][e] << 16)), (int)(hb[2][e] | (hb[3][e] << 16))};
              *reinterpret_cast<i32x2 *>(Kt + (c * 16 + e) * C::KT_STRIDE + quad * 8) = pk;
            }
            if (c < C::NCH_V) {
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const i32x4 lo = {(int)(hb[r][0] | (hb[r][1] << 16)), (int)(hb[r][2] | (hb[r][3] << 16)),
                                  (int)(hb[r][4] | (hb[r][5] << 16)), (int)(hb[r][6] | (hb[r][7] << 16))};
                const i32x4 hi = {(int)(hb[r][8] | (hb[r][9] << 16)), (int)(hb[r][10] | (hb[r][11] << 16)),
                                  (int)(hb[r][12] | (hb[r][13] << 16)), (int)(hb[r][14] | (hb[r][15] << 16))};
                unsigned char *dst = Kd + (quad * 4 + r) * C::KD_STRIDE + c * 32;
                *reinterpret_cast<i32x4 *>(dst) = lo;
                *reinterpret_cast<i32x4 *>(dst + 16) = hi;
              }
            }
            if (c == 0) {
#pragma unroll
              for (int r = 0; r < 4; ++r) Ksc[quad * 4 + r] = sc[r];
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
              const i32x2 pk = {(int)(h[0] | (h[1] << 16)), (int)(h[2] | (h[3] << 16))};
              *reinterpret_cast<i32x2 *>(Kt + (c * 8 + e) * C::KT_STRIDE + quad * 8) = pk;
            }
          }
        }
      }
      wave_lds_sync();

      // ---- S = Q K^T and dP = dO V^T  (M = head, N = slot) ----
      f32x16 sacc, dpacc;
#pragma unroll
      for (int a = 0; a < 16; ++a) {
        sacc[a] = 0.0f;
        dpacc[a] = 0.0f;
      }
#pragma unroll
      for (int k = 0; k < C::KSTEPS; ++k) {
        if constexpr (FP8) {
          const long kb = *reinterpret_cast<const long *>(Kl + l32 * C::KL_STRIDE + 16 * k + 8 * g32);
          sacc = __builtin_amdgcn_mfma_f32_32x32x16_fp8_fp8(qA[k], kb, sacc, 0, 0, 0);
        } else {
          const i32x4 kb = *reinterpret_cast<const i32x4 *>(Kl + l32 * C::KL_STRIDE + (16 * k + 8 * g32) * 2);
          sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qA[k], as_bf16x8(kb), sacc, 0, 0, 0);
        }
      }
#pragma unroll
      for (int k = 0; k < C::VSTEPS; ++k) {
        i32x4 vb;
        if constexpr (FP8)
          vb = *reinterpret_cast<const i32x4 *>(Kd + l32 * C::KD_STRIDE + (16 * k + 8 * g32) * 2);
        else
          vb = *reinterpret_cast<const i32x4 *>(Kl + l32 * C::KL_STRIDE + (16 * k + 8 * g32) * 2);
        dpacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(doA[k], as_bf16x8(vb), dpacc, 0, 0, 0);
      }

      // ---- P, dS (lane = slot l32, heads 8i + 4*g32 + j) ----
      const bool valid = my_idx >= 0;
      float xs = p.sl2;
      if constexpr (FP8) xs *= qsc * Ksc[l32];
      float P[16], dS[16];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x4 l4 = *reinterpret_cast<const f32x4 *>(LD + 8 * i + 4 * g32);
        const f32x4 d4 = *reinterpret_cast<const f32x4 *>(LD + 32 + 8 * i + 4 * g32);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int a = 4 * i + j;
          const float pv = valid ? exp2f(sacc[a] * xs - l4[j]) : 0.0f;
          P[a] = pv;
          dS[a] = pv * (dpacc[a] - d4[j]) * p.scale;
        }
      }
      // dS^T -> LDS as dS_t[head][slot] (bf16) for the dQ GEMM
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          *reinterpret_cast<uint16_t *>(DSt + (8 * i + 4 * g32 + j) * C::DS_STRIDE + l32 * 2) =
              (uint16_t)f32_to_bf16_bits(dS[4 * i + j]);

      // ---- c[slot][d] = dS Q + P dO  (M = slot, N = d, K = head) -> partials ----
      bf16x8 dsA[2], pA[2];
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        i32x4 ds4, p4;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          ds4[e] = (int)pack_bf16x2(dS[8 * kc + 2 * e], dS[8 * kc + 2 * e + 1]);
          p4[e] = (int)pack_bf16x2(P[8 * kc + 2 * e], P[8 * kc + 2 * e + 1]);
        }
        dsA[kc] = as_bf16x8(ds4);
        pA[kc] = as_bf16x8(p4);
      }
      const uint64_t vmask = __ballot(valid);
#pragma unroll
      for (int dt = 0; dt < C::DQT; ++dt) {
        f32x16 cacc;
#pragma unroll
        for (int a = 0; a < 16; ++a) cacc[a] = 0.0f;
#pragma unroll
        for (int kc = 0; kc < 2; ++kc)
          cacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(dsA[kc], qB[kc][dt], cacc, 0, 0, 0);
        if (dt < C::DVT) {
#pragma unroll
          for (int kc = 0; kc < 2; ++kc)
            cacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pA[kc], doB[kc][dt < C::DVT ? dt : 0], cacc, 0, 0, 0);
        }
        // lane: d = dt*32 + l32, slots 8i + 4*g32 + j
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int slot = 8 * i + 4 * g32 + j;
            if ((vmask >> slot) & 1ull) {
              const int64_t key = entry0 + slot0 + slot;
              p.partials[(key * p.ntiles + tile) * D_QK + dt * 32 + l32] = cacc[4 * i + j];
            }
          }
      }
      wave_lds_sync();

      // ---- dQ[head][d] += dS_t[head][slot] Kt[d][slot]^T  (M = head, N = d, K = slot) ----
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        const i32x4 av = *reinterpret_cast<const i32x4 *>(DSt + l32 * C::DS_STRIDE + (16 * kc + 8 * g32) * 2);
#pragma unroll
        for (int dt = 0; dt < C::DQT; ++dt) {
          const i32x4 bv = *reinterpret_cast<const i32x4 *>(Kt + (dt * 32 + l32) * C::KT_STRIDE + (16 * kc + 8 * g32) * 2);
          dqacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(av), as_bf16x8(bv), dqacc[dt], 0, 0, 0);
        }
      }
      wave_lds_sync();
    }
  }

  // ---------------- merge dQ over the slot splits (fixed order) ----------------
  __syncthreads();
  float *Ob = reinterpret_cast<float *>(wsm);
  if (active) {
#pragma unroll
    for (int dt = 0; dt < C::DQT; ++dt)
#pragma unroll
      for (int a = 0; a < 16; ++a) Ob[(dt * 16 + a) * 64 + lane] = dqacc[dt][a];
  }
  __syncthreads();
  if (active && split == 0) {
    // lane: d = dt*32 + l32 (N), heads 8i + 4*g32 + j (M)
#pragma unroll
    for (int dt = 0; dt < C::DQT; ++dt) {
#pragma unroll
      for (int a = 0; a < 16; ++a) {
        float acc = 0.0f;
        for (int s2 = 0; s2 < p.splits; ++s2) {
          const float *Os = reinterpret_cast<const float *>(smem + (w + s2) * C::WAVE_BYTES);
          acc += Os[(dt * 16 + a) * 64 + lane];
        }
        const int hl = tile * 32 + 8 * (a >> 2) + 4 * g32 + (a & 3);
        if (hl < p.hpg) {
          const int64_t row = tok * p.H + g * p.hpg + hl;
          p.dq[row * D_QK + dt * 32 + l32] = (uint16_t)f32_to_bf16_bits(acc);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Inverse index (kv row -> entries) and the deterministic dKV reduction
// ---------------------------------------------------------------------------
__global__ void fill_i32_kernel(int32_t *p, int64_t n, int32_t v) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

struct CsrParams {
  const int32_t *idx;
  int32_t *cnt;
  int32_t *cur;
  int32_t *rowptr;
  int32_t *refs;
  int64_t entries;  // B*S*G*topk
  int64_t S, S_kv, G, topk;
};

__device__ __forceinline__ int64_t entry_row(const CsrParams &p, int64_t e, int32_t j) {
  const int64_t tokg = e / p.topk;
  const int64_t g = tokg % p.G;
  const int64_t b = (tokg / p.G) / p.S;
  return (b * p.S_kv + j) * p.G + g;
}

__global__ void csr_count_kernel(const CsrParams p) {
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < p.entries;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int32_t j = p.idx[e];
    if (j >= 0 && j < p.S_kv) atomicAdd(p.cnt + entry_row(p, e, j), 1);
  }
}

__global__ void csr_fill_kernel(const CsrParams p) {
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < p.entries;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int32_t j = p.idx[e];
    if (j >= 0 && j < p.S_kv) {
      const int64_t r = entry_row(p, e, j);
      const int32_t pos = p.rowptr[r] + atomicAdd(p.cur + r, 1);
      p.refs[pos] = (int32_t)e;
    }
  }
}

// Exclusive scan of cnt[0..n) into rowptr[0..n] with one 1024-thread workgroup.
__global__ void __launch_bounds__(1024) csr_scan_kernel(const int32_t *cnt, int32_t *rowptr, int64_t n) {
  __shared__ int32_t wsum[16];
  const int tid = threadIdx.x;
  const int64_t per = (n + 1023) / 1024;
  const int64_t lo = tid * per, hi = lo + per < n ? lo + per : n;
  int32_t s = 0;
  for (int64_t i = lo; i < hi; ++i) s += cnt[i];
  // inclusive scan of s over the block
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
  int32_t run = (wv > 0 ? wsum[wv - 1] : 0) + v - s;  // exclusive prefix of this thread
  for (int64_t i = lo; i < hi; ++i) {
    rowptr[i] = run;
    run += cnt[i];
  }
  if (tid == 1023) rowptr[n] = wsum[15];
}

constexpr int kReduceCap = 4096;  // entries sorted in LDS; longer segments sort in place in global memory

// Ascending sort of a[0..n) with an all-ascending bitonic network (the "flip"
// form), so elements at or beyond n act as +inf and are never touched.
template <typename Ptr>
__device__ void bitonic_sort_asc(Ptr a, int n, int npow2) {
  for (int k = 2; k <= npow2; k <<= 1) {
    for (int i = threadIdx.x; i < npow2; i += blockDim.x) {
      const int pr = i ^ (k - 1);
      if (pr > i && pr < n) {
        const int32_t x = a[i], y = a[pr];
        if (x > y) { a[i] = y; a[pr] = x; }
      }
    }
    __syncthreads();
    for (int d = k >> 2; d > 0; d >>= 1) {
      for (int i = threadIdx.x; i < npow2; i += blockDim.x) {
        const int pr = i ^ d;
        if (pr > i && pr < n) {
          const int32_t x = a[i], y = a[pr];
          if (x > y) { a[i] = y; a[pr] = x; }
        }
      }
      __syncthreads();
    }
  }
}

template <int D_QK>
__global__ void __launch_bounds__(256)
dkv_reduce_kernel(const int32_t *rowptr, int32_t *refs, const float *partials, uint16_t *dkv,
                  int64_t nrows, int ntiles) {
  __shared__ int32_t keys[kReduceCap];
  __shared__ float part[4][D_QK];
  const int64_t r = blockIdx.x;
  if (r >= nrows) return;
  const int32_t base = rowptr[r];
  const int n = rowptr[r + 1] - base;
  const int tid = threadIdx.x;
  if (n == 0) {
    for (int d = tid; d < D_QK; d += 256) dkv[r * D_QK + d] = 0;
    return;
  }
  int npow2 = 1;
  while (npow2 < n) npow2 <<= 1;
  const int32_t *sorted;
  if (n <= kReduceCap) {
    for (int i = tid; i < n; i += 256) keys[i] = refs[base + i];
    __syncthreads();
    bitonic_sort_asc(keys, n, npow2);
    sorted = keys;
  } else {
    bitonic_sort_asc(refs + base, n, npow2);
    sorted = refs + base;
  }
  // four contiguous quarters, one per wave, combined in a fixed order
  const int w = tid >> 6, lane = tid & 63;
  const int q0 = (int)((int64_t)n * w / 4), q1 = (int)((int64_t)n * (w + 1) / 4);
  constexpr int PER = (D_QK + 63) / 64;
  float acc[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) acc[k] = 0.0f;
  for (int i = q0; i < q1; ++i) {
    const int64_t key = sorted[i];
    for (int t = 0; t < ntiles; ++t) {
      const float *row = partials + (key * ntiles + t) * D_QK;
#pragma unroll
      for (int k = 0; k < PER; ++k) {
        const int d = lane + 64 * k;
        if (d < D_QK) acc[k] += row[d];
      }
    }
  }
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int d = lane + 64 * k;
    if (d < D_QK) part[w][d] = acc[k];
  }
  __syncthreads();
  for (int d = tid; d < D_QK; d += 256) {
    const float v = ((part[0][d] + part[1][d]) + part[2][d]) + part[3][d];
    dkv[r * D_QK + d] = (uint16_t)f32_to_bf16_bits(v);
  }
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct BwdWorkspace {
  size_t partials, cnt, cur, rowptr, refs, total;
};

static BwdWorkspace bwd_layout(int64_t B, int64_t S, int64_t S_kv, int64_t H, int64_t G, int64_t D_qk,
                               int64_t topk) {
  int nt, tw, sp, wpt;
  plan_head_tiles(H / (G > 0 ? G : 1), &nt, &tw, &sp, &wpt);
  const size_t entries = (size_t)B * S * G * topk;
  const size_t rows = (size_t)B * S_kv * G;
  BwdWorkspace L;
  size_t off = 0;
  L.partials = off;
  off += align256(entries * nt * D_qk * sizeof(float));
  L.cnt = off;
  off += align256(rows * 4);
  L.cur = off;
  off += align256(rows * 4);
  L.rowptr = off;
  off += align256((rows + 1) * 4);
  L.refs = off;
  off += align256(entries * 4);
  L.total = off;
  return L;
}

template <int D_QK, int D_V, bool FP8>
static int launch_bwd_main(const BwdParams &p, int64_t nblocks, hipStream_t st) {
  using C = BwdCfg<D_QK, D_V, FP8>;
  const size_t lds = 4 * (size_t)C::WAVE_BYTES;
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute((const void *)sparse_mla_bwd_main_kernel<D_QK, D_V, FP8>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return set_error(DSA_ERR_HIP, "sparse_mla_bwd: LDS attribute: %s", hipGetErrorString(e));
  }
  hipLaunchKernelGGL((sparse_mla_bwd_main_kernel<D_QK, D_V, FP8>), dim3((unsigned)nblocks), dim3(256), lds, st, p);
  return check_launch("sparse_mla_bwd_main");
}

}  // namespace dsa

using namespace dsa;

extern "C" size_t dsa_sparse_mla_bwd_workspace_size(int64_t B, int64_t S, int64_t S_kv, int64_t H,
                                                    int64_t G, int64_t D_qk, int64_t D_v, int64_t topk) {
  (void)D_v;
  if (B <= 0 || S <= 0 || S_kv <= 0 || H <= 0 || G <= 0 || topk <= 0 || D_qk <= 0) return 0;
  return bwd_layout(B, S, S_kv, H, G, D_qk, topk).total;
}

extern "C" int dsa_sparse_mla_bwd(const void *q, const void *kv, const void *o, const void *dO,
                                  const int32_t *indices, const float *lse2, const float *delta,
                                  void *dq, void *dkv,
                                  void *workspace, size_t workspace_bytes, int64_t B, int64_t S,
                                  int64_t S_kv, int64_t H, int64_t G, int64_t D_qk, int64_t D_v,
                                  int64_t topk, float sm_scale, int dtype, const float *q_scale,
                                  const float *kv_scale, void *stream) {
  DSA_REQUIRE(B >= 0 && S >= 0 && S_kv > 0 && H > 0 && G > 0 && topk > 0,
              "dsa_sparse_mla_bwd: bad dims B=%lld S=%lld S_kv=%lld H=%lld G=%lld topk=%lld",
              (long long)B, (long long)S, (long long)S_kv, (long long)H, (long long)G, (long long)topk);
  DSA_REQUIRE(H % G == 0, "dsa_sparse_mla_bwd: H=%lld not divisible by G=%lld", (long long)H, (long long)G);
  DSA_REQUIRE(D_v > 0 && D_v <= D_qk, "dsa_sparse_mla_bwd: need 0 < d_v <= d_qk");
  DSA_REQUIRE(dtype == DSA_DTYPE_BF16 || dtype == DSA_DTYPE_E4M3, "dsa_sparse_mla_bwd: dtype %d", dtype);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t rows = B * S_kv * G;
  if (B == 0) return DSA_OK;
  DSA_REQUIRE(dkv, "dsa_sparse_mla_bwd: null dkv");
  const int64_t entries = B * S * G * topk;
  DSA_REQUIRE(entries < (1ll << 31) && rows < (1ll << 31), "dsa_sparse_mla_bwd: too many entries for int32 keys");
  DSA_REQUIRE(q && kv && o && dO && indices && lse2 && dq, "dsa_sparse_mla_bwd: null tensor pointer");
  if (dtype == DSA_DTYPE_E4M3)
    DSA_REQUIRE(q_scale && kv_scale, "dsa_sparse_mla_bwd: e4m3 input needs q_scale and kv_scale");
  const bool f8 = dtype == DSA_DTYPE_E4M3;
  const bool shape_ok = (D_qk == 128 && D_v == 64) || (D_qk == 128 && D_v == 128) ||
                        (D_qk == 192 && D_v == 128) || (D_qk == 64 && D_v == 32 && !f8);
  if (!shape_ok)
    return set_error(DSA_ERR_UNSUPPORTED, "dsa_sparse_mla_bwd: no kernel for d_qk=%lld d_v=%lld dtype=%d",
                     (long long)D_qk, (long long)D_v, dtype);
  const BwdWorkspace L = bwd_layout(B, S, S_kv, H, G, D_qk, topk);
  if (!workspace || workspace_bytes < L.total)
    return set_error(DSA_ERR_WORKSPACE, "dsa_sparse_mla_bwd: workspace %zu < required %zu", workspace_bytes,
                     L.total);
  unsigned char *ws = static_cast<unsigned char *>(workspace);
  if (S == 0) {  // no queries: dKV is zero
    hipLaunchKernelGGL(fill_i32_kernel, dim3(256), dim3(256), 0, st, reinterpret_cast<int32_t *>(dkv),
                       (rows * D_qk) / 2, 0);
    return check_launch("sparse_mla_bwd(fill)");
  }

  CsrParams cp;
  cp.idx = indices;
  cp.cnt = reinterpret_cast<int32_t *>(ws + L.cnt);
  cp.cur = reinterpret_cast<int32_t *>(ws + L.cur);
  cp.rowptr = reinterpret_cast<int32_t *>(ws + L.rowptr);
  cp.refs = reinterpret_cast<int32_t *>(ws + L.refs);
  cp.entries = entries;
  cp.S = S;
  cp.S_kv = S_kv;
  cp.G = G;
  cp.topk = topk;
  // cnt and cur are adjacent: clear both with one fill kernel (graph-capture safe).
  hipLaunchKernelGGL(fill_i32_kernel, dim3(256), dim3(256), 0, st, cp.cnt,
                     (int64_t)((L.rowptr - L.cnt) / 4), 0);
  const int64_t eb = (entries + 255) / 256;
  const unsigned egrid = (unsigned)(eb < 8192 ? eb : 8192);
  hipLaunchKernelGGL(csr_count_kernel, dim3(egrid), dim3(256), 0, st, cp);
  hipLaunchKernelGGL(csr_scan_kernel, dim3(1), dim3(1024), 0, st, cp.cnt, cp.rowptr, rows);
  hipLaunchKernelGGL(csr_fill_kernel, dim3(egrid), dim3(256), 0, st, cp);
  int rc = check_launch("sparse_mla_bwd(csr)");
  if (rc) return rc;

  BwdParams p;
  p.q = static_cast<const unsigned char *>(q);
  p.kv = static_cast<const unsigned char *>(kv);
  p.o = static_cast<const uint16_t *>(o);
  p.dO = static_cast<const uint16_t *>(dO);
  p.idx = indices;
  p.lse = lse2;
  p.delta = delta;
  p.dq = static_cast<uint16_t *>(dq);
  p.q_scale = q_scale;
  p.kv_scale = kv_scale;
  p.partials = reinterpret_cast<float *>(ws + L.partials);
  p.S = S;
  p.S_kv = S_kv;
  p.H = H;
  p.G = G;
  p.topk = topk;
  p.hpg = (int)(H / G);
  plan_head_tiles(p.hpg, &p.ntiles, &p.tiles_per_wg, &p.splits, &p.wg_per_tok);
  p.sl2 = sm_scale * kLog2e;
  p.scale = sm_scale;
  const int64_t nblocks = B * S * G * p.wg_per_tok;
  DSA_REQUIRE(nblocks < (1ll << 31), "dsa_sparse_mla_bwd: grid too large");
  if (D_qk == 128 && D_v == 64) rc = f8 ? launch_bwd_main<128, 64, true>(p, nblocks, st) : launch_bwd_main<128, 64, false>(p, nblocks, st);
  else if (D_qk == 128 && D_v == 128) rc = f8 ? launch_bwd_main<128, 128, true>(p, nblocks, st) : launch_bwd_main<128, 128, false>(p, nblocks, st);
  else if (D_qk == 192 && D_v == 128) rc = f8 ? launch_bwd_main<192, 128, true>(p, nblocks, st) : launch_bwd_main<192, 128, false>(p, nblocks, st);
  else rc = launch_bwd_main<64, 32, false>(p, nblocks, st);
  if (rc) return rc;

  uint16_t *dkv16 = static_cast<uint16_t *>(dkv);
  if (D_qk == 128) hipLaunchKernelGGL(dkv_reduce_kernel<128>, dim3((unsigned)rows), dim3(256), 0, st, cp.rowptr, cp.refs, p.partials, dkv16, rows, p.ntiles);
  else if (D_qk == 192) hipLaunchKernelGGL(dkv_reduce_kernel<192>, dim3((unsigned)rows), dim3(256), 0, st, cp.rowptr, cp.refs, p.partials, dkv16, rows, p.ntiles);
  else hipLaunchKernelGGL(dkv_reduce_kernel<64>, dim3((unsigned)rows), dim3(256), 0, st, cp.rowptr, cp.refs, p.partials, dkv16, rows, p.ntiles);
  return check_launch("sparse_mla_bwd(reduce)");
}
