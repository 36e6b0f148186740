// SparseMLA forward and backward for wide heads on gfx950 (d_qk = 576 latent +
// rope with d_v = 512: the DeepSeek-V3.2 MLA row and the reference's default
// head dims; or d_v = 576, what a caller that passes no d_v gets).
//
// Reference semantics are those of the narrow kernels:
// cppmega/megatron/sparse_mla_ops/tilelang_sparse_mla_fwd.py:137-290 (fwd),
// tilelang_sparse_mla_fwd_fp8.py:187-393 (e4m3 fwd) and
// tilelang_sparse_mla_bwd.py:123-419 (bwd).
//
// A wide row does not fit one wave's registers: Q over 576 dims is 144 VGPRs
// per 32 heads and the O accumulator over 512 dims is 256.  So one workgroup of
// four waves owns one (token, kv group, 32-head tile) item and the waves split
// the head dims:
//   * the 32 kv rows of a block (36 KiB) are gathered by all 256 threads into
//     one row-major LDS tile (16-byte chunks, one block ahead in registers);
//   * S^T[slot][head] = K Q^T is split over d_qk: wave w runs k-steps
//     [w * KQ, (w + 1) * KQ) with its quarter of Q resident in registers, writes
//     its fp32 partial tile to LDS, and every wave then sums the four partials
//     in wave order, so all waves hold bit-identical scores and run the same
//     online softmax;
//   * O^T[d][head] += V^T P^T is split over d_v: wave w accumulates every
//     fourth 32-column tile of d_v, t = w + 4q (V^T read with transposing LDS
//     reads in accumulator order, P straight from registers).
// The backward (bf16 and e4m3) splits S and dP the same way, then gives each wave every
// fourth 32-column tile of d_qk for dQ^T = K^T dS^T and for the per-slot dKV
// row c^T = Q^T dS^T + dO^T P^T, written at the entry's CSR position as fp16
// scaled by a per-row power of two fixed from a bound before the products (as
// in the narrow kernels), or as fp32 with DSA_BWD_FP32_PARTIALS; the kv-major
// reduction sums those rows in a fixed order.
#include <type_traits>

#include "dsa_common.hpp"
#include "sparse_mla_gather.hpp"
#include "sparse_mla_params.hpp"
#include "sparse_mla_wide.hpp"

namespace dsa {

template <int D_QK, int D_V, bool FP8, int NTHR_ = 256>
struct WideCfg {
  static constexpr int NTHR = NTHR_;               // threads that gather a block
  static constexpr int ELT = FP8 ? 1 : 2;          // bytes per element in HBM
  static constexpr int ROWB = D_QK * ELT;          // bytes per kv row
  static constexpr int NCH = ROWB / 16;            // 16-byte chunks per row
  static constexpr int NCH_V = D_V * ELT / 16;     // chunks of the V prefix
  static constexpr int UNITS = 32 * NCH;           // (row, chunk) units per block
  static constexpr int UPT = (UNITS + NTHR - 1) / NTHR;  // units per thread
  static constexpr int KL_STRIDE = ROWB + 32;      // padded LDS row (conflict-free transposed reads)
  static constexpr int KD_STRIDE = D_V * 2 + 32;   // e4m3: dequantised V rows (bf16)
  static constexpr int KSTEPS = D_QK / 16;         // 32x32x16 k-steps over d_qk
  static constexpr int KQ = KSTEPS / 4;            // S k-steps per wave
  static constexpr int DT = D_V / 32;              // 32-column tiles of d_v
  static constexpr int DTW = (DT + 3) / 4;         // O^T tiles per wave (tile t = w + 4 q, t < DT)
  static_assert(ROWB % 16 == 0 && (D_V * ELT) % 16 == 0, "rows must be whole 16-byte chunks");
  static_assert(KSTEPS % 4 == 0 && D_V % 32 == 0 && D_V <= D_QK, "head dims must split over four waves");
  struct Regs {
    i32x4 v[UPT];
    float sc[UPT];
    uint32_t valid;  // bit i: unit i is a real (unmasked) slot's chunk
  };
};

// Issue the loads of one block's 32 rows: thread t takes units t + NTHR i,
// unit u = chunk u % NCH of row u / NCH.  my_idx is the kv row of slot
// (lane & 31) of this wave (-1: masked).
// kv_scale_b holds one scale per row (sc_pitch 1) or, MX, one per 32-channel
// block of every row (sc_pitch floats apart): a unit loads its own block's.
// UNCOND (the backward): the loads are unconditional, a unit past the block
// (or a masked slot) reading row 0, which wide_store drops, so that every wave
// issues the same loads on every block.
template <class C, bool FP8, bool MX = false, bool UNCOND = false>
__device__ __forceinline__ void wide_issue(typename C::Regs &rg, const unsigned char *kv_b, const float *kv_scale_b,
                                           int my_idx, uint32_t row_pitch, uint32_t sc_pitch = 1u) {
  const int t = threadIdx.x;
  uint32_t valid = 0;
#pragma unroll
  for (int i = 0; i < C::UPT; ++i) {
    const int u = t + C::NTHR * i;
    const int row = (u / C::NCH) & 31;
    const int c = u % C::NCH;
    const int ri = __shfl(my_idx, row, 64);
    const bool exists = (i + 1 < C::UPT) || u < C::UNITS;
    const bool ok = ri >= 0 && exists;
    const uint32_t r = ok ? (uint32_t)ri : 0u;
    if constexpr (UNCOND) {
      rg.v[i] = ld_global_16(kv_b + r * row_pitch + c * 16);
      if constexpr (FP8) rg.sc[i] = kv_scale_b[r * sc_pitch + (MX ? (uint32_t)(c >> 1) : 0u)];
    } else {
      rg.v[i] = i32x4{0, 0, 0, 0};
      if (exists) rg.v[i] = ld_global_16(kv_b + r * row_pitch + c * 16);
      if constexpr (FP8) rg.sc[i] = exists ? kv_scale_b[r * sc_pitch + (MX ? (uint32_t)(c >> 1) : 0u)] : 0.0f;
    }
    valid |= (ok ? 1u : 0u) << i;
  }
  rg.valid = valid;
}

// Store the staged rows: raw bytes row-major into Kl (masked slots zero); for
// e4m3 also the first NCH_D chunks dequantised to bf16 (value * kv_scale, RNE)
// into Kd (row stride KD_STRIDE) and the per-slot scales into Ksc (MX: the
// per-(slot, block) scales, block-major Ksc[block * 32 + slot]).
template <class C, bool FP8, int NCH_D = C::NCH_V, int KD_STRIDE = C::KD_STRIDE, bool MX = false>
__device__ __forceinline__ void wide_store(const typename C::Regs &rg, unsigned char *Kl, unsigned char *Kd,
                                           float *Ksc) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < C::UPT; ++i) {
    const int u = t + C::NTHR * i;
    if ((i + 1 < C::UPT) || u < C::UNITS) {
      const int row = u / C::NCH, c = u % C::NCH;
      const bool ok = (rg.valid >> i) & 1u;
      const i32x4 v = ok ? rg.v[i] : i32x4{0, 0, 0, 0};
      *reinterpret_cast<i32x4 *>(Kl + row * C::KL_STRIDE + c * 16) = v;
      if constexpr (FP8) {
        const float s = ok ? rg.sc[i] : 0.0f;
        if (c < NCH_D) {
          uint32_t wd[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const f32x2 v2 = e4m3x2_to_f32((uint32_t)v[e >> 1], (e & 1) != 0);
            wd[e] = pack_bf16x2(v2[0] * s, v2[1] * s);
          }
          unsigned char *dst = Kd + row * KD_STRIDE + c * 32;
          *reinterpret_cast<i32x4 *>(dst) = i32x4{(int)wd[0], (int)wd[1], (int)wd[2], (int)wd[3]};
          *reinterpret_cast<i32x4 *>(dst + 16) = i32x4{(int)wd[4], (int)wd[5], (int)wd[6], (int)wd[7]};
        }
        if constexpr (MX) {
          if ((c & 1) == 0) Ksc[(c >> 1) * 32 + row] = s;
        } else if (c == 0) {
          Ksc[row] = s;
        }
      }
    }
  }
}

// Sum of the four waves' partial 32x32 fp32 tiles (stored lane-linear per wave:
// Sp[w][q4][lane][4]) in wave order: the same bits in every wave.
__device__ __forceinline__ void sum_partials(const float *Sp, int stride_w, float (&s)[16]) {
  const int lane = lane_id();
#pragma unroll
  for (int q4 = 0; q4 < 4; ++q4) {
    const f32x4 v0 = *reinterpret_cast<const f32x4 *>(Sp + 0 * stride_w + (q4 * 64 + lane) * 4);
    const f32x4 v1 = *reinterpret_cast<const f32x4 *>(Sp + 1 * stride_w + (q4 * 64 + lane) * 4);
    const f32x4 v2 = *reinterpret_cast<const f32x4 *>(Sp + 2 * stride_w + (q4 * 64 + lane) * 4);
    const f32x4 v3 = *reinterpret_cast<const f32x4 *>(Sp + 3 * stride_w + (q4 * 64 + lane) * 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) s[4 * q4 + j] = ((v0[j] + v1[j]) + v2[j]) + v3[j];
    __builtin_amdgcn_sched_barrier(0);  // bound the loads in flight (register pressure)
  }
}

// Split form of sum_partials for four waves: wave w sums quarter w (64 lanes x
// 4 floats) of the four partial tiles in the same order and writes it to the
// reduced tile Sr; after a barrier every wave reads the whole reduced tile
// (get_reduced), so each reads 8 KiB of LDS instead of 16.
__device__ __forceinline__ void reduce_quarter(const float *Sp, int stride_w, float *Sr, int w) {
  const int lane = lane_id();
  const f32x4 v0 = *reinterpret_cast<const f32x4 *>(Sp + 0 * stride_w + (w * 64 + lane) * 4);
  const f32x4 v1 = *reinterpret_cast<const f32x4 *>(Sp + 1 * stride_w + (w * 64 + lane) * 4);
  const f32x4 v2 = *reinterpret_cast<const f32x4 *>(Sp + 2 * stride_w + (w * 64 + lane) * 4);
  const f32x4 v3 = *reinterpret_cast<const f32x4 *>(Sp + 3 * stride_w + (w * 64 + lane) * 4);
  f32x4 r;
#pragma unroll
  for (int j = 0; j < 4; ++j) r[j] = ((v0[j] + v1[j]) + v2[j]) + v3[j];
  *reinterpret_cast<f32x4 *>(Sr + (w * 64 + lane) * 4) = r;
}
__device__ __forceinline__ void get_reduced(const float *Sr, float (&s)[16]) {
  const int lane = lane_id();
#pragma unroll
  for (int q4 = 0; q4 < 4; ++q4) {
    const f32x4 v = *reinterpret_cast<const f32x4 *>(Sr + (q4 * 64 + lane) * 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) s[4 * q4 + j] = v[j];
  }
}

__device__ __forceinline__ void put_partial(float *dst, const f32x16 &acc) {
  const int lane = lane_id();
#pragma unroll
  for (int q4 = 0; q4 < 4; ++q4)
    *reinterpret_cast<f32x4 *>(dst + (q4 * 64 + lane) * 4) =
        f32x4{acc[4 * q4], acc[4 * q4 + 1], acc[4 * q4 + 2], acc[4 * q4 + 3]};
}

// ---------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------
template <int D_QK, int D_V, bool FP8, bool MX = false, int NT = 1>
struct WideFwdLds {
  using C = WideCfg<D_QK, D_V, FP8, 256 * NT>;
  static constexpr int NBLK = D_QK / 32;  // MX scale blocks per row
  static constexpr int OFF_KL = 0;
  static constexpr int OFF_KD = OFF_KL + 32 * C::KL_STRIDE;
  static constexpr int OFF_SC = OFF_KD + (FP8 ? 32 * C::KD_STRIDE : 0);
  static constexpr int OFF_SP = (OFF_SC + (FP8 ? (MX ? NBLK : 1) * 32 * 4 : 0) + 15) / 16 * 16;
  static constexpr int SP_W = 16 * 64;  // floats per wave's partial tile
  static constexpr int OFF_SR = OFF_SP + 4 * NT * SP_W * 4;  // a partial tile per wave
  static constexpr int BYTES = OFF_SR + NT * SP_W * 4;       // a reduced tile per head tile
};

// MX partial scores of one wave over its k-steps [k0, k0 + KQ) of d_qk (k0 of
// parity PAR): every 32-channel block (two k-steps; the wave's first or last
// block may be a half that the neighbouring wave completes) accumulates a fresh
// partial on the e4m3 codes, scaled by kv_scale[slot][block] * q_scale[head][block]
// before it joins sacc.  The block scaling is linear, so the four waves'
// partials still sum to the full score.
template <class C, int PAR>
__device__ __forceinline__ void mx_wave_scores(f32x16 &sacc, const unsigned char *Kl, const long (&qreg)[C::KQ],
                                               const float (&qbs)[C::KQ / 2 + 1], const float *Ksc, int k0,
                                               int l32, int g32) {
  const int cb0 = (k0 - PAR) >> 1;  // first block this wave touches
  f32x16 part;
#pragma unroll
  for (int a = 0; a < 16; ++a) part[a] = 0.0f;
#pragma unroll
  for (int k = 0; k < C::KQ; ++k) {
    const long a = *reinterpret_cast<const long *>(Kl + l32 * C::KL_STRIDE + 16 * (k0 + k) + 8 * g32);
    part = __builtin_amdgcn_mfma_f32_32x32x16_fp8_fp8(a, qreg[k], part, 0, 0, 0);
    if (((k + PAR) & 1) || k == C::KQ - 1) {  // the block of k-step k0 + k ends here (for this wave)
      const int cl = (k + PAR) >> 1;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x4 k4 = *reinterpret_cast<const f32x4 *>(Ksc + (cb0 + cl) * 32 + 8 * i + 4 * g32);
#pragma unroll
        for (int j = 0; j < 4; ++j) sacc[4 * i + j] = fmaf(part[4 * i + j], k4[j] * qbs[cl], sacc[4 * i + j]);
      }
#pragma unroll
      for (int a = 0; a < 16; ++a) part[a] = 0.0f;
    }
  }
}

// NT head tiles per workgroup: waves 4 ht .. 4 ht + 3 own 32-head tile ht of
// the item and split its head dims as described above; all 4 NT waves gather
// (and, e4m3, dequantise) the block's kv rows once for the NT tiles.  QMX: the
// bf16 kernel with Q given as e4m3 codes and one scale per 32 channels,
// converted to bf16 as it is loaded.
template <int D_QK, int D_V, bool FP8, bool MX = false, int NT = 1, bool QMX = false>
__global__ void __launch_bounds__(256 * NT) __attribute__((amdgpu_waves_per_eu(D_V <= 512 ? 2 : 1)))
sparse_mla_fwd_wide_kernel(const FwdParams p) {
  static_assert(!MX || FP8, "MX is an e4m3 mode");
  static_assert(!QMX || !FP8, "QMX converts Q for the bf16 kernel");
  if (p.gate != nullptr && *p.gate != p.gate_run) return;  // workgroup-uniform: the call's other kernel computes it
  using C = WideCfg<D_QK, D_V, FP8, 256 * NT>;
  using L = WideFwdLds<D_QK, D_V, FP8, MX, NT>;
  typedef typename std::conditional<FP8, long, bf16x8>::type qop_t;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

  const int lane = lane_id(), wv = __builtin_amdgcn_readfirstlane(wave_id());
  const int ht = wv >> 2, w = wv & 3;  // head tile within the item, wave within the tile
  const int g32 = lane >> 5, l32 = lane & 31;
  const int64_t item = xcd_remap(blockIdx.x, gridDim.x);
  const int ntg = (p.ntiles + NT - 1) / NT;  // items per (token, kv group)
  const int tile = (int)(item % ntg) * NT + ht;
  const int64_t rest = item / ntg;
  const int64_t g = rest % p.G;
  const int64_t tok = rest / p.G;
  const int64_t b = tok / p.S;

  unsigned char *Kl = smem + L::OFF_KL;
  unsigned char *Kd = smem + L::OFF_KD;
  float *Ksc = reinterpret_cast<float *>(smem + L::OFF_SC);
  float *Sp = reinterpret_cast<float *>(smem + L::OFF_SP);
  float *Sr = reinterpret_cast<float *>(smem + L::OFF_SR) + ht * L::SP_W;
  const unsigned char *Vsrc = FP8 ? Kd : Kl;
  constexpr int V_STRIDE = FP8 ? C::KD_STRIDE : C::KL_STRIDE;

  const int h_local = tile * 32 + l32;
  const bool head_ok = h_local < p.hpg;
  const int64_t qrow = tok * p.H + g * p.hpg + h_local;
  const int32_t *idx_row = p.idx + (tok * p.G + g) * p.topk;
  const unsigned char *kv_b = p.kv + ((b * p.S_kv) * p.G + g) * C::ROWB;
  // kv scales: [B, S_kv] per row, or MX [B, S_kv, G, D_QK / 32] per (row, block)
  const float *kv_scale_b = !FP8 ? nullptr : (MX ? p.kv_scale + ((b * p.S_kv) * p.G + g) * L::NBLK
                                                 : p.kv_scale + b * p.S_kv);
  const uint32_t sc_pitch = MX ? (uint32_t)(p.G * L::NBLK) : 1u;
  const uint32_t row_pitch = (uint32_t)(p.G * C::ROWB);
  const int nblk = (int)((p.topk + 31) / 32);

  // indices two blocks ahead as raw loads, masked where they are used a block
  // later: the block loop never waits on an index load it has just issued
  const auto idx_rs = slot_rsrc(idx_row, p.topk);
  int idx_cur = slot_index(load_slot_raw(idx_rs, 0, l32), 0, l32, p.topk, p.S_kv);
  int raw_nxt = load_slot_raw(idx_rs, 1, l32);
  typename C::Regs rg;
  wide_issue<C, FP8, MX>(rg, kv_b, kv_scale_b, idx_cur, row_pitch, sc_pitch);

  // this wave's quarter of Q as the B operand: lane = head, 8 consecutive d per k-step
  const int k0 = w * C::KQ;
  qop_t qreg[C::KQ];
#pragma unroll
  for (int k = 0; k < C::KQ; ++k) {
    if constexpr (FP8) {
      qreg[k] = head_ok ? *reinterpret_cast<const long *>(p.q + qrow * D_QK + 16 * (k0 + k) + 8 * g32) : 0l;
    } else if constexpr (QMX) {
      const int d0 = 16 * (k0 + k) + 8 * g32;  // 8 channels of block d0 / 32
      uint2 c8 = {0u, 0u};
      float sc = 0.0f;
      if (head_ok) {
        c8 = *reinterpret_cast<const uint2 *>(p.q + qrow * D_QK + d0);
        sc = p.q_scale[qrow * (D_QK / 32) + (d0 >> 5)];
      }
      qreg[k] = e4m3x8_to_bf16_scaled(c8.x, c8.y, sc);
    } else {
      i32x4 v = {0, 0, 0, 0};
      if (head_ok) v = ld_global_16(p.q + (qrow * D_QK + 16 * (k0 + k) + 8 * g32) * 2);
      qreg[k] = as_bf16x8(v);
    }
  }
  float qsc = 1.0f;
  if constexpr (FP8 && !MX) qsc = p.q_scale[tok];
  const float tscale = p.sl2 * qsc;
  // MX: this lane's head's scales of the blocks this wave's k-steps touch
  // (q_scale [B, S, H, D_QK / 32])
  const int par = (k0 & 1);
  float qbs[C::KQ / 2 + 1];
  if constexpr (MX) {
    const int cb0 = (k0 - par) >> 1;
#pragma unroll
    for (int cl = 0; cl < C::KQ / 2 + 1; ++cl)
      qbs[cl] = (head_ok && cb0 + cl < L::NBLK) ? p.q_scale[qrow * L::NBLK + cb0 + cl] : 0.0f;
  }

  float m_run = kNegBig, l_run = 0.0f;
  f32x16 oacc[C::DTW];
#pragma unroll
  for (int t = 0; t < C::DTW; ++t)
#pragma unroll
    for (int a = 0; a < 16; ++a) oacc[t][a] = 0.0f;

  for (int blk = 0; blk < nblk; ++blk) {
    wide_store<C, FP8, C::NCH_V, C::KD_STRIDE, MX>(rg, Kl, Kd, Ksc);
    const uint64_t vmask = __ballot(idx_cur >= 0);
    __syncthreads();  // the block's rows are in LDS
    const int raw_nn = load_slot_raw(idx_rs, blk + 2, l32);
    const int idx_nxt = slot_index(raw_nxt, blk + 1, l32, p.topk, p.S_kv);
    if (blk + 1 < nblk) wide_issue<C, FP8, MX>(rg, kv_b, kv_scale_b, idx_nxt, row_pitch, sc_pitch);

    // ---- partial S^T = K Q^T over this wave's k-steps ----
    f32x16 sacc;
#pragma unroll
    for (int a = 0; a < 16; ++a) sacc[a] = 0.0f;
    if constexpr (MX) {
      if (par) mx_wave_scores<C, 1>(sacc, Kl, qreg, qbs, Ksc, k0, l32, g32);
      else mx_wave_scores<C, 0>(sacc, Kl, qreg, qbs, Ksc, k0, l32, g32);
    }
#pragma unroll
    for (int k = 0; k < (MX ? 0 : C::KQ); ++k) {
      if constexpr (FP8) {
        const long a = *reinterpret_cast<const long *>(Kl + l32 * C::KL_STRIDE + 16 * (k0 + k) + 8 * g32);
        sacc = __builtin_amdgcn_mfma_f32_32x32x16_fp8_fp8(a, qreg[k], sacc, 0, 0, 0);
      } else {
        const i32x4 a = *reinterpret_cast<const i32x4 *>(Kl + l32 * C::KL_STRIDE + (16 * (k0 + k) + 8 * g32) * 2);
        sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), qreg[k], sacc, 0, 0, 0);
      }
    }
    put_partial(Sp + wv * L::SP_W, sacc);
    __syncthreads();  // all partial tiles written
    reduce_quarter(Sp + 4 * ht * L::SP_W, L::SP_W, Sr, w);
    __syncthreads();  // the head tile's reduced scores are whole
    float s[16];
    get_reduced(Sr, s);

    // ---- online softmax (log2 domain, lazy rescale; identical in every wave) ----
    // this lane's slots are 8i + 4*g32 + j: their valid bits sit at 8i + j of lmask;
    // a block without masked slots (the common case, wave-uniform) skips the tests
    const bool all_valid = (uint32_t)vmask == 0xffffffffu;
    const uint32_t lmask = (uint32_t)vmask >> (4 * g32);
    float xs[16];
    float mloc = kNegBig;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float ksc4[4] = {1.0f, 1.0f, 1.0f, 1.0f};
      if constexpr (FP8 && !MX) {
        const f32x4 s4 = *reinterpret_cast<const f32x4 *>(Ksc + 8 * i + 4 * g32);
        ksc4[0] = s4[0]; ksc4[1] = s4[1]; ksc4[2] = s4[2]; ksc4[3] = s4[3];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float v = s[4 * i + j];
        if constexpr (FP8 && !MX) v *= ksc4[j];
        xs[4 * i + j] = v;  // raw score, scaled inside the exp
      }
    }
    if (!all_valid) {
#pragma unroll
      for (int a = 0; a < 16; ++a)
        if (!((lmask >> (8 * (a >> 2) + (a & 3))) & 1u)) xs[a] = -INFINITY;
    }
#pragma unroll
    for (int a = 0; a < 16; a += 2) mloc = fmaxf(mloc, fmaxf(xs[a], xs[a + 1]));
    mloc = max_halves(mloc) * tscale;
    if (__ballot(mloc > m_run + 8.0f) != 0ull) {
      const float m_new = fmaxf(m_run, mloc);
      const float alpha = exp2_fast(m_run - m_new);
      l_run *= alpha;
      m_run = m_new;
#pragma unroll
      for (int dt = 0; dt < C::DTW; ++dt)
#pragma unroll
        for (int a = 0; a < 16; ++a) oacc[dt][a] *= alpha;
    }
    float t[16];
    float lsum = 0.0f;
#pragma unroll
    for (int a = 0; a < 16; ++a) {
      t[a] = exp2_fast(fmaf(xs[a], tscale, -m_run));
      lsum += t[a];
    }
    lsum = sum_halves(lsum);
    l_run += lsum;

    // ---- O^T[d][head] += V^T[d][slot] P^T[slot][head] on this wave's d_v tiles ----
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      i32x4 pb;
#pragma unroll
      for (int e = 0; e < 4; ++e) pb[e] = (int)pack_bf16x2(t[8 * kc + 2 * e], t[8 * kc + 2 * e + 1]);
      const bf16x8 bop = as_bf16x8(pb);
#pragma unroll
      for (int dt = 0; dt < C::DTW; ++dt) {
        const int tv = w + 4 * dt;
        if (tv < C::DT) {
          const i32x4 av = tr_operand(Vsrc, V_STRIDE, tv * 32, 16 * kc, 8, 4);
          oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(av), bop, oacc[dt], 0, 0, 0);
        }
      }
    }
    __syncthreads();  // rows and partial tiles consumed before the next block overwrites them
    idx_cur = idx_nxt;
    raw_nxt = raw_nn;
  }

  // ---- normalise and write: lane = head l32, d = (w + 4*dt)*32 + 8i + 4*g32 + j ----
  if (head_ok) {
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    uint16_t *orow = p.out + qrow * D_V;
#pragma unroll
    for (int dt = 0; dt < C::DTW; ++dt) {
      const int tv = w + 4 * dt;
      if (tv < C::DT) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const i32x2 pk = {(int)pack_bf16x2(oacc[dt][4 * i] * inv, oacc[dt][4 * i + 1] * inv),
                            (int)pack_bf16x2(oacc[dt][4 * i + 2] * inv, oacc[dt][4 * i + 3] * inv)};
          *reinterpret_cast<i32x2 *>(orow + tv * 32 + 8 * i + 4 * g32) = pk;
        }
      }
    }
    if (w == 0 && g32 == 0) p.lse[qrow] = l_run > 0.0f ? log2f(l_run) + m_run : -INFINITY;
  }
}

template <int D_QK, int D_V, bool FP8, bool MX, int NT, bool QMX = false>
static int launch_fwd_wide_nt(const FwdParams &p, hipStream_t st) {
  using L = WideFwdLds<D_QK, D_V, FP8, MX, NT>;
  const size_t lds = L::BYTES;
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute((const void *)sparse_mla_fwd_wide_kernel<D_QK, D_V, FP8, MX, NT, QMX>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return set_error(DSA_ERR_HIP, "sparse_mla_fwd(wide): LDS attribute: %s", hipGetErrorString(e));
  }
  const int64_t nitems = p.B * p.S * p.G * ((p.ntiles + NT - 1) / NT);  // one workgroup per item
  if (nitems >= (1ll << 31)) return set_error(DSA_ERR_INVALID_ARG, "sparse_mla_fwd(wide): grid too large");
  hipLaunchKernelGGL((sparse_mla_fwd_wide_kernel<D_QK, D_V, FP8, MX, NT, QMX>), dim3((unsigned)nitems), dim3(256 * NT),
                     lds, st, p);
  return check_launch("sparse_mla_fwd(wide)");
}

// Two head tiles per workgroup when a kv group has at least 64 heads (the
// gather and dequantisation of a block serve both), else one.
template <int D_QK, int D_V, bool FP8, bool MX = false, bool QMX = false>
static int launch_fwd_wide_t(const FwdParams &p, hipStream_t st) {
  return p.ntiles >= 2 ? launch_fwd_wide_nt<D_QK, D_V, FP8, MX, 2, QMX>(p, st)
                       : launch_fwd_wide_nt<D_QK, D_V, FP8, MX, 1, QMX>(p, st);
}

int launch_fwd_wide(const FwdParams &p, int64_t d_qk, int64_t d_v, bool fp8, hipStream_t st, bool mx, bool qmx) {
  if (qmx) {
    if (d_qk == 576 && d_v == 512) return launch_fwd_wide_t<576, 512, false, false, true>(p, st);
    return set_error(DSA_ERR_UNSUPPORTED, "sparse_mla_fwd(wide): no converted-Q kernel for d_qk=%lld d_v=%lld",
                     (long long)d_qk, (long long)d_v);
  }
  if (mx) {
    if (d_qk == 576 && d_v == 512) return launch_fwd_wide_t<576, 512, true, true>(p, st);
    return set_error(DSA_ERR_UNSUPPORTED, "sparse_mla_fwd(wide): no MXFP8 kernel for d_qk=%lld d_v=%lld",
                     (long long)d_qk, (long long)d_v);
  }
  if (d_qk == 576 && d_v == 512) return fp8 ? launch_fwd_wide_t<576, 512, true>(p, st) : launch_fwd_wide_t<576, 512, false>(p, st);
  if (d_qk == 576 && d_v == 576) return fp8 ? launch_fwd_wide_t<576, 576, true>(p, st) : launch_fwd_wide_t<576, 576, false>(p, st);
  return set_error(DSA_ERR_UNSUPPORTED, "sparse_mla_fwd(wide): no kernel for d_qk=%lld d_v=%lld", (long long)d_qk,
                   (long long)d_v);
}

// ---------------------------------------------------------------------------
// Backward main pass (bf16 and e4m3)
// ---------------------------------------------------------------------------
// LDS of one workgroup: QL [head][d] and DOL [head][d] (bf16; e4m3 Q
// dequantised, for the S / dP A operands and the transposed Q^T / dO^T
// operands), LD = LSE (heads 0..31) and Delta * sm_scale (32..63), Kl [slot][d]
// gathered rows (raw bytes), for e4m3 also Kd [slot][d] (rows dequantised to
// bf16, the V and K operands of dP and dQ) and Ksc (row scales), the waves'
// partial score tiles, and one dS[slot][head] tile per wave.  bf16 exchanges
// the S and dP partials together (8 tiles); e4m3 has room for four and
// exchanges them one after the other, as the reference's e4m3 kernel computes
// QK^T on the codes and the other products on dequantised bf16.
template <int D_QK, int D_V, bool FP8>
struct WideBwdLds {
  // (after DS) MX: per-wave max |Q| (0..3) and max |dO| (4..7) of the item
  using C = WideCfg<D_QK, D_V, FP8>;
  static constexpr int QL_STRIDE = D_QK * 2 + 32;
  static constexpr int DOL_STRIDE = D_V * 2 + 32;
  static constexpr int DS_STRIDE = 32 * 2 + 32;
  static constexpr int KDB_STRIDE = D_QK * 2 + 32;  // e4m3: whole rows dequantised
  static constexpr int OFF_QL = 0;
  static constexpr int OFF_DOL = OFF_QL + 32 * QL_STRIDE;
  static constexpr int OFF_LD = OFF_DOL + 32 * DOL_STRIDE;
  static constexpr int OFF_KL = OFF_LD + 64 * 4;
  static constexpr int OFF_KD = OFF_KL + 32 * C::KL_STRIDE;
  static constexpr int OFF_SC = OFF_KD + (FP8 ? 32 * KDB_STRIDE : 0);
  static constexpr int OFF_SP = OFF_SC + (FP8 ? 32 * 4 : 0);
  static constexpr int SP_W = 16 * 64;  // floats per partial tile
  static constexpr int SP_TILES = FP8 ? 4 : 8;
  static constexpr int OFF_DS = OFF_SP + SP_TILES * SP_W * 4;
  static constexpr int OFF_MX = OFF_DS + 4 * 32 * DS_STRIDE;
  static constexpr int BYTES = OFF_MX + 8 * 4;
  static_assert(BYTES <= 160 * 1024, "wide backward LDS");
};

template <int D_QK, int D_V, bool FP8, bool F32P>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1)))
sparse_mla_bwd_wide_kernel(const BwdParams p) {
  using C = WideCfg<D_QK, D_V, FP8>;
  using L = WideBwdLds<D_QK, D_V, FP8>;
  constexpr int DQT = D_QK / 32;          // 32-column tiles of d_qk
  constexpr int DQW = (DQT + 3) / 4;      // tiles per wave (tile t = w + 4 q)
  constexpr int DVT = D_V / 32;
  constexpr int VQ = D_V / 16 / 4;        // dP k-steps per wave
  static_assert((D_V / 16) % 4 == 0, "d_v k-steps split over four waves");
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

  const int lane = lane_id(), w = __builtin_amdgcn_readfirstlane(wave_id());
  const int g32 = lane >> 5, l32 = lane & 31;
  const int64_t item = xcd_remap(blockIdx.x, gridDim.x);
  const int tile = (int)(item % p.ntiles);
  const int64_t rest = item / p.ntiles;
  const int64_t g = rest % p.G;
  const int64_t tok = rest / p.G;
  const int64_t b = tok / p.S;

  unsigned char *QL = smem + L::OFF_QL;
  unsigned char *DOL = smem + L::OFF_DOL;
  float *LD = reinterpret_cast<float *>(smem + L::OFF_LD);
  unsigned char *Kl = smem + L::OFF_KL;
  unsigned char *Kd = smem + L::OFF_KD;
  float *Ksc = reinterpret_cast<float *>(smem + L::OFF_SC);
  float *Sp = reinterpret_cast<float *>(smem + L::OFF_SP);
  const unsigned char *Ksrc = FP8 ? Kd : Kl;  // bf16 K / V rows for dP and dQ
  constexpr int K_STRIDE = FP8 ? L::KDB_STRIDE : C::KL_STRIDE;
  unsigned char *DS = smem + L::OFF_DS + w * 32 * L::DS_STRIDE;
  float *MX = reinterpret_cast<float *>(smem + L::OFF_MX);

  const int64_t head0 = tok * p.H + g * p.hpg + tile * 32;
  const int nheads = p.hpg - tile * 32 < 32 ? p.hpg - tile * 32 : 32;
  const int64_t entry0 = (tok * p.G + g) * p.topk;
  const int64_t n_entries = p.B * p.S * p.G * p.topk;
  const int32_t *idx_row = p.idx + entry0;
  const unsigned char *kv_b = p.kv + ((b * p.S_kv) * p.G + g) * C::ROWB;
  const float *kv_scale_b = FP8 ? p.kv_scale + b * p.S_kv : nullptr;
  const uint32_t row_pitch = (uint32_t)(p.G * C::ROWB);

  // Indices (two blocks ahead), rows and CSR positions (one block ahead) are
  // loaded unconditionally through resources that end at the item's top-k, and
  // every partial-row store is unconditional (masked slots write the trash row
  // past the entries), so each wave issues the same memory operations on every
  // block and the compiler's waits count exactly: waiting for a block's rows
  // or positions leaves the previous block's stores in flight.
  const auto idx_rs = slot_rsrc(idx_row, p.topk);
  const auto pos_rs = slot_rsrc(p.pos_of + entry0, p.topk);
  int idx_cur = slot_index(load_slot_raw(idx_rs, 0, l32), 0, l32, p.topk, p.S_kv);
  int raw_nxt = load_slot_raw(idx_rs, 1, l32);
  typename C::Regs rg;
  wide_issue<C, FP8, false, true>(rg, kv_b, kv_scale_b, idx_cur, row_pitch);
  int pos_cur = load_slot_raw(pos_rs, 0, l32);
  // blocks up to the last valid slot: the same count in every wave (the loop has workgroup barriers)
  const int nblk = valid_blocks(idx_rs, p.topk, p.S_kv);
  // partial row no entry owns (this workgroup's trash row)
  const uint64_t trash = (uint64_t)n_entries * (uint64_t)p.ntiles + (uint64_t)(item % kTrashRows);

  float qsc = 1.0f;
  if constexpr (FP8) qsc = p.q_scale[tok];
  // ---------------- prologue: Q, dO tiles, LSE, Delta ----------------
  {
    const int t = threadIdx.x;
    constexpr int QCH = D_QK / 8;
    float mq = 0.0f, md = 0.0f;  // max |Q|, |dO| seen by this thread (fp16 rows only)
    for (int u = t; u < 32 * QCH; u += 256) {
      const int h = u / QCH, c = u % QCH;
      i32x4 v = {0, 0, 0, 0};
      if (h < nheads) {
        if constexpr (FP8) {
          const unsigned long raw = *reinterpret_cast<const unsigned long *>(p.q + (head0 + h) * D_QK + 8 * c);
          uint32_t wq[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {  // codes 2e, 2e + 1 of the 8 in raw
            const f32x2 v2 = e4m3x2_to_f32((uint32_t)(raw >> (32 * (e >> 1))), (e & 1) != 0);
            wq[e] = pack_bf16x2(v2[0] * qsc, v2[1] * qsc);
          }
          v = i32x4{(int)wq[0], (int)wq[1], (int)wq[2], (int)wq[3]};
        } else {
          v = ld_global_16(p.q + ((head0 + h) * D_QK + 8 * c) * 2);
        }
      }
      *reinterpret_cast<i32x4 *>(QL + h * L::QL_STRIDE + c * 16) = v;
      if constexpr (!F32P) mq = fmaxf(mq, bf16x8_absmax(v));
    }
    // dO rows and Delta = sum_d O dO: one wave per head, lane = 8-element chunk
    constexpr int VCH = D_V / 8;
    for (int h = w; h < 32; h += 4) {
      float part = 0.0f;
      for (int c = lane; c < VCH; c += 64) {
        i32x4 dv = {0, 0, 0, 0}, ov = {0, 0, 0, 0};
        if (h < nheads) {
          dv = ld_global_16(p.dO + (head0 + h) * D_V + 8 * c);
          ov = ld_global_16(p.o + (head0 + h) * D_V + 8 * c);
        }
        *reinterpret_cast<i32x4 *>(DOL + h * L::DOL_STRIDE + c * 16) = dv;
        if constexpr (!F32P) md = fmaxf(md, bf16x8_absmax(dv));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t du = (uint32_t)dv[e], ou = (uint32_t)ov[e];
          part += bf16_bits_to_f32(ou & 0xffffu) * bf16_bits_to_f32(du & 0xffffu);
          part += bf16_bits_to_f32(ou >> 16) * bf16_bits_to_f32(du >> 16);
        }
      }
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) part += __shfl_xor(part, off, 64);
      if (lane == 0) {
        float dl = part;
        if (p.delta != nullptr && h < nheads) dl = p.delta[head0 + h];
        LD[32 + h] = dl * p.scale;
      }
    }
    if (t < 32) {
      float lse_h = INFINITY;  // padded heads: P = exp2(x - inf) = 0
      if (t < nheads) {
        const float l = p.lse[head0 + t];
        lse_h = (l == -INFINITY) ? INFINITY : l;  // all-masked row: zero gradient
      }
      LD[t] = lse_h;
    }
    if constexpr (!F32P) {
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) {
        mq = fmaxf(mq, __shfl_xor(mq, off, 64));
        md = fmaxf(md, __shfl_xor(md, off, 64));
      }
      if (lane == 0) {
        MX[w] = mq;
        MX[4 + w] = md;
      }
    }
  }

  // e4m3: this wave's quarter of the raw Q codes, the A operand of QK^T (head l32)
  long qA8[FP8 ? C::KQ : 1];
  if constexpr (FP8) {
#pragma unroll
    for (int k = 0; k < C::KQ; ++k)
      qA8[k] = l32 < nheads ? *reinterpret_cast<const long *>(p.q + (head0 + l32) * D_QK + 16 * (w * C::KQ + k) + 8 * g32)
                            : 0l;
  }
  f32x16 dqacc[DQW];
#pragma unroll
  for (int q = 0; q < DQW; ++q)
#pragma unroll
    for (int a = 0; a < 16; ++a) dqacc[q][a] = 0.0f;

  const int k0 = w * C::KQ, v0 = w * VQ;
  // the first block's rows and positions have landed: nothing is in flight on
  // entry, so the loop's waits follow its own order (s_waitcnt vmcnt(0) with
  // expcnt and lgkmcnt left open, gfx9 encoding)
  __builtin_amdgcn_s_waitcnt(0x0F70);
  for (int blk = 0; blk < nblk; ++blk) {
    const int slot0 = blk * 32;
    wide_store<C, FP8, C::NCH, L::KDB_STRIDE>(rg, Kl, Kd, Ksc);
    const bool valid = idx_cur >= 0;  // slot slot0 + l32
    const int32_t pos = pos_cur;
    const bool wr = valid && pos >= 0 && pos < n_entries;  // (always true for a valid slot; a guard)
    __syncthreads();  // rows (and, on the first block, the prologue tiles) are in LDS
    const int raw_nn = load_slot_raw(idx_rs, blk + 2, l32);
    const int idx_nxt = slot_index(raw_nxt, blk + 1, l32, p.topk, p.S_kv);
    wide_issue<C, FP8, false, true>(rg, kv_b, kv_scale_b, idx_nxt, row_pitch);  // past the last block too
    const int pos_nxt = load_slot_raw(pos_rs, blk + 1, l32);

    // ---- partial S = Q K^T and dP = dO V^T (M = head, N = slot) over this wave's k-steps ----
    f32x16 sacc, dpacc;
#pragma unroll
    for (int a = 0; a < 16; ++a) {
      sacc[a] = 0.0f;
      dpacc[a] = 0.0f;
    }
#pragma unroll
    for (int k = 0; k < C::KQ; ++k) {
      const int d0 = 16 * (k0 + k) + 8 * g32;
      if constexpr (FP8) {
        const long kb = *reinterpret_cast<const long *>(Kl + l32 * C::KL_STRIDE + d0);
        sacc = __builtin_amdgcn_mfma_f32_32x32x16_fp8_fp8(qA8[k], kb, sacc, 0, 0, 0);
      } else {
        const i32x4 qa = *reinterpret_cast<const i32x4 *>(QL + l32 * L::QL_STRIDE + d0 * 2);
        const i32x4 kb = *reinterpret_cast<const i32x4 *>(Kl + l32 * C::KL_STRIDE + d0 * 2);
        sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(qa), as_bf16x8(kb), sacc, 0, 0, 0);
      }
    }
#pragma unroll
    for (int k = 0; k < VQ; ++k) {
      const int d0 = 16 * (v0 + k) + 8 * g32;
      const i32x4 da = *reinterpret_cast<const i32x4 *>(DOL + l32 * L::DOL_STRIDE + d0 * 2);
      const i32x4 vb = *reinterpret_cast<const i32x4 *>(Ksrc + l32 * K_STRIDE + d0 * 2);
      dpacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(da), as_bf16x8(vb), dpacc, 0, 0, 0);
    }
    float s[16], dp[16];
    if constexpr (FP8) {
      put_partial(Sp + w * L::SP_W, sacc);
      __syncthreads();  // S partial tiles written
      sum_partials(Sp, L::SP_W, s);
      __syncthreads();  // read before the dP partials reuse the tiles
      put_partial(Sp + w * L::SP_W, dpacc);
      __syncthreads();
      sum_partials(Sp, L::SP_W, dp);
    } else {
      put_partial(Sp + (2 * w) * L::SP_W, sacc);
      put_partial(Sp + (2 * w + 1) * L::SP_W, dpacc);
      __syncthreads();  // all partial tiles written
      sum_partials(Sp, 2 * L::SP_W, s);
      sum_partials(Sp + L::SP_W, 2 * L::SP_W, dp);
    }

    // ---- P, dS (lane = slot slot0 + l32, heads 8i + 4*g32 + j; identical in every wave) ----
    float xs = p.sl2;
    if constexpr (FP8) xs *= qsc * Ksc[l32];
    bf16x8 dsB[2], pB[2];
    int pexp = 0;  // fp16 rows: the slot's partial-row scale exponent (identical in every wave)
    {
      uint32_t dsw[8], pw[8];
      float P[16], dS[16];
      float sabs = 0.0f, psum = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x4 l4 = *reinterpret_cast<const f32x4 *>(LD + 8 * i + 4 * g32);
        const f32x4 d4 = *reinterpret_cast<const f32x4 *>(LD + 32 + 8 * i + 4 * g32);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int a = 4 * i + j;
          const float pv = valid ? exp2_fast(s[a] * xs - l4[j]) : 0.0f;
          P[a] = pv;
          dS[a] = pv * fmaf(dp[a], p.scale, -d4[j]);
          sabs += fabsf(dS[a]);
          psum += pv;
        }
        dsw[2 * i] = pack_bf16x2(dS[4 * i], dS[4 * i + 1]);
        dsw[2 * i + 1] = pack_bf16x2(dS[4 * i + 2], dS[4 * i + 3]);
        *reinterpret_cast<i32x2 *>(DS + l32 * L::DS_STRIDE + (8 * i + 4 * g32) * 2) =
            i32x2{(int)dsw[2 * i], (int)dsw[2 * i + 1]};
      }
      float rs = 1.0f;
      if constexpr (!F32P) {
        // |c[d]| <= max|Q| sum_h |dS_h| + max|dO| sum_h P_h over the slot's 32
        // heads; the margin 2^-6 covers the bf16 rounding of dS / P (2^-8) and
        // the fp32 sums.  c is computed from dS 2^s and P 2^s (exact scalings).
        const float maxq = fmaxf(fmaxf(MX[0], MX[1]), fmaxf(MX[2], MX[3]));
        const float maxdo = fmaxf(fmaxf(MX[4], MX[5]), fmaxf(MX[6], MX[7]));
        const float bnd = sum_halves(fmaf(maxq, sabs, maxdo * psum)) * 1.015625f;
        pexp = partial_row_exponent_bound(bnd);
        rs = exp2i(pexp);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          dsw[2 * i] = pack_bf16x2(dS[4 * i] * rs, dS[4 * i + 1] * rs);
          dsw[2 * i + 1] = pack_bf16x2(dS[4 * i + 2] * rs, dS[4 * i + 3] * rs);
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pw[2 * i] = pack_bf16x2(P[4 * i] * rs, P[4 * i + 1] * rs);
        pw[2 * i + 1] = pack_bf16x2(P[4 * i + 2] * rs, P[4 * i + 3] * rs);
      }
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        dsB[kc] = as_bf16x8(i32x4{(int)dsw[4 * kc], (int)dsw[4 * kc + 1], (int)dsw[4 * kc + 2], (int)dsw[4 * kc + 3]});
        pB[kc] = as_bf16x8(i32x4{(int)pw[4 * kc], (int)pw[4 * kc + 1], (int)pw[4 * kc + 2], (int)pw[4 * kc + 3]});
      }
    }
    wave_lds_sync();  // this wave's dS tile

    // ---- dQ^T[d][head] += K^T[d][slot] dS^T[slot][head] on tiles t = w + 4q ----
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      const i32x4 bv = tr_operand(DS, L::DS_STRIDE, 0, 16 * kc, 4, 8);
#pragma unroll
      for (int q = 0; q < DQW; ++q) {
        const int t = w + 4 * q;
        if (t < DQT) {
          const i32x4 av = tr_operand(Ksrc, K_STRIDE, t * 32, 16 * kc, 4, 8);
          dqacc[q] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(av), as_bf16x8(bv), dqacc[q], 0, 0, 0);
        }
      }
    }

    // ---- c^T[d][slot] = Q^T dS^T + dO^T P^T on tiles t = w + 4q (fp16 rows: times 2^pexp) ----
    const uint64_t prow = wr ? (uint64_t)(uint32_t)pos * (uint32_t)p.ntiles + tile : trash;
    unsigned char *dst = p.partials + prow * (uint64_t)(D_QK * (F32P ? 4 : 2));
    if constexpr (!F32P) p.partial_exp[prow] = (int8_t)pexp;  // every wave and lane half stores the same byte
#pragma unroll
    for (int q = 0; q < DQW; ++q) {
      // a wave without a tile of its own on the last step redoes tile DQT - 1
      // and stores the same bits again, so that every wave issues the same
      // stores on every block
      const int t = w + 4 * q < DQT ? w + 4 * q : DQT - 1;
      {
        f32x16 cacc;
#pragma unroll
        for (int a = 0; a < 16; ++a) cacc[a] = 0.0f;
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) {
          const i32x4 av = tr_operand(QL, L::QL_STRIDE, t * 32, 16 * kc, 8, 4);
          cacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(av), dsB[kc], cacc, 0, 0, 0);
        }
        if (t < DVT) {
#pragma unroll
          for (int kc = 0; kc < 2; ++kc) {
            const i32x4 av = tr_operand(DOL, L::DOL_STRIDE, t * 32, 16 * kc, 8, 4);
            cacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(av), pB[kc], cacc, 0, 0, 0);
          }
        }
        {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int d0 = t * 32 + 8 * i + 4 * g32;
            // plain (write-back) stores: a row's pieces come from four waves and
            // several instructions, and L2 merges them into whole lines
            if constexpr (F32P) {
              *reinterpret_cast<f32x4 *>(dst + d0 * 4) = f32x4{cacc[4 * i], cacc[4 * i + 1], cacc[4 * i + 2],
                                                               cacc[4 * i + 3]};
            } else {
              *reinterpret_cast<i32x2 *>(dst + d0 * 2) =
                  i32x2{(int)pack_f16x2(cacc[4 * i], cacc[4 * i + 1]), (int)pack_f16x2(cacc[4 * i + 2], cacc[4 * i + 3])};
            }
          }
        }
      }
    }
    __syncthreads();  // rows, partial tiles and dS tiles consumed before the next block
    idx_cur = idx_nxt;
    raw_nxt = raw_nn;
    pos_cur = pos_nxt;
  }

  // ---- dQ: lane = head l32, d = t*32 + 8i + 4*g32 + j ----
  if (l32 < nheads) {
    uint16_t *drow = p.dq + (head0 + l32) * D_QK;
#pragma unroll
    for (int q = 0; q < DQW; ++q) {
      const int t = w + 4 * q;
      if (t < DQT) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const i32x2 pk = {(int)pack_bf16x2(dqacc[q][4 * i], dqacc[q][4 * i + 1]),
                            (int)pack_bf16x2(dqacc[q][4 * i + 2], dqacc[q][4 * i + 3])};
          *reinterpret_cast<i32x2 *>(drow + t * 32 + 8 * i + 4 * g32) = pk;
        }
      }
    }
  }
}

template <int D_QK, int D_V, bool FP8, bool F32P>
static int launch_bwd_wide_t(const BwdParams &p, hipStream_t st) {
  using L = WideBwdLds<D_QK, D_V, FP8>;
  const size_t lds = L::BYTES;
  hipError_t e = hipFuncSetAttribute((const void *)sparse_mla_bwd_wide_kernel<D_QK, D_V, FP8, F32P>,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return set_error(DSA_ERR_HIP, "sparse_mla_bwd(wide): LDS attribute: %s", hipGetErrorString(e));
  const int64_t nitems = p.B * p.S * p.G * p.ntiles;
  if (nitems >= (1ll << 31)) return set_error(DSA_ERR_INVALID_ARG, "sparse_mla_bwd(wide): grid too large");
  hipLaunchKernelGGL((sparse_mla_bwd_wide_kernel<D_QK, D_V, FP8, F32P>), dim3((unsigned)nitems), dim3(256), lds, st,
                     p);
  return check_launch("sparse_mla_bwd_main(wide)");
}

template <int D_QK, int D_V>
static int launch_bwd_wide_f(const BwdParams &p, bool fp8, bool f32p, hipStream_t st) {
  if (fp8) return f32p ? launch_bwd_wide_t<D_QK, D_V, true, true>(p, st) : launch_bwd_wide_t<D_QK, D_V, true, false>(p, st);
  return f32p ? launch_bwd_wide_t<D_QK, D_V, false, true>(p, st) : launch_bwd_wide_t<D_QK, D_V, false, false>(p, st);
}

int launch_bwd_main_wide(const BwdParams &p, int64_t d_qk, int64_t d_v, bool fp8, bool f32p, hipStream_t st) {
  if (d_qk == 576 && d_v == 512) return launch_bwd_wide_f<576, 512>(p, fp8, f32p, st);
  if (d_qk == 576 && d_v == 576) return launch_bwd_wide_f<576, 576>(p, fp8, f32p, st);
  return set_error(DSA_ERR_UNSUPPORTED, "sparse_mla_bwd(wide): no kernel for d_qk=%lld d_v=%lld", (long long)d_qk,
                   (long long)d_v);
}

}  // namespace dsa
