// SparseMLA forward for gfx950 (bf16 and OCP-e4m3 tensorwise).
//
// Reference semantics: cppmega/megatron/sparse_mla_ops/tilelang_sparse_mla_fwd.py:137-290
// (bf16) and tilelang_sparse_mla_fwd_fp8.py:187-393 (fp8).  For every query
// token the selected latent-KV rows are gathered, S = scale * Q K^T is formed
// over d_qk, an online exp2 softmax runs over the slots, P is rounded to bf16
// and O = P V is accumulated in fp32 over the d_v prefix; LSE is emitted in
// log2 units.
//
// Work decomposition: one wave owns one (token, kv group, 32-head tile) work
// item and walks all of its top-k slots in blocks of 32; a workgroup is four
// independent waves (no workgroup barrier).  Per block:
//   1. gather: 16-byte row-chunk loads (16 lanes cover one 256-byte row) of the
//      32 selected rows, issued one block ahead into registers while the
//      previous block computes, then stored row-major to the wave's LDS tile
//      (e4m3: plus the V prefix dequantised to bf16);
//   2. S^T[slot][head] = K Q^T (32x32x16 MFMA, K rows as the A operand, Q
//      resident in registers as the B operand): each lane then owns one head
//      and 16 slots, so the softmax row reduction is in-lane plus one
//      cross-half exchange;
//   3. P (fp32 -> bf16) is re-used straight from the accumulator registers as
//      the B operand of O^T[d][head] += V^T P^T; the A operand V^T[d][slot] is
//      read from the row-major tile with transposing LDS reads
//      (ds_read_b64_tr_b16) in the accumulator's slot order.
// Indices for block b+2 and rows for block b+1 are in flight while block b
// computes.
#include "dsa_common.hpp"
#include "sparse_mla_gather.hpp"
#include "sparse_mla_params.hpp"
#include "sparse_mla_wide.hpp"

namespace dsa {

template <int D_QK, int D_V, bool FP8, bool MX = false, bool VPRE = false>
struct FwdCfg {
  using Gat = GatherCfg<D_QK, D_V, FP8, MX>;
  // e4m3 with V dequantised once per call: the V rows are gathered as bf16
  // straight into the V tile (a bf16 gather over d_v columns), not converted
  using VGat = GatherCfg<D_V, D_V, false>;
  static_assert(!VPRE || FP8, "pre-dequantised V exists for e4m3 input only");
  static constexpr int KL_BYTES = 32 * Gat::KL_STRIDE;
  static constexpr int KD_STRIDE = D_V * 2 + 32;          // e4m3: dequantised V rows (bf16)
  static constexpr int KD_BYTES = FP8 ? 32 * KD_STRIDE : 0;
  static constexpr int SC_BYTES = FP8 ? (MX ? Gat::NBLK : 1) * 32 * 4 : 0;
  // bf16 rows: the gather's slot offsets go through LDS (32 ints) and the K
  // tile's chunks are swizzled by row bit 3 (gather_store_k)
  static constexpr bool XL = !FP8;
  static constexpr int OFFS_BYTES = XL ? 32 * 4 : 0;
  static constexpr int WAVE_BYTES = (KL_BYTES + KD_BYTES + SC_BYTES + OFFS_BYTES + 15) / 16 * 16;
  // bf16 source of the V^T operand: the raw tile, or the dequantised one for e4m3
  static constexpr int V_STRIDE = FP8 ? KD_STRIDE : Gat::KL_STRIDE;
  static constexpr int DT = D_V / 32;
  static constexpr int KSTEPS = D_QK / 16;
  static_assert(D_V % 32 == 0 && D_QK % 16 == 0 && D_V <= D_QK, "unsupported head dims");
};

// QMX: the bf16 kernel with Q given as e4m3 codes and one scale per 32
// channels (q_scale [B, S, H, D_QK / 32]), converted to bf16 as it is loaded.
template <int D_QK, int D_V, bool FP8, bool MX = false, bool VPRE = false, bool QMX = false>
__global__ void __launch_bounds__(256)
sparse_mla_fwd_kernel(const FwdParams p) {
  static_assert(!QMX || !FP8, "QMX converts Q for the bf16 kernel");
  if (p.gate != nullptr && *p.gate != p.gate_run) return;  // the call's other kernel computes it
  using C = FwdCfg<D_QK, D_V, FP8, MX, VPRE>;
  using Gat = typename C::Gat;
  using VGat = typename C::VGat;
  static_assert(VGat::KL_STRIDE == C::KD_STRIDE, "bf16 V rows land in the V tile's layout");
  // tensorwise e4m3: S on the 32x32x64 f8f6f4 MFMA (unit block scales), whose
  // lane (row l32, half g32) holds channels [16 g32, +16) and [32 + 16 g32, +16)
  // of each 64-channel chunk; MX keeps 32x32x16 (one partial per 32-channel block)
  constexpr bool F8X = FP8 && !MX && D_QK % 64 == 0;
  constexpr int QK = F8X ? D_QK / 64 : C::KSTEPS;  // Q operand registers (MFMA k-steps)
  typedef typename std::conditional<F8X, i32x8, typename std::conditional<FP8, long, bf16x8>::type>::type qop_t;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

  const int lane = lane_id(), w = wave_id();
  const int g32 = lane >> 5, l32 = lane & 31;
  // item = (tok * G + g) * ntiles + tile, tok = b * S + s; every factor is
  // below 2^31 (checked on the host), so 32-bit divisions suffice
  const uint32_t nitems = (uint32_t)(p.B * p.S * p.G * p.ntiles);
  const uint32_t item = (uint32_t)xcd_remap(blockIdx.x, gridDim.x) * 4u + (uint32_t)w;
  if (item >= nitems) return;  // waves are independent: no workgroup barrier below
  const uint32_t ntl = (uint32_t)p.ntiles, ng = (uint32_t)p.G;
  const uint32_t rest = ntl == 1 ? item : item / ntl;
  const int tile = (int)(item - rest * ntl);
  const int64_t tok = ng == 1 ? rest : rest / ng;
  const int64_t g = (int64_t)rest - tok * (int64_t)ng;
  const int64_t b = (int64_t)((uint32_t)tok / (uint32_t)p.S);

  unsigned char *Kl = smem + w * C::WAVE_BYTES;
  unsigned char *Kd = Kl + C::KL_BYTES;
  float *Ksc = reinterpret_cast<float *>(Kd + C::KD_BYTES);
  int *offs = reinterpret_cast<int *>(Kd + C::KD_BYTES + C::SC_BYTES);
  const unsigned char *Vsrc = FP8 ? Kd : Kl;

  const int h_local = tile * 32 + l32;
  const bool head_ok = h_local < p.hpg;
  const int64_t qrow = tok * p.H + g * p.hpg + h_local;
  const int32_t *idx_row = p.idx + (tok * p.G + g) * p.topk;
  const unsigned char *kv_b = p.kv + ((b * p.S_kv) * p.G + g) * Gat::ROWB;
  // kv scales: [B, S_kv] per row, or MX [B, S_kv, G, D_QK / 32] per (row, block)
  const float *kv_scale_b = !FP8 ? nullptr : (MX ? p.kv_scale + ((b * p.S_kv) * p.G + g) * Gat::NBLK
                                                 : p.kv_scale + b * p.S_kv);
  const uint32_t sc_pitch = MX ? (uint32_t)(p.G * Gat::NBLK * 4) : 4u;
  const uint32_t row_pitch = (uint32_t)(p.G * Gat::ROWB);
  const int nblk = (int)((p.topk + 31) / 32);

  // Indices of blocks 0 and 1, then the rows of block 0, go out before the Q loads.
  const auto idx_rs = slot_rsrc(idx_row, p.topk);
  int idx_cur = slot_index(load_slot_raw(idx_rs, 0, l32), 0, l32, p.topk, p.S_kv);
  int raw_nxt = load_slot_raw(idx_rs, 1, l32);
  const auto kv_rs = make_buffer_rsrc(kv_b, (uint32_t)(p.S_kv * (int64_t)row_pitch));
  const auto sc_rs = make_buffer_rsrc(kv_scale_b, FP8 ? (uint32_t)(p.S_kv * sc_pitch) : 0u);
  typename Gat::Regs rg;
  if constexpr (C::XL) {
    gather_put_offsets(offs, idx_cur, row_pitch);
    wave_lds_sync();
    gather_issue_offs<Gat>(rg, kv_rs, offs);
  } else {
    gather_issue<Gat>(rg, kv_rs, sc_rs, idx_cur, row_pitch, sc_pitch);
  }
  // pre-dequantised V rows of this (batch, group): bf16, v16_ld elements per
  // row of [B, S_kv, G], V in the leading D_V
  const uint32_t v_pitch = (uint32_t)(p.G * p.v16_ld * 2);
  const auto v_rs = make_buffer_rsrc(VPRE ? p.v16 + ((b * p.S_kv) * p.G + g) * p.v16_ld : nullptr,
                                     VPRE ? (uint32_t)(p.S_kv * (int64_t)v_pitch) : 0u);
  typename VGat::Regs rgv;
  if constexpr (VPRE) gather_issue<VGat>(rgv, v_rs, v_rs, idx_cur, v_pitch);

  // Q as the B operand: lane = head, 8 consecutive d per k-step, through a
  // resource that ends at the tile's last head (padded heads read zeros), so
  // the loads carry no branches.
  const int64_t qrow0 = tok * p.H + g * p.hpg + tile * 32;
  const int nh = p.hpg - tile * 32 < 32 ? p.hpg - tile * 32 : 32;
  constexpr int QB = FP8 || QMX ? 1 : 2;  // bytes per Q element
  const auto q_rs = make_buffer_rsrc(p.q + qrow0 * D_QK * QB, (uint32_t)(nh * D_QK * QB));
  qop_t qreg[QK];
  float qmxs[QMX ? D_QK / 32 : 1];  // QMX: this lane's head's block scales
  if constexpr (QMX) {
#pragma unroll
    for (int c = 0; c < D_QK / 32; ++c) qmxs[c] = head_ok ? p.q_scale[qrow * (D_QK / 32) + c] : 0.0f;
  }
#pragma unroll
  for (int k = 0; k < QK; ++k) {
    if constexpr (F8X) {
      const auto lo = __builtin_amdgcn_raw_buffer_load_b128(q_rs, l32 * D_QK + 64 * k + 16 * g32, 0, 0);
      const auto hi = __builtin_amdgcn_raw_buffer_load_b128(q_rs, l32 * D_QK + 64 * k + 32 + 16 * g32, 0, 0);
      qreg[k] = i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
    } else if constexpr (FP8) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b64(q_rs, l32 * D_QK + 16 * k + 8 * g32, 0, 0);
      qreg[k] = __builtin_bit_cast(long, v);
    } else if constexpr (QMX) {
      // channels 16k + 8 g32 .. + 7 all lie in block k / 2
      const auto v = __builtin_amdgcn_raw_buffer_load_b64(q_rs, l32 * D_QK + 16 * k + 8 * g32, 0, 0);
      qreg[k] = e4m3x8_to_bf16_scaled((uint32_t)v[0], (uint32_t)v[1], qmxs[k >> 1]);
    } else {
      qreg[k] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(
                                               q_rs, (l32 * D_QK + 16 * k + 8 * g32) * 2, 0, 0));
    }
  }
  float qsc = 1.0f;
  if constexpr (FP8 && !MX) qsc = p.q_scale[tok];
  const float tscale = p.sl2 * qsc;
  // MX: this lane's head's block scales (q_scale [B, S, H, D_QK / 32])
  float qbs[MX ? Gat::NBLK : 1];
  if constexpr (MX) {
#pragma unroll
    for (int c = 0; c < Gat::NBLK; ++c) qbs[c] = head_ok ? p.q_scale[qrow * Gat::NBLK + c] : 0.0f;
  }

  float m_run = kNegBig, l_run = 0.0f;
  f32x16 oacc[C::DT];
#pragma unroll
  for (int t = 0; t < C::DT; ++t)
#pragma unroll
    for (int a = 0; a < 16; ++a) oacc[t][a] = 0.0f;

  for (int blk = 0; blk < nblk; ++blk) {
    // ---- stage block blk: K row-major, V transposed (bf16, dequantised for e4m3) ----
    gather_store_k<Gat, C::XL>(rg, Kl);
    if constexpr (FP8) {
      if constexpr (VPRE)
        gather_store_k<VGat>(rgv, Kd);
      else
        gather_store_dequant<Gat, Gat::NCH_V>(rg, Kd, C::KD_STRIDE);
      gather_store_scale<Gat>(rg, Ksc);
    }
    const uint64_t vmask = __ballot(idx_cur >= 0);
    const int idx_nxt = slot_index(raw_nxt, blk + 1, l32, p.topk, p.S_kv);
    if constexpr (C::XL) gather_put_offsets(offs, idx_nxt, row_pitch);
    wave_lds_sync();
    // ---- prefetch: rows of block blk+1, indices of block blk+2 ----
    // (issued unconditionally, past the last block too, so every wait is counted exactly)
    const int raw_nn = load_slot_raw(idx_rs, blk + 2, l32);
    if constexpr (C::XL)
      gather_issue_offs<Gat>(rg, kv_rs, offs);
    else
      gather_issue<Gat>(rg, kv_rs, sc_rs, idx_nxt, row_pitch, sc_pitch);
    if constexpr (VPRE) gather_issue<VGat>(rgv, v_rs, v_rs, idx_nxt, v_pitch);

    // ---- S^T = K Q^T  (M = slot, N = head, K = d) ----
    f32x16 sacc;
#pragma unroll
    for (int a = 0; a < 16; ++a) sacc[a] = 0.0f;
    if constexpr (MX) {
      // per 32-channel block: a partial product on the codes, then
      // S += partial * kv_scale[slot][block] * q_scale[head][block]
#pragma unroll
      for (int c = 0; c < Gat::NBLK; ++c) {
        f32x16 part;
#pragma unroll
        for (int a = 0; a < 16; ++a) part[a] = 0.0f;
#pragma unroll
        for (int k = 2 * c; k < 2 * c + 2; ++k) {
          const long a = *reinterpret_cast<const long *>(Kl + l32 * Gat::KL_STRIDE + 16 * k + 8 * g32);
          part = __builtin_amdgcn_mfma_f32_32x32x16_fp8_fp8(a, qreg[k], part, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const f32x4 k4 = *reinterpret_cast<const f32x4 *>(Ksc + c * 32 + 8 * i + 4 * g32);
#pragma unroll
          for (int j = 0; j < 4; ++j) sacc[4 * i + j] = fmaf(part[4 * i + j], k4[j] * qbs[c], sacc[4 * i + j]);
        }
      }
    }
#pragma unroll
    for (int k = 0; k < (MX ? 0 : QK); ++k) {
      if constexpr (F8X) {
        const unsigned char *kr = Kl + l32 * Gat::KL_STRIDE + 64 * k + 16 * g32;
        const i32x4 lo = *reinterpret_cast<const i32x4 *>(kr);
        const i32x4 hi = *reinterpret_cast<const i32x4 *>(kr + 32);
        const i32x8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        sacc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, qreg[k], sacc, 0, 0, 0, 127, 0, 127);
      } else if constexpr (FP8) {
        const long a = *reinterpret_cast<const long *>(Kl + l32 * Gat::KL_STRIDE + 16 * k + 8 * g32);
        sacc = __builtin_amdgcn_mfma_f32_32x32x16_fp8_fp8(a, qreg[k], sacc, 0, 0, 0);
      } else {
        // chunk 2k + g32 of row l32, at chunk (2k + g32) ^ ((l32 >> 3) & 1) of the swizzled tile
        const i32x4 a = *reinterpret_cast<const i32x4 *>(Kl + l32 * Gat::KL_STRIDE + 32 * k +
                                                         16 * (g32 ^ ((l32 >> 3) & 1)));
        sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), qreg[k], sacc, 0, 0, 0);
      }
    }

    // ---- online softmax over this block's 32 slots (log2 domain, lazy rescale) ----
    // P = exp2(s * scale' - m_ref) against a reference max that only moves when
    // a score exceeds it by more than 2^8: P stays <= 256 (exact range for
    // bf16 / fp32) and O, l are rescaled only on those (rare, wave-uniform) steps.
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
        float v = sacc[4 * i + j];
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
    if (__ballot(mloc > m_run + 8.0f) != 0ull) {  // some head's max moved: rescale O, l
      const float m_new = fmaxf(m_run, mloc);
      const float alpha = exp2_fast(m_run - m_new);
      l_run *= alpha;
      m_run = m_new;
#pragma unroll
      for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
        for (int a = 0; a < 16; ++a) oacc[dt][a] *= alpha;
    }
    float t[16];
    float lsum = 0.0f;
#pragma unroll
    for (int a = 0; a < 16; ++a) {
      t[a] = exp2_fast(fmaf(xs[a], tscale, -m_run));  // -inf (masked slot) -> 0
      lsum += t[a];
    }
    lsum = sum_halves(lsum);
    l_run += lsum;

    // ---- O^T[d][head] += V^T[d][slot] P^T[slot][head]  (K = slot, accumulator order) ----
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      i32x4 pb;
#pragma unroll
      for (int e = 0; e < 4; ++e) pb[e] = (int)pack_bf16x2(t[8 * kc + 2 * e], t[8 * kc + 2 * e + 1]);
      const bf16x8 bop = as_bf16x8(pb);
#pragma unroll
      for (int dt = 0; dt < C::DT; ++dt) {
        const i32x4 av = C::XL ? tr_operand_swz(Vsrc, C::V_STRIDE, dt * 32, 16 * kc)
                               : tr_operand(Vsrc, C::V_STRIDE, dt * 32, 16 * kc, 8, 4);
        oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(av), bop, oacc[dt], 0, 0, 0);
      }
    }
    wave_lds_sync();
    idx_cur = idx_nxt;
    raw_nxt = raw_nn;
  }

  // ---- normalise and write: lane = head l32, d = dt*32 + 8i + 4*g32 + j ----
  if (head_ok) {
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    uint16_t *orow = p.out + qrow * D_V;
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const i32x2 pk = {(int)pack_bf16x2(oacc[dt][4 * i] * inv, oacc[dt][4 * i + 1] * inv),
                          (int)pack_bf16x2(oacc[dt][4 * i + 2] * inv, oacc[dt][4 * i + 3] * inv)};
        *reinterpret_cast<i32x2 *>(orow + dt * 32 + 8 * i + 4 * g32) = pk;
      }
    }
    if (g32 == 0) p.lse[qrow] = l_run > 0.0f ? log2f(l_run) + m_run : -INFINITY;
  }
}

template <int D_QK, int D_V, bool FP8, bool MX, bool VPRE, bool QMX = false>
static int launch_fwd_t(const FwdParams &p, hipStream_t st) {
  using C = FwdCfg<D_QK, D_V, FP8, MX, VPRE>;
  const size_t lds = 4 * (size_t)C::WAVE_BYTES;
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute((const void *)sparse_mla_fwd_kernel<D_QK, D_V, FP8, MX, VPRE, QMX>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return set_error(DSA_ERR_HIP, "sparse_mla_fwd: LDS attribute: %s", hipGetErrorString(e));
  }
  const int64_t nitems = p.B * p.S * p.G * p.ntiles;
  const int64_t nblocks = (nitems + 3) / 4;
  if (nitems >= (1ll << 31)) return set_error(DSA_ERR_INVALID_ARG, "sparse_mla_fwd: grid too large");
  hipLaunchKernelGGL((sparse_mla_fwd_kernel<D_QK, D_V, FP8, MX, VPRE, QMX>), dim3((unsigned)nblocks), dim3(256), lds,
                     st, p);
  return check_launch("sparse_mla_fwd");
}

// e4m3: the kernel reads pre-dequantised V rows when p.v16 is set
template <int D_QK, int D_V, bool FP8, bool MX = false>
static int launch_fwd(const FwdParams &p, hipStream_t st) {
  if constexpr (FP8) {
    if (p.v16) return launch_fwd_t<D_QK, D_V, true, MX, true>(p, st);
  }
  return launch_fwd_t<D_QK, D_V, FP8, MX, false>(p, st);
}

// V rows of e4m3 kv dequantised to bf16 once per call, with the arithmetic of
// the kernels' in-LDS dequantisation (hardware e4m3 pair decode, times the
// row's or the 32-channel block's scale, round to nearest even), so the values
// are bit-identical.  One thread per 8 consecutive V columns of a row; rows
// are (b, s_kv, g), kv_scale [B, S_kv] per (b, s_kv), or MX [B, S_kv, G, D_qk / 32].
template <bool MX>
__global__ void __launch_bounds__(256)
dequant_v_kernel(const unsigned char *kv, const float *kv_scale, uint16_t *v16, int64_t rows, int G, int D_qk,
                 int D_v) {
  const int per_row = D_v / 8;
  const int64_t n = rows * per_row;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / per_row;
    const int c8 = (int)(i - row * per_row);
    const uint2 raw = *reinterpret_cast<const uint2 *>(kv + row * D_qk + 8 * c8);
    const float s = MX ? kv_scale[row * (D_qk / 32) + (8 * c8) / 32] : kv_scale[row / G];
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const f32x2 v2 = e4m3x2_to_f32(e < 2 ? raw.x : raw.y, (e & 1) != 0);
      w[e] = pack_bf16x2(v2[0] * s, v2[1] * s);
    }
    *reinterpret_cast<i32x4 *>(v16 + row * D_v + 8 * c8) = i32x4{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
  }
}

// MX forward with a workspace, first of its two passes: every kv row
// dequantised to bf16 (code times its 32-channel block scale, round to nearest
// even: the values the block-scaled kernel forms for V) into kv16 [B, S_kv, G,
// D_qk], and every q and kv block scale checked.  *gate (cleared by
// mx_gate_reset_kernel) becomes 1 unless each scale passes mx_scale_exact.  If
// all do, every dequantised value (and Q converted the same way at load) is
// exact, and the bf16 kernel on them computes the block-scaled scores up to the
// order of the fp32 sums; otherwise the block-scaled e4m3 kernel runs instead.
__global__ void __launch_bounds__(256)
mx_prepass_kernel(const unsigned char *kv, const float *kv_scale, uint16_t *kv16, int64_t rows, int D_qk,
                  const float *q_scale, int64_t n_qscales, int *gate) {
  const int per_row = D_qk / 8;
  const int64_t n = rows * per_row;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  bool bad = false;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += stride) {
    const int64_t row = i / per_row;
    const int c8 = (int)(i - row * per_row);
    const uint2 raw = *reinterpret_cast<const uint2 *>(kv + row * D_qk + 8 * c8);
    const float sc = kv_scale[row * (D_qk / 32) + (8 * c8) / 32];
    bad |= !mx_scale_exact(sc);
    *reinterpret_cast<bf16x8 *>(kv16 + row * D_qk + 8 * c8) = e4m3x8_to_bf16_scaled(raw.x, raw.y, sc);
  }
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n_qscales; i += stride)
    bad |= !mx_scale_exact(q_scale[i]);
  if (__ballot(bad) != 0ull && lane_id() == 0) atomicOr(gate, 1);
}

__global__ void mx_gate_reset_kernel(int *gate) {
  if (threadIdx.x == 0) *gate = 0;
}

}  // namespace dsa

using namespace dsa;

static size_t v16_bytes(int64_t B, int64_t S_kv, int64_t G, int64_t D_v) {
  return ((size_t)B * S_kv * G * D_v * 2 + 255) & ~(size_t)255;
}

// MX shapes with the exact-dequantisation path (a bf16 kernel for d_qk / d_v)
static bool mx_exact_shape(int64_t D_qk, int64_t D_v) {
  return (D_qk == 128 && (D_v == 64 || D_v == 128)) || (D_qk == 192 && D_v == 128) || (D_qk == 576 && D_v == 512);
}
// MX workspace: whole kv rows in bf16, then the gate (256 bytes)
static size_t mx_ws_bytes(int64_t B, int64_t S_kv, int64_t G, int64_t D_qk) {
  return v16_bytes(B, S_kv, G, D_qk) + 256;
}

static int sparse_mla_fwd_impl(const void *q, const void *kv, const int32_t *indices, void *out, float *lse2,
                               int64_t B, int64_t S, int64_t S_kv, int64_t H, int64_t G, int64_t D_qk, int64_t D_v,
                               int64_t topk, float sm_scale, int dtype, const float *q_scale, const float *kv_scale,
                               void *workspace, size_t workspace_bytes, void *stream) {
  DSA_REQUIRE(B >= 0 && S >= 0 && S_kv > 0 && H > 0 && G > 0 && topk > 0,
              "dsa_sparse_mla_fwd: bad dims B=%lld S=%lld S_kv=%lld H=%lld G=%lld topk=%lld",
              (long long)B, (long long)S, (long long)S_kv, (long long)H, (long long)G, (long long)topk);
  DSA_REQUIRE(H % G == 0, "dsa_sparse_mla_fwd: H=%lld not divisible by G=%lld", (long long)H, (long long)G);
  DSA_REQUIRE(D_v > 0 && D_v <= D_qk, "dsa_sparse_mla_fwd: need 0 < d_v <= d_qk (got %lld, %lld)",
              (long long)D_v, (long long)D_qk);
  DSA_REQUIRE(dtype == DSA_DTYPE_BF16 || dtype == DSA_DTYPE_E4M3 || dtype == DSA_DTYPE_MXFP8,
              "dsa_sparse_mla_fwd: dtype %d", dtype);
  DSA_REQUIRE(S_kv < (1ll << 31) && topk < (1ll << 31), "dsa_sparse_mla_fwd: S_kv/topk too large");
  if (B == 0 || S == 0) return DSA_OK;
  DSA_REQUIRE(q && kv && indices && out && lse2, "dsa_sparse_mla_fwd: null tensor pointer");
  if (dtype == DSA_DTYPE_E4M3 || dtype == DSA_DTYPE_MXFP8)
    DSA_REQUIRE(q_scale && kv_scale, "dsa_sparse_mla_fwd: e4m3 input needs q_scale and kv_scale");
  FwdParams p;
  p.q = static_cast<const unsigned char *>(q);
  p.kv = static_cast<const unsigned char *>(kv);
  p.idx = indices;
  p.out = static_cast<uint16_t *>(out);
  p.lse = lse2;
  p.q_scale = q_scale;
  p.kv_scale = kv_scale;
  p.v16 = nullptr;
  p.v16_ld = (int)D_v;
  p.gate = nullptr;
  p.gate_run = 0;
  p.B = B;
  p.S = S;
  p.S_kv = S_kv;
  p.H = H;
  p.G = G;
  p.topk = topk;
  p.hpg = (int)(H / G);
  p.ntiles = (p.hpg + 31) / 32;
  p.sl2 = sm_scale * kLog2e;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool f8 = dtype == DSA_DTYPE_E4M3;
  DSA_REQUIRE(S_kv * G * D_qk * 2 <= (int64_t)kMaskedOff, "dsa_sparse_mla_fwd: kv rows of one batch exceed 4 GiB - 64 KiB");
  if (workspace != nullptr && dtype == DSA_DTYPE_MXFP8 && mx_exact_shape(D_qk, D_v)) {
    // MX: kv rows dequantised once (and the scales checked), then two kernels
    // gated on the check: the bf16 kernel on the dequantised rows with Q
    // converted at load when every scale makes the conversion exact, else the
    // block-scaled e4m3 kernel (reading V from the dequantised rows when narrow)
    const size_t need = mx_ws_bytes(B, S_kv, G, D_qk);
    DSA_REQUIRE(workspace_bytes >= need, "dsa_sparse_mla_fwd: workspace %zu < required %zu", workspace_bytes, need);
    uint16_t *kv16 = static_cast<uint16_t *>(workspace);
    int *gate = reinterpret_cast<int *>(static_cast<unsigned char *>(workspace) + v16_bytes(B, S_kv, G, D_qk));
    const int64_t rows = B * S_kv * G;
    const int64_t units = rows * (D_qk / 8);
    const unsigned grid = (unsigned)((units + 255) / 256 < 8192 ? (units + 255) / 256 : 8192);
    hipLaunchKernelGGL(mx_gate_reset_kernel, dim3(1), dim3(64), 0, st, gate);
    hipLaunchKernelGGL(mx_prepass_kernel, dim3(grid), dim3(256), 0, st, p.kv, kv_scale, kv16, rows, (int)D_qk, q_scale,
                       B * S * H * (D_qk / 32), gate);
    int rc = check_launch("sparse_mla_fwd(MX dequantise)");
    if (rc) return rc;
    FwdParams pe = p;
    pe.kv = reinterpret_cast<const unsigned char *>(kv16);
    pe.kv_scale = nullptr;
    pe.gate = gate;
    pe.gate_run = 0;
    if (wide_shape(D_qk, D_v)) rc = launch_fwd_wide(pe, D_qk, D_v, false, st, false, true);
    else if (D_qk == 128 && D_v == 64) rc = launch_fwd_t<128, 64, false, false, false, true>(pe, st);
    else if (D_qk == 128) rc = launch_fwd_t<128, 128, false, false, false, true>(pe, st);
    else rc = launch_fwd_t<192, 128, false, false, false, true>(pe, st);
    if (rc) return rc;
    p.gate = gate;
    p.gate_run = 1;
    if (!wide_shape(D_qk, D_v)) {
      p.v16 = kv16;
      p.v16_ld = (int)D_qk;
    }
  } else if (workspace != nullptr && dtype != DSA_DTYPE_BF16 && !wide_shape(D_qk, D_v)) {
    // e4m3: dequantise the V rows once instead of once per gather
    DSA_REQUIRE(workspace_bytes >= v16_bytes(B, S_kv, G, D_v), "dsa_sparse_mla_fwd: workspace %zu < required %zu",
                workspace_bytes, v16_bytes(B, S_kv, G, D_v));
    uint16_t *v16 = static_cast<uint16_t *>(workspace);
    const int64_t rows = B * S_kv * G;
    const int64_t n = rows * (D_v / 8);
    const unsigned grid = (unsigned)((n + 255) / 256 < 8192 ? (n + 255) / 256 : 8192);
    if (dtype == DSA_DTYPE_MXFP8)
      hipLaunchKernelGGL(dequant_v_kernel<true>, dim3(grid), dim3(256), 0, st, p.kv, kv_scale, v16, rows, (int)G,
                         (int)D_qk, (int)D_v);
    else
      hipLaunchKernelGGL(dequant_v_kernel<false>, dim3(grid), dim3(256), 0, st, p.kv, kv_scale, v16, rows, (int)G,
                         (int)D_qk, (int)D_v);
    const int rc = check_launch("sparse_mla_fwd(dequant V)");
    if (rc) return rc;
    p.v16 = v16;
  }
  if (dtype == DSA_DTYPE_MXFP8) {  // e4m3 with one scale per 32 channels of every row
    if (D_qk == 128 && D_v == 64) return launch_fwd<128, 64, true, true>(p, st);
    if (D_qk == 128 && D_v == 128) return launch_fwd<128, 128, true, true>(p, st);
    if (D_qk == 192 && D_v == 128) return launch_fwd<192, 128, true, true>(p, st);
    if (wide_shape(D_qk, D_v)) return launch_fwd_wide(p, D_qk, D_v, true, st, true);
    return set_error(DSA_ERR_UNSUPPORTED, "dsa_sparse_mla_fwd: no MXFP8 kernel for d_qk=%lld d_v=%lld",
                     (long long)D_qk, (long long)D_v);
  }
  if (wide_shape(D_qk, D_v)) return launch_fwd_wide(p, D_qk, D_v, f8, st);
  if (D_qk == 128 && D_v == 64) return f8 ? launch_fwd<128, 64, true>(p, st) : launch_fwd<128, 64, false>(p, st);
  if (D_qk == 128 && D_v == 128) return f8 ? launch_fwd<128, 128, true>(p, st) : launch_fwd<128, 128, false>(p, st);
  if (D_qk == 192 && D_v == 128) return f8 ? launch_fwd<192, 128, true>(p, st) : launch_fwd<192, 128, false>(p, st);
  if (D_qk == 64 && D_v == 32 && !f8) return launch_fwd<64, 32, false>(p, st);
  return set_error(DSA_ERR_UNSUPPORTED, "dsa_sparse_mla_fwd: no kernel for d_qk=%lld d_v=%lld dtype=%d",
                   (long long)D_qk, (long long)D_v, dtype);
}

extern "C" int dsa_sparse_mla_fwd(const void *q, const void *kv, const int32_t *indices, void *out,
                                  float *lse2, int64_t B, int64_t S, int64_t S_kv, int64_t H,
                                  int64_t G, int64_t D_qk, int64_t D_v, int64_t topk, float sm_scale,
                                  int dtype, const float *q_scale, const float *kv_scale,
                                  void *stream) {
  return sparse_mla_fwd_impl(q, kv, indices, out, lse2, B, S, S_kv, H, G, D_qk, D_v, topk, sm_scale, dtype, q_scale,
                             kv_scale, nullptr, 0, stream);
}

extern "C" size_t dsa_sparse_mla_fwd_workspace_size(int64_t B, int64_t S_kv, int64_t G, int64_t D_qk,
                                                    int64_t D_v, int dtype) {
  if (B <= 0 || S_kv <= 0 || G <= 0 || D_v <= 0 || dtype == DSA_DTYPE_BF16) return 0;
  if (dtype == DSA_DTYPE_MXFP8 && mx_exact_shape(D_qk, D_v)) return mx_ws_bytes(B, S_kv, G, D_qk);
  // the wide (d_qk = 576) e4m3 kernel keeps converting V in LDS: at cfg5 reading
  // bf16 V rows (1 KiB each, beside 576 B of codes) was no faster than converting them
  if (wide_shape(D_qk, D_v)) return 0;
  return v16_bytes(B, S_kv, G, D_v);
}

extern "C" int dsa_sparse_mla_fwd_ws(const void *q, const void *kv, const int32_t *indices, void *out,
                                     float *lse2, int64_t B, int64_t S, int64_t S_kv, int64_t H, int64_t G,
                                     int64_t D_qk, int64_t D_v, int64_t topk, float sm_scale, int dtype,
                                     const float *q_scale, const float *kv_scale, void *workspace,
                                     size_t workspace_bytes, void *stream) {
  const size_t need = dsa_sparse_mla_fwd_workspace_size(B, S_kv, G, D_qk, D_v, dtype);
  DSA_REQUIRE(need == 0 || workspace, "dsa_sparse_mla_fwd_ws: null workspace (%zu bytes required)", need);
  return sparse_mla_fwd_impl(q, kv, indices, out, lse2, B, S, S_kv, H, G, D_qk, D_v, topk, sm_scale, dtype, q_scale,
                             kv_scale, need ? workspace : nullptr, workspace_bytes, stream);
}
