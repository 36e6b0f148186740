// SparseMLA backward for gfx950 (bf16 and OCP-e4m3 tensorwise), deterministic.
//
// Reference semantics: cppmega/megatron/sparse_mla_ops/tilelang_sparse_mla_bwd.py:123-167
// (Delta), :204-419 (P recompute, dP, dS, dQ, dKV scatter) and :170-201 (fp32 ->
// bf16 dKV), plus tilelang_sparse_mla_bwd_fp8.py:199-489 for the e4m3 form
// (QK^T on e4m3 codes, bf16-dequantised Q / KV for the other GEMMs).
//
// The reference scatters dKV with fp32 atomics, whose order (and so result)
// varies run to run; on MI355X that scatter alone also costs ~0.9 ms at the
// NAM56R shape.  Here the backward is:
//   1. inverse index kv-row -> entries, as a stable counting sort
//      (sparse_mla_csr.hpp): entries of a row come out in ascending
//      (token, kv group, slot) order;
//   2. bwd_main, query-major, one wave per (token, kv group, 32-head tile):
//      Delta = sum O*dO, P = exp2(s * scale' - LSE2), dP = dO V^T,
//      dS = P (dP - Delta) scale, dQ = dS K (written once at the end), and the
//      per-(token, slot) dKV row c = dS^T Q + P^T dO, stored as fp16 scaled by
//      a per-row power of two (11 significant bits relative to the row max,
//      exact to undo), or kept fp32 with DSA_BWD_FP32_PARTIALS, and written as
//      one coalesced row;
//   3. dkv_reduce, kv-major, one wave per kv row: its entries' rows are summed
//      in fp32 in CSR order, then cast to bf16.
// Every addition happens in an order fixed by the indices alone, so repeated
// calls are bitwise identical.
//
// bwd_main MFMA orientation (32x32x16 per block of 32 slots).  All LDS tiles
// are row-major; transposed operands come from ds_read_b64_tr_b16:
//   S = Q K^T, dP = dO V^T        M = head, N = slot: Q / dO from registers,
//                                 K / V rows from the gathered tile; each lane
//                                 then owns one slot and 16 heads;
//   c^T[d][slot] = Q^T dS^T + dO^T P^T
//                                 M = d, N = slot, K = head: dS / P straight
//                                 from the accumulator registers, Q^T / dO^T
//                                 transposed-read from row-major Q / dO tiles
//                                 with permuted column groups, so each lane
//                                 gets runs of 8 consecutive d of one slot;
//   dQ^T[d][head] = K^T dS^T      M = d, N = head, K = slot: both operands
//                                 transposed-read (K tile, dS[slot][head] tile).
#include "dsa_common.hpp"
#include "sparse_mla_csr.hpp"
#include "sparse_mla_gather.hpp"
#include "sparse_mla_params.hpp"
#include "sparse_mla_wide.hpp"

namespace dsa {

// LDS of one workgroup (one (token, kv group, 32-head tile) item, WPT waves):
//   shared  QL [head][d] bf16 (e4m3: dequantised), DOL [head][d] bf16,
//           LD [64] = LSE (heads 0..31) and Delta * sm_scale (32..63)
//   per wave  Kl [slot][d] raw K rows, Kd (e4m3: dequantised rows),
//             DS [slot][head] bf16, Ksc (e4m3: row scales)
// After the block loop the whole allocation is reused to combine the waves'
// dQ partial sums.
template <int D_QK, int D_V, bool FP8, bool F32P>
struct BwdCfg {
  using Gat = GatherCfg<D_QK, D_V, FP8>;
  static constexpr int WPT = 2;                          // waves per item
  static constexpr int PSZ = F32P ? 4 : 2;               // bytes per partial element
  static constexpr int QL_STRIDE = D_QK * 2 + 32;        // 32-byte pads: conflict-free transposed reads
  static constexpr int DOL_STRIDE = D_V * 2 + 32;
  static constexpr int OFF_QL = 0;
  static constexpr int OFF_DOL = OFF_QL + 32 * QL_STRIDE;
  static constexpr int OFF_LD = OFF_DOL + 32 * DOL_STRIDE;
  // LD: 64 floats (LSE, Delta * scale), then 4 (per-wave max|Q| and max|dO| of the item)
  static constexpr int SHARED_BYTES = (OFF_LD + 68 * 4 + 15) / 16 * 16;
  static constexpr int KSTEPS = D_QK / 16;
  static constexpr int VSTEPS = D_V / 16;
  // bf16 input with fp16 partial rows: each partial row's power-of-two scale is
  // taken from a bound before its products
  static constexpr bool BEXP = !FP8 && !F32P;
  // bf16 input: the Q / dO operands of S and dP stay in registers where they
  // fit beside the accumulators (2 waves per SIMD up to d_qk = 128, 1 above)
  static constexpr bool REGQ = !FP8 && (KSTEPS + VSTEPS <= 12 || D_QK > 128);
  static constexpr int KL_BYTES = 32 * Gat::KL_STRIDE;
  static constexpr int KD_STRIDE = D_QK * 2 + 32;        // e4m3: dequantised rows (bf16)
  static constexpr int KD_BYTES = FP8 ? 32 * KD_STRIDE : 0;
  static constexpr int DS_STRIDE = 32 * 2 + 32;          // dS[slot][head] bf16
  static constexpr int DS_BYTES = 32 * DS_STRIDE;
  static constexpr int CS_STRIDE = D_QK * 2 + 16;        // staged fp16 partial rows (over Kl, Kd): 16-byte
                                                         // writes of 32 rows land in distinct banks
  static constexpr int ROW_CHUNKS = D_QK * 2 / 16;       // 16-byte chunks per fp16 partial row
  static_assert((32 * ROW_CHUNKS) % 64 == 0, "whole store rounds");
  static constexpr int W_KD = KL_BYTES;
  static constexpr int W_DS = W_KD + KD_BYTES;
  static_assert(32 * CS_STRIDE <= W_DS, "staged rows fit the K tiles");
  static constexpr int W_SC = W_DS + DS_BYTES;
  static constexpr int WAVE_BYTES = (W_SC + (FP8 ? 32 * 4 : 0) + 15) / 16 * 16;
  static constexpr int DQ_PART_BYTES = 32 * D_QK * 4;    // one wave's fp32 dQ tile
  static constexpr int LOOP_BYTES = SHARED_BYTES + WPT * WAVE_BYTES;
  static constexpr int COMBINE_BYTES = DQ_PART_BYTES;        // each wave hands over half its tiles
  static constexpr int LDS_BYTES = LOOP_BYTES > COMBINE_BYTES ? LOOP_BYTES : COMBINE_BYTES;
  static constexpr int DQT = D_QK / 32;
  static constexpr int DVT = D_V / 32;
  // bf16 source of K / V rows for the dP / dQ GEMMs
  static constexpr int K_STRIDE = FP8 ? KD_STRIDE : Gat::KL_STRIDE;
  static_assert(D_V % 32 == 0 && D_QK % 32 == 0 && D_V <= D_QK, "unsupported head dims");
};

template <int D_QK, int D_V, bool FP8, bool F32P>
__global__ void __launch_bounds__(128) __attribute__((amdgpu_waves_per_eu(D_QK <= 128 ? 2 : 1)))
sparse_mla_bwd_main_kernel(const BwdParams p) {
  using C = BwdCfg<D_QK, D_V, FP8, F32P>;
  static_assert(C::WPT == 2, "launch bounds assume two waves per workgroup");
  using Gat = typename C::Gat;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

  const int lane = lane_id(), w = __builtin_amdgcn_readfirstlane(wave_id());
  const int g32 = lane >> 5, l32 = lane & 31;
  // item = (tok * G + g) * ntiles + tile, tok = b * S + s; every factor is
  // below 2^31 (checked on the host), so 32-bit divisions suffice
  const uint32_t item = (uint32_t)xcd_remap(blockIdx.x, gridDim.x);
  const uint32_t ntl = (uint32_t)p.ntiles, ng = (uint32_t)p.G;
  const uint32_t rest = ntl == 1 ? item : item / ntl;
  const int tile = (int)(item - rest * ntl);
  const int64_t tok = ng == 1 ? rest : rest / ng;
  const int64_t g = (int64_t)rest - tok * (int64_t)ng;
  const int64_t b = (int64_t)((uint32_t)tok / (uint32_t)p.S);

  unsigned char *QL = smem + C::OFF_QL;
  unsigned char *DOL = smem + C::OFF_DOL;
  float *LD = reinterpret_cast<float *>(smem + C::OFF_LD);
  unsigned char *wsm = smem + C::SHARED_BYTES + w * C::WAVE_BYTES;
  unsigned char *Kl = wsm;
  unsigned char *Kd = wsm + C::W_KD;
  unsigned char *DS = wsm + C::W_DS;
  float *Ksc = reinterpret_cast<float *>(wsm + C::W_SC);
  const unsigned char *Ksrc = FP8 ? Kd : Kl;

  const int64_t head0 = tok * p.H + g * p.hpg + tile * 32;  // q row of head 0 of this tile
  const int nheads = p.hpg - tile * 32 < 32 ? p.hpg - tile * 32 : 32;
  const int64_t entry0 = (tok * p.G + g) * p.topk;  // entry (CSR key) of slot 0
  const int64_t n_entries = p.B * p.S * p.G * p.topk;
  const int32_t *idx_row = p.idx + entry0;
  const unsigned char *kv_b = p.kv + ((b * p.S_kv) * p.G + g) * Gat::ROWB;
  const float *kv_scale_b = FP8 ? p.kv_scale + b * p.S_kv : nullptr;
  const uint32_t row_pitch = (uint32_t)(p.G * Gat::ROWB);
  int nblk = (int)((p.topk + 31) / 32);  // set to the blocks up to the last valid slot below

  // this wave's blocks: w, w + WPT, ...
  // Indices, CSR positions and rows of a wave's next block are loaded one block
  // (indices two) ahead with unconditional loads, and the partial-row stores
  // below are unconditional too (masked lanes write a trash row past the
  // entries), so the compiler's memory waits count exactly: waiting for the
  // next block's rows never waits for this block's stores.
  int blk = w;
  const auto idx_rs = slot_rsrc(idx_row, p.topk);
  const int raw0 = load_slot_raw(idx_rs, blk, l32);
  int raw_nxt = load_slot_raw(idx_rs, blk + C::WPT, l32);
  // CSR position of an entry: its kv row's start (rowstart), plus the row's
  // entries in earlier token chunks (base[b][chunk][row]), plus the chunk's
  // earlier tokens that picked the row (the bits below this token in
  // mask[b][chunk][row]).  Where a token of the chunk repeats a row of the
  // row's part the bits cannot count the chunk's earlier entries of the row:
  // the inverse index wrote a zero mask word there and left that count (the
  // entry's rank in entry order) in pos_of (the resource is empty for chunks
  // without repeats, so the load reads nothing).
  const int64_t s_in_b = tok - b * p.S;
  const int chunk = (int)(s_in_b / kChunkTokens), tl = (int)(s_in_b % kChunkTokens);
  const uint32_t below = (1u << tl) - 1u;
  const int64_t plane = (b * p.NC + chunk) * p.R;
  const bool dupc = p.dup[b * p.NC + chunk] != 0;
  const auto mask_rs = make_buffer_rsrc(p.mask + plane, (uint32_t)(p.R * 4));
  const auto base_rs = make_buffer_rsrc(p.base + plane, (uint32_t)(p.R * 4));
  const auto rptr_rs = make_buffer_rsrc(p.rowstart + b * p.R, (uint32_t)(p.R * 4));
  const auto pos_rs = slot_rsrc(p.pos_of + entry0, dupc ? p.topk : 0);
  struct PosParts { int m, b, s, p; };
  auto load_pos_parts = [&](int idxv, int bk) {
    const uint32_t off = idxv >= 0 ? (uint32_t)(idxv * p.G + g) * 4u : 0xffffffffu;
    PosParts r;
    r.m = (int)__builtin_amdgcn_raw_buffer_load_b32(mask_rs, (int)off, 0, 0);
    r.b = (int)__builtin_amdgcn_raw_buffer_load_b32(base_rs, (int)off, 0, 0);
    r.s = (int)__builtin_amdgcn_raw_buffer_load_b32(rptr_rs, (int)off, 0, 0);
    r.p = load_slot_raw(pos_rs, bk, l32);
    return r;
  };
  auto csr_pos = [&](const PosParts &r) {
    return r.s + r.b + (r.m == 0 ? r.p : (int)__popc((uint32_t)r.m & below));
  };
  const auto kv_rs = make_buffer_rsrc(kv_b, (uint32_t)(p.S_kv * (int64_t)row_pitch));
  const auto sc_rs = make_buffer_rsrc(kv_scale_b, FP8 ? (uint32_t)(p.S_kv * 4) : 0u);
  // partial row no entry owns (this workgroup's trash row).  A pass's partial
  // rows (trash rows included) stay below 4 GiB (the host caps a pass below
  // it), so row numbers and byte offsets into them are 32-bit, and the stores
  // take a scalar base plus a 32-bit offset
  const uint32_t trash = (uint32_t)n_entries * (uint32_t)p.ntiles + item % (uint32_t)kTrashRows;

  // ---------------- prologue (all waves): Q, dO tiles, Delta, LSE ----------------
  // Every load of the prologue is issued at once, through resources that end
  // at the item's last head (padded heads read zeros), before the first
  // block's gather: one memory round trip instead of one per loop step.
  constexpr int NT = 64 * C::WPT;
  constexpr int QCH = D_QK / 8;   // 8-element chunks per q row
  constexpr int VCH = D_V / 8;    // 8-element chunks per dO / O row
  constexpr int QIT = (32 * QCH + NT - 1) / NT;
  constexpr int VIT = (32 * VCH + NT - 1) / NT;
  static_assert(VCH <= 16 && (VCH & (VCH - 1)) == 0, "d_v chunks per head: power of two <= 16");
  const int t = threadIdx.x;
  const auto q_rs = make_buffer_rsrc(p.q + head0 * D_QK * (FP8 ? 1 : 2), (uint32_t)(nheads * D_QK * (FP8 ? 1 : 2)));
  const auto do_rs = make_buffer_rsrc(p.dO + head0 * D_V, (uint32_t)(nheads * D_V * 2));
  const auto o_rs = make_buffer_rsrc(p.o + head0 * D_V, (uint32_t)(nheads * D_V * 2));
  const auto lse_rs = make_buffer_rsrc(p.lse + head0, (uint32_t)(nheads * 4));
  i32x4 qv[QIT], dv[VIT], ov[VIT];
#pragma unroll
  for (int it = 0; it < QIT; ++it) {
    const int u = t + NT * it;  // (head u / QCH, chunk u % QCH); u past 32 rows lands past the resource
    if constexpr (FP8) {
      const auto r = __builtin_amdgcn_raw_buffer_load_b64(q_rs, u * 8, 0, 0);
      qv[it] = i32x4{(int)r[0], (int)r[1], 0, 0};
    } else {
      qv[it] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(q_rs, u * 16, 0, 0));
    }
  }
#pragma unroll
  for (int it = 0; it < VIT; ++it) {
    const int u = t + NT * it;
    dv[it] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(do_rs, u * 16, 0, 0));
    ov[it] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(o_rs, u * 16, 0, 0));
  }
  const float lse_raw = buffer_load_f32(lse_rs, (t & 31) * 4, 0);
  float qsc = 1.0f;
  if constexpr (FP8) qsc = p.q_scale[tok];

  int idx_cur = slot_index(raw0, blk, l32, p.topk, p.S_kv);
  typename Gat::Regs rg;
  gather_issue<Gat>(rg, kv_rs, sc_rs, idx_cur, row_pitch);
  PosParts pp_cur = load_pos_parts(idx_cur, blk);
  // blocks up to the last valid slot (loads issued after the prologue's, so they overlap)
  nblk = valid_blocks(idx_rs, p.topk, p.S_kv);

  {
    // Q rows: 32 heads x QCH chunks of 8 elements (e4m3: dequantised to bf16)
#pragma unroll
    for (int it = 0; it < QIT; ++it) {
      const int u = t + NT * it;
      if ((32 * QCH) % NT == 0 || u < 32 * QCH) {
        const int h = u / QCH, c = u % QCH;
        i32x4 v = qv[it];
        if constexpr (FP8) {
          uint32_t wq[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {  // codes 2e, 2e + 1 of the 8 in qv[it][0..1]
            const f32x2 v2 = e4m3x2_to_f32((uint32_t)qv[it][e >> 1], (e & 1) != 0);
            wq[e] = pack_bf16x2(v2[0] * qsc, v2[1] * qsc);
          }
          v = i32x4{(int)wq[0], (int)wq[1], (int)wq[2], (int)wq[3]};
        }
        *reinterpret_cast<i32x4 *>(QL + h * C::QL_STRIDE + c * 16) = v;
      }
    }
    // dO rows and Delta = sum_d O dO (VCH consecutive threads share a head)
#pragma unroll
    for (int it = 0; it < VIT; ++it) {
      const int u = t + NT * it;
      const int h = u / VCH, c = u % VCH;
      const bool in_tile = (32 * VCH) % NT == 0 || u < 32 * VCH;
      if (in_tile) *reinterpret_cast<i32x4 *>(DOL + h * C::DOL_STRIDE + c * 16) = dv[it];
      float part = 0.0f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t du = (uint32_t)dv[it][e], ou = (uint32_t)ov[it][e];
        part += bf16_bits_to_f32(ou & 0xffffu) * bf16_bits_to_f32(du & 0xffffu);
        part += bf16_bits_to_f32(ou >> 16) * bf16_bits_to_f32(du >> 16);
      }
#pragma unroll
      for (int off = 1; off < VCH; off <<= 1) part += __shfl_xor(part, off, 64);
      if (in_tile && c == 0) {
        float dl = part;
        if (p.delta != nullptr && h < nheads) dl = p.delta[head0 + h];
        LD[32 + h] = dl * p.scale;
      }
    }
    if (t < 32) {
      float lse_h = INFINITY;  // padded heads: P = exp2(x - inf) = 0
      if (t < nheads) lse_h = (lse_raw == -INFINITY) ? INFINITY : lse_raw;  // all-masked row: zero gradient
      LD[t] = lse_h;
    }
    if constexpr (C::BEXP) {
      // max |Q| and max |dO| over the item (padded heads read zeros): the bound
      // of every partial row's magnitude below
      float mq = 0.0f, md = 0.0f;
#pragma unroll
      for (int it = 0; it < QIT; ++it)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t u = (uint32_t)qv[it][e];
          mq = fmaxf(mq, fmaxf(__uint_as_float((u << 16) & 0x7fff0000u), __uint_as_float(u & 0x7fff0000u)));
        }
#pragma unroll
      for (int it = 0; it < VIT; ++it)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t u = (uint32_t)dv[it][e];
          md = fmaxf(md, fmaxf(__uint_as_float((u << 16) & 0x7fff0000u), __uint_as_float(u & 0x7fff0000u)));
        }
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) {
        mq = fmaxf(mq, __shfl_xor(mq, off, 64));
        md = fmaxf(md, __shfl_xor(md, off, 64));
      }
      if (lane == 0) {
        LD[64 + 2 * w] = mq;
        LD[65 + 2 * w] = md;
      }
    }
  }
  __syncthreads();

  // bf16 path: the S / dP A operands (head l32, d = 16k + 8 g32 + e) stay in registers
  i32x4 qA[C::REGQ ? C::KSTEPS : 1], doA[C::REGQ ? C::VSTEPS : 1];
  float maxq = 0.0f, maxdo = 0.0f;
  if constexpr (C::REGQ) {
#pragma unroll
    for (int k = 0; k < C::KSTEPS; ++k)
      qA[k] = *reinterpret_cast<const i32x4 *>(QL + l32 * C::QL_STRIDE + (16 * k + 8 * g32) * 2);
#pragma unroll
    for (int k = 0; k < C::VSTEPS; ++k)
      doA[k] = *reinterpret_cast<const i32x4 *>(DOL + l32 * C::DOL_STRIDE + (16 * k + 8 * g32) * 2);
  }
  if constexpr (C::BEXP) {
    maxq = fmaxf(LD[64], LD[66]);
    maxdo = fmaxf(LD[65], LD[67]);
  }

  // e4m3: raw Q codes as the A operand of S on the 32x32x64 f8f6f4 MFMA (unit
  // block scales; lane (head l32, half g32) holds channels [16 g32, +16) and
  // [32 + 16 g32, +16) of each 64-channel chunk)
  constexpr int K8 = D_QK / 64;
  static_assert(!FP8 || D_QK % 64 == 0, "e4m3 rows come in 64-channel chunks");
  i32x8 qA8[FP8 ? K8 : 1];
  if constexpr (FP8) {
#pragma unroll
    for (int k = 0; k < K8; ++k) {
      i32x4 lo = {0, 0, 0, 0}, hi = {0, 0, 0, 0};
      if (l32 < nheads) {
        const unsigned char *qr = p.q + (head0 + l32) * D_QK + 64 * k + 16 * g32;
        lo = *reinterpret_cast<const i32x4 *>(qr);
        hi = *reinterpret_cast<const i32x4 *>(qr + 32);
      }
      qA8[k] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
  }
  f32x16 dqacc[C::DQT];
#pragma unroll
  for (int t = 0; t < C::DQT; ++t)
#pragma unroll
    for (int a = 0; a < 16; ++a) dqacc[t][a] = 0.0f;

  // The first block's rows and CSR positions have landed before the loop (its
  // first use waits for them anyway).  With nothing in flight on entry, the
  // compiler's memory waits inside the loop follow the loop's own order only,
  // so waiting for the next block's rows and positions leaves this block's
  // partial-row stores (issued after them) in flight; without it the waits at
  // the loop head drain every store.  (s_waitcnt vmcnt(0) with expcnt and
  // lgkmcnt left open, gfx9 encoding.)
  __builtin_amdgcn_s_waitcnt(0x0F70);
  for (; blk < nblk; blk += C::WPT) {
    const int slot0 = blk * 32;
    // ---- stage block: K rows (+ e4m3: dequantised rows, scales) ----
    gather_store_k<Gat>(rg, Kl);
    if constexpr (FP8) {
      gather_store_dequant<Gat, Gat::NCH>(rg, Kd, C::KD_STRIDE);
      gather_store_scale<Gat>(rg, Ksc);
    }
    const bool valid = idx_cur >= 0;  // slot slot0 + l32
    const int32_t pos = csr_pos(pp_cur);
    const bool wr = valid && pos >= 0 && pos < n_entries;  // (always true for a valid slot; a guard)
    const uint32_t prow_me = wr ? (uint32_t)pos * (uint32_t)p.ntiles + (uint32_t)tile : trash;
    wave_lds_sync();
    const int raw_nn = load_slot_raw(idx_rs, blk + 2 * C::WPT, l32);
    const int idx_nxt = slot_index(raw_nxt, blk + C::WPT, l32, p.topk, p.S_kv);
    gather_issue<Gat>(rg, kv_rs, sc_rs, idx_nxt, row_pitch);
    const PosParts pp_nxt = load_pos_parts(idx_nxt, blk + C::WPT);

    // ---- S = Q K^T and dP = dO V^T  (M = head, N = slot; Q / dO rows from LDS) ----
    f32x16 sacc, dpacc;
#pragma unroll
    for (int a = 0; a < 16; ++a) {
      sacc[a] = 0.0f;
      dpacc[a] = 0.0f;
    }
#pragma unroll
    for (int k = 0; k < (FP8 ? K8 : C::KSTEPS); ++k) {
      if constexpr (FP8) {
        const unsigned char *kr = Kl + l32 * Gat::KL_STRIDE + 64 * k + 16 * g32;
        const i32x4 lo = *reinterpret_cast<const i32x4 *>(kr);
        const i32x4 hi = *reinterpret_cast<const i32x4 *>(kr + 32);
        const i32x8 kb = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        sacc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(qA8[k], kb, sacc, 0, 0, 0, 127, 0, 127);
      } else {
        // V is the leading D_V columns of K: one K read feeds S and dP
        const i32x4 kb = *reinterpret_cast<const i32x4 *>(Kl + l32 * Gat::KL_STRIDE + (16 * k + 8 * g32) * 2);
        const i32x4 qa =
            C::REGQ ? qA[C::REGQ ? k : 0]
                    : *reinterpret_cast<const i32x4 *>(QL + l32 * C::QL_STRIDE + (16 * k + 8 * g32) * 2);
        sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(qa), as_bf16x8(kb), sacc, 0, 0, 0);
        if (k < C::VSTEPS) {
          const i32x4 da =
              C::REGQ ? doA[C::REGQ ? k : 0]
                      : *reinterpret_cast<const i32x4 *>(DOL + l32 * C::DOL_STRIDE + (16 * k + 8 * g32) * 2);
          dpacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(da), as_bf16x8(kb), dpacc, 0, 0, 0);
        }
      }
    }
    if constexpr (FP8) {  // dP on the dequantised rows
#pragma unroll
      for (int k = 0; k < C::VSTEPS; ++k) {
        const i32x4 da = *reinterpret_cast<const i32x4 *>(DOL + l32 * C::DOL_STRIDE + (16 * k + 8 * g32) * 2);
        const i32x4 vb = *reinterpret_cast<const i32x4 *>(Ksrc + l32 * C::K_STRIDE + (16 * k + 8 * g32) * 2);
        dpacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(da), as_bf16x8(vb), dpacc, 0, 0, 0);
      }
    }

    // ---- P, dS  (lane = slot slot0 + l32, heads 8i + 4*g32 + j) ----
    float xs = p.sl2;
    if constexpr (FP8) xs *= qsc * Ksc[l32];
    bf16x8 dsB[2], pB[2];
    int pexp = 0;  // bf16 path: the partial row's scale exponent, fixed before its products
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
          const float pv = valid ? exp2_fast(sacc[a] * xs - l4[j]) : 0.0f;
          P[a] = pv;
          dS[a] = pv * fmaf(dpacc[a], p.scale, -d4[j]);  // P (dP - Delta) scale
          sabs += fabsf(dS[a]);
          psum += pv;
        }
        dsw[2 * i] = pack_bf16x2(dS[4 * i], dS[4 * i + 1]);
        dsw[2 * i + 1] = pack_bf16x2(dS[4 * i + 2], dS[4 * i + 3]);
        // dS[slot][heads 8i + 4*g32 .. +3] row-major for the dQ GEMM
        *reinterpret_cast<i32x2 *>(DS + l32 * C::DS_STRIDE + (8 * i + 4 * g32) * 2) =
            i32x2{(int)dsw[2 * i], (int)dsw[2 * i + 1]};
      }
      float rs = 1.0f;
      if constexpr (C::BEXP) {
        // |c[d]| <= max|Q| sum_h |dS_h| + max|dO| sum_h P_h over the slot's 32
        // heads; the margin 2^-6 covers the bf16 rounding of dS / P (2^-8) and
        // the fp32 sums (< 2^-17)
        const float bnd = sum_halves(fmaf(maxq, sabs, maxdo * psum)) * 1.015625f;
        pexp = partial_row_exponent_bound(bnd);
        rs = exp2i(pexp);
#pragma unroll
        for (int i = 0; i < 4; ++i) {  // bf16(x 2^s) = bf16(x) 2^s: the scaled rows are exact
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
    wave_lds_sync();

    // ---- dQ^T[d][head] += K^T[d][slot] dS^T[slot][head]  (M = d, N = head, K = slot) ----
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      const i32x4 bv = tr_operand(DS, C::DS_STRIDE, 0, 16 * kc, 4, 8);
#pragma unroll
      for (int dt = 0; dt < C::DQT; ++dt) {
        const i32x4 av = tr_operand(Ksrc, C::K_STRIDE, dt * 32, 16 * kc, 4, 8);
        dqacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(av), as_bf16x8(bv), dqacc[dt], 0, 0, 0);
      }
    }

    if constexpr (C::BEXP) {
      // ---- c^T[d][slot] = Q^T dS^T + dO^T P^T, one 32-row d-tile at a time ----
      // dS and P already carry the row's 2^pexp, so each d-tile is converted to
      // fp16 and staged (over the consumed K tile) right after its MFMAs: one
      // 16-register accumulator instead of four, which leaves the registers
      // for the LDS operand reads to run ahead of the MFMAs.
      wave_lds_sync();  // the dQ GEMM's reads of the K / dS tiles are complete
      unsigned char *Cs = Kl;
      int *Lpos = reinterpret_cast<int *>(DS);
      static_assert(C::DQT % 2 == 0, "d-tiles in pairs");
#pragma unroll
      for (int dp = 0; dp < C::DQT; dp += 2) {
        // two d-tiles' independent MFMA chains, then both conversions
        f32x16 cacc[2];
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int a = 0; a < 16; ++a) cacc[u][a] = 0.0f;
#pragma unroll
        for (int kc = 0; kc < 2; ++kc)
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const i32x4 av = tr_operand_perm(QL, C::QL_STRIDE, (dp + u) * 32, 16 * kc);
            cacc[u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(av), dsB[kc], cacc[u], 0, 0, 0);
          }
#pragma unroll
        for (int kc = 0; kc < 2; ++kc)
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            if (dp + u < C::DVT) {
              const i32x4 av = tr_operand_perm(DOL, C::DOL_STRIDE, (dp + u) * 32, 16 * kc);
              cacc[u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(av), pB[kc], cacc[u], 0, 0, 0);
            }
          }
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2) {
            const int d0 = (dp + u) * 32 + 16 * s2 + 8 * g32;
            *reinterpret_cast<i32x4 *>(Cs + l32 * C::CS_STRIDE + d0 * 2) =
                i32x4{(int)pack_f16x2(cacc[u][8 * s2], cacc[u][8 * s2 + 1]),
                      (int)pack_f16x2(cacc[u][8 * s2 + 2], cacc[u][8 * s2 + 3]),
                      (int)pack_f16x2(cacc[u][8 * s2 + 4], cacc[u][8 * s2 + 5]),
                      (int)pack_f16x2(cacc[u][8 * s2 + 6], cacc[u][8 * s2 + 7])};
          }
      }
      if (g32 == 0) Lpos[l32] = (int)prow_me;  // the slot's partial row (or its trash row)
      p.partial_exp[prow_me] = (int8_t)pexp;  // both lane halves store the same byte
      wave_lds_sync();
      // all LDS reads first, then the stores, so the reads overlap
      constexpr int ITS = 32 * C::ROW_CHUNKS / 64;
      int ps[ITS];
      i32x4 v[ITS];
#pragma unroll
      for (int it = 0; it < ITS; ++it) {
        const int u = it * 64 + lane;
        const int row = u / C::ROW_CHUNKS, ch = u % C::ROW_CHUNKS;
        ps[it] = Lpos[row];
        v[it] = *reinterpret_cast<const i32x4 *>(Cs + row * C::CS_STRIDE + ch * 16);
      }
#pragma unroll
      for (int it = 0; it < ITS; ++it) {
        const int ch = (it * 64 + lane) % C::ROW_CHUNKS;
        st_stream_16(p.partials + ((uint32_t)ps[it] * (uint32_t)(D_QK * 2) + (uint32_t)ch * 16u), v[it]);
      }
      wave_lds_sync();  // K / dS tiles are consumed before the next block's gather lands
      idx_cur = idx_nxt;
      raw_nxt = raw_nn;
      pp_cur = pp_nxt;
      continue;
    }

    // ---- c^T[d][slot] = Q^T dS^T + dO^T P^T  (M = d, N = slot, K = head, accumulator order) ----
    f32x16 cacc[C::DQT];
#pragma unroll
    for (int dt = 0; dt < C::DQT; ++dt) {
#pragma unroll
      for (int a = 0; a < 16; ++a) cacc[dt][a] = 0.0f;
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        const i32x4 av = tr_operand_perm(QL, C::QL_STRIDE, dt * 32, 16 * kc);
        cacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(av), dsB[kc], cacc[dt], 0, 0, 0);
      }
      if (dt < C::DVT) {
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) {
          const i32x4 av = tr_operand_perm(DOL, C::DOL_STRIDE, dt * 32, 16 * kc);
          cacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(av), pB[kc], cacc[dt], 0, 0, 0);
        }
      }
    }

    // ---- the slot's partial row, written at its CSR position ----
    // lane: slot l32, d = dt*32 + 16(i>>1) + 8*g32 + 4(i&1) + j (the permuted Q^T / dO^T columns).
    if constexpr (F32P) {
      // fp32 rows: the two lanes of a slot store adjacent 16-byte pieces, with
      // plain (write-back) stores so that L2 merges a row's pieces into lines
      unsigned char *dst = p.partials + prow_me * (uint32_t)(D_QK * 4);
#pragma unroll
      for (int dt = 0; dt < C::DQT; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int d0 = dt * 32 + 16 * (i >> 1) + 8 * g32 + 4 * (i & 1);
          *reinterpret_cast<f32x4 *>(dst + d0 * 4) = f32x4{cacc[dt][4 * i], cacc[dt][4 * i + 1],
                                                           cacc[dt][4 * i + 2], cacc[dt][4 * i + 3]};
        }
    } else {
      // fp16 rows scaled by a power of two mapping the row max into [2^13, 2^14)
      // (exact to undo), staged in LDS (over the consumed K tile) and written
      // as whole rows: 16 lanes store one row's 256 contiguous bytes
      float rscale = 1.0f;  // bf16 path: c already carries 2^pexp
      if constexpr (!C::BEXP) {
        float amax = 0.0f;
#pragma unroll
        for (int dt = 0; dt < C::DQT; ++dt)
#pragma unroll
          for (int a = 0; a < 16; ++a) amax = fmaxf(amax, fabsf(cacc[dt][a]));
        amax = max_halves(amax);
        pexp = partial_row_exponent(amax);
        rscale = exp2i(pexp);
      }
      wave_lds_sync();  // the dQ GEMM's reads of the K / dS tiles are complete
      unsigned char *Cs = Kl;  // spans Kl (and Kd for e4m3)
      int *Lpos = reinterpret_cast<int *>(DS);
#pragma unroll
      for (int dt = 0; dt < C::DQT; ++dt)
#pragma unroll
        for (int s = 0; s < 2; ++s) {  // d = dt*32 + 16s + 8*g32 + (0..7): cacc[dt][8s .. 8s+7]
          const int d0 = dt * 32 + 16 * s + 8 * g32;
          *reinterpret_cast<i32x4 *>(Cs + l32 * C::CS_STRIDE + d0 * 2) =
              i32x4{(int)pack_f16x2(cacc[dt][8 * s] * rscale, cacc[dt][8 * s + 1] * rscale),
                    (int)pack_f16x2(cacc[dt][8 * s + 2] * rscale, cacc[dt][8 * s + 3] * rscale),
                    (int)pack_f16x2(cacc[dt][8 * s + 4] * rscale, cacc[dt][8 * s + 5] * rscale),
                    (int)pack_f16x2(cacc[dt][8 * s + 6] * rscale, cacc[dt][8 * s + 7] * rscale)};
        }
      if (g32 == 0) Lpos[l32] = (int)prow_me;  // the slot's partial row (or its trash row)
      p.partial_exp[prow_me] = (int8_t)pexp;  // both lane halves store the same byte
      wave_lds_sync();
      // all LDS reads first, then the stores, so the reads overlap
      constexpr int ITS = 32 * C::ROW_CHUNKS / 64;
      int ps[ITS];
      i32x4 v[ITS];
#pragma unroll
      for (int it = 0; it < ITS; ++it) {
        const int u = it * 64 + lane;
        const int row = u / C::ROW_CHUNKS, ch = u % C::ROW_CHUNKS;
        ps[it] = Lpos[row];
        v[it] = *reinterpret_cast<const i32x4 *>(Cs + row * C::CS_STRIDE + ch * 16);
      }
#pragma unroll
      for (int it = 0; it < ITS; ++it) {
        const int ch = (it * 64 + lane) % C::ROW_CHUNKS;
        st_stream_16(p.partials + ((uint32_t)ps[it] * (uint32_t)(D_QK * 2) + (uint32_t)ch * 16u), v[it]);
      }
    }
    wave_lds_sync();  // K / dS tiles are consumed before the next block's gather lands
    idx_cur = idx_nxt;
    raw_nxt = raw_nn;
    pp_cur = pp_nxt;
  }

  // ---- combine the two waves' dQ partial sums, then write dQ ----
  // Wave w keeps d-tiles [w * HT, w * HT + HT) and hands the other half to its
  // partner through LDS; both add in wave order (wave 0's sum + wave 1's), so
  // the result does not depend on which wave writes a tile.
  constexpr int HT = C::DQT / 2;
  static_assert(C::DQT % 2 == 0, "d-tiles split evenly between the two waves");
  __syncthreads();  // every wave is done with the loop's LDS
  float *dqp = reinterpret_cast<float *>(smem);  // [exporter][tile][16][64]
  auto export_tiles = [&](int first) {
#pragma unroll
    for (int tt = 0; tt < HT; ++tt)
#pragma unroll
      for (int a = 0; a < 16; ++a) dqp[((w * HT + tt) * 16 + a) * 64 + lane] = dqacc[first + tt][a];
  };
  auto finish_tiles = [&](int first) {
#pragma unroll
    for (int tt = 0; tt < HT; ++tt) {
      const int dt = first + tt;
#pragma unroll
      for (int a = 0; a < 16; ++a) {
        const float other = dqp[(((1 - w) * HT + tt) * 16 + a) * 64 + lane];
        dqacc[dt][a] = w == 0 ? dqacc[dt][a] + other : other + dqacc[dt][a];
      }
      // lane = head l32, d = dt*32 + 8i + 4*g32 + j
      if (l32 < nheads) {
        uint16_t *drow = p.dq + (head0 + l32) * D_QK;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const i32x2 pk = {(int)pack_bf16x2(dqacc[dt][4 * i], dqacc[dt][4 * i + 1]),
                            (int)pack_bf16x2(dqacc[dt][4 * i + 2], dqacc[dt][4 * i + 3])};
          *reinterpret_cast<i32x2 *>(drow + dt * 32 + 8 * i + 4 * g32) = pk;
        }
      }
    }
  };
  if (w == 0) export_tiles(HT); else export_tiles(0);
  __syncthreads();
  if (w == 0) finish_tiles(0); else finish_tiles(HT);
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Passes of the backward.  A pass is a contiguous range of the flattened
// [B * S] tokens: whole batches while their partial rows fit the per-pass cap,
// else a slice of one batch (a multiple of 32 tokens).  Each pass builds its
// own inverse index, runs the main kernel on its tokens and reduces its
// partial rows; when a batch spans several passes the kv rows' sums are
// carried between them in fp32 (first pass stores, later passes add, the
// last casts to bf16), in pass order, so the result stays deterministic.
constexpr uint64_t kBwdPassBytes = 4ull << 30;  // default: partial rows (+ exponents) per pass
// A pass's partial rows stay below 4 GiB (the main kernel addresses them
// with 32-bit offsets): caps at or above this are lowered to it.
constexpr uint64_t kBwdPassMax = (4ull << 30) - (1ull << 20);

// The per-pass cap of a call: its pass_bytes argument, 0 meaning the default,
// at most kBwdPassMax.
static uint64_t pass_cap(uint64_t pass_bytes) {
  const uint64_t cap = pass_bytes == 0 ? kBwdPassBytes : pass_bytes;
  return cap < kBwdPassMax ? cap : kBwdPassMax;
}

struct BwdPlan {
  int64_t nb;   // batches per pass
  int64_t ct;   // tokens of one batch per pass (S unless a batch is split)
  int64_t npb;  // passes per batch (1 unless split)
  int NC;       // 32-token chunks per batch within a pass
};

// bytes per partial element: fp32 with DSA_BWD_FP32_PARTIALS, else fp16
static int64_t partial_elem_bytes(int flags, int64_t D_qk) {
  (void)D_qk;
  return (flags & DSA_BWD_FP32_PARTIALS) ? 4 : 2;
}

static BwdPlan bwd_plan(int64_t B, int64_t S, int64_t H, int64_t G, int64_t D_qk, int64_t topk, int flags,
                        uint64_t cap) {
  const int64_t hpg = H / (G > 0 ? G : 1);
  const int64_t ntiles = (hpg + 31) / 32;
  const uint64_t per_token = (uint64_t)(G * topk * ntiles) * (uint64_t)(D_qk * partial_elem_bytes(flags, D_qk) + 1);
  BwdPlan pl;
  if ((uint64_t)S * per_token <= cap) {
    pl.ct = S;
    pl.npb = 1;
    const int64_t fit = (int64_t)(cap / ((uint64_t)S * per_token));
    pl.nb = fit < 1 ? 1 : (fit < B ? fit : B);
  } else {
    int64_t ct = (int64_t)(cap / per_token) / kChunkTokens * kChunkTokens;
    pl.ct = ct < kChunkTokens ? kChunkTokens : ct;
    pl.npb = (S + pl.ct - 1) / pl.ct;
    pl.nb = 1;
  }
  pl.NC = csr_chunks(pl.ct);
  return pl;
}

// Workspace: the partial-row section (rows, exponents, carry) and the
// inverse-index section (per 32-token chunk and kv row a token bitmask and a
// base word, chunk flags, row totals and starts, CSR positions), each sized for
// one pass.  dsa_sparse_mla_bwd takes both in one buffer (rows first);
// dsa_sparse_mla_bwd_indexed takes the index section as a separate buffer that
// dsa_sparse_mla_bwd_build_index filled ahead of the call.
struct BwdWorkspace {
  size_t partials, pexp, carry, rows_total;          // offsets in the rows section
  size_t mask, base, dup, dupc, tot, rowstart, pos_of, next, index_total;  // offsets in the index section
  size_t total;                                      // rows section + index section
  BwdPlan plan;
};

static BwdWorkspace bwd_layout(int64_t B, int64_t S, int64_t S_kv, int64_t H, int64_t G, int64_t D_qk,
                               int64_t topk, int flags, uint64_t pass_bytes) {
  const int64_t hpg = H / (G > 0 ? G : 1);
  const int ntiles = (int)((hpg + 31) / 32);
  BwdWorkspace L;
  L.plan = bwd_plan(B, S, H, G, D_qk, topk, flags, pass_cap(pass_bytes));
  const BwdPlan &pl = L.plan;
  const size_t entries = (size_t)pl.nb * pl.ct * G * topk;  // of one pass
  const int64_t R = S_kv * G;
  const size_t psz = (size_t)partial_elem_bytes(flags, D_qk);
  size_t off = 0;
  L.partials = off;
  off += align256((entries * ntiles + kTrashRows) * D_qk * psz);  // + trash rows for masked slots
  L.pexp = off;
  off += align256(entries * ntiles + kTrashRows);
  L.carry = off;  // fp32 sums of one batch's kv rows, carried across its passes
  off += pl.npb > 1 ? align256((size_t)R * D_qk * 4) : 0;
  L.rows_total = off;
  off = 0;
  L.mask = off;
  off += align256((size_t)pl.nb * pl.NC * R * 4);
  L.base = off;
  off += align256((size_t)pl.nb * pl.NC * R * 4);
  // row parts per chunk: a pass with fewer chunks takes more parts, at most
  // max(16, R / 16384 rounded up)
  const int64_t spl_max = (R + 16383) / 16384 > 16 ? (R + 16383) / 16384 : 16;
  L.dup = off;
  off += align256((size_t)pl.nb * pl.NC * spl_max * 4);
  L.dupc = off;
  off += align256((size_t)pl.nb * pl.NC * 4);
  L.tot = off;
  off += align256((size_t)pl.nb * R * 4);
  L.rowstart = off;
  off += align256((size_t)pl.nb * R * 4);
  L.pos_of = off;
  off += align256(entries * 4);
  L.next = off;
  off += align256((size_t)pl.nb * 4);
  L.index_total = off;
  L.total = L.rows_total + L.index_total;
  return L;
}

static int64_t bwd_passes(const BwdPlan &pl, int64_t B) {
  return pl.npb > 1 ? B * pl.npb : (B + pl.nb - 1) / pl.nb;
}

// The inverse index of one pass (tokens [T0, T0 + nbp * ctp) of the flattened
// [B * S]) in the index section ix.
static CsrParams bwd_csr_params(const int32_t *indices, const BwdWorkspace &L, unsigned char *ix, int64_t T0,
                                int64_t nbp, int64_t ctp, int64_t S_kv, int64_t G, int64_t topk, bool wide) {
  CsrParams cp;
  cp.idx = indices + T0 * G * topk;
  cp.mask = reinterpret_cast<uint32_t *>(ix + L.mask);
  cp.base = reinterpret_cast<int32_t *>(ix + L.base);
  cp.dup = reinterpret_cast<int32_t *>(ix + L.dup);
  cp.dupc = reinterpret_cast<int32_t *>(ix + L.dupc);
  cp.tot = reinterpret_cast<int32_t *>(ix + L.tot);
  cp.rowstart = reinterpret_cast<int32_t *>(ix + L.rowstart);
  cp.pos_of = reinterpret_cast<int32_t *>(ix + L.pos_of);
  cp.S = ctp;
  cp.S_kv = S_kv;
  cp.G = G;
  cp.topk = topk;
  cp.R = S_kv * G;
  cp.NC = csr_chunks(ctp);
  cp.SPL = csr_split((int64_t)cp.NC * nbp, cp.R);
  cp.RP = (cp.R + cp.SPL - 1) / cp.SPL;
  cp.local_ranks = wide ? 0 : 1;  // the narrow main kernel derives every position itself
  cp.next = reinterpret_cast<int32_t *>(ix + L.next);
  return cp;
}

template <int D_QK, int D_V, bool FP8, bool F32P>
static int launch_bwd_main(const BwdParams &p, hipStream_t st) {
  using C = BwdCfg<D_QK, D_V, FP8, F32P>;
  const size_t lds = C::LDS_BYTES;
  if (lds > 160 * 1024) return set_error(DSA_ERR_UNSUPPORTED, "sparse_mla_bwd: needs %zu bytes of LDS", lds);
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute((const void *)sparse_mla_bwd_main_kernel<D_QK, D_V, FP8, F32P>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return set_error(DSA_ERR_HIP, "sparse_mla_bwd: LDS attribute: %s", hipGetErrorString(e));
  }
  const int64_t nitems = p.B * p.S * p.G * p.ntiles;  // one workgroup per item
  if (nitems >= (1ll << 31)) return set_error(DSA_ERR_INVALID_ARG, "sparse_mla_bwd: grid too large");
  hipLaunchKernelGGL((sparse_mla_bwd_main_kernel<D_QK, D_V, FP8, F32P>), dim3((unsigned)nitems),
                     dim3(64 * C::WPT), lds, st, p);
  return check_launch("sparse_mla_bwd_main");
}

template <int D_QK, int D_V, bool FP8>
static int launch_bwd_main_p(const BwdParams &p, bool f32p, hipStream_t st) {
  return f32p ? launch_bwd_main<D_QK, D_V, FP8, true>(p, st) : launch_bwd_main<D_QK, D_V, FP8, false>(p, st);
}

template <int D_QK>
static int launch_reduce(const CsrParams &cp, const unsigned char *partials, const int8_t *pexp, uint16_t *dkv,
                         float *carry, int mode, int64_t rows, int ntiles, bool f32p, hipStream_t st) {
  const unsigned grid = (unsigned)rows;  // one workgroup per kv row
  if (f32p)
    hipLaunchKernelGGL((dkv_reduce_kernel<D_QK, true>), dim3(grid), dim3(256), 0, st, cp.rowstart, cp.tot,
                       partials, pexp, dkv, carry, mode, rows, ntiles);
  else
    hipLaunchKernelGGL((dkv_reduce_kernel<D_QK, false>), dim3(grid), dim3(256), 0, st, cp.rowstart, cp.tot,
                       partials, pexp, dkv, carry, mode, rows, ntiles);
  return check_launch("sparse_mla_bwd(reduce)");
}

}  // namespace dsa

using namespace dsa;

extern "C" size_t dsa_sparse_mla_bwd_workspace_size(int64_t B, int64_t S, int64_t S_kv, int64_t H, int64_t G,
                                                    int64_t D_qk, int64_t D_v, int64_t topk, int flags,
                                                    uint64_t pass_bytes) {
  (void)D_v;
  if (B <= 0 || S <= 0 || S_kv <= 0 || H <= 0 || G <= 0 || topk <= 0 || D_qk <= 0) return 0;
  return bwd_layout(B, S, S_kv, H, G, D_qk, topk, flags, pass_bytes).total;
}

static int bwd_check(const char *fn, int64_t B, int64_t S, int64_t S_kv, int64_t H, int64_t G, int64_t D_qk,
                     int64_t D_v, int64_t topk, int dtype, int flags) {
  DSA_REQUIRE(B >= 0 && S >= 0 && S_kv > 0 && H > 0 && G > 0 && topk > 0,
              "%s: bad dims B=%lld S=%lld S_kv=%lld H=%lld G=%lld topk=%lld", fn, (long long)B, (long long)S,
              (long long)S_kv, (long long)H, (long long)G, (long long)topk);
  DSA_REQUIRE(H % G == 0, "%s: H=%lld not divisible by G=%lld", fn, (long long)H, (long long)G);
  DSA_REQUIRE(D_v > 0 && D_v <= D_qk, "%s: need 0 < d_v <= d_qk", fn);
  DSA_REQUIRE(dtype == DSA_DTYPE_BF16 || dtype == DSA_DTYPE_E4M3, "%s: dtype %d", fn, dtype);
  DSA_REQUIRE((flags & ~DSA_BWD_FP32_PARTIALS) == 0, "%s: unknown flags 0x%x", fn, flags);
  const int64_t R = S_kv * G;
  const int64_t entries = B * S * G * topk;
  const int64_t ntiles = (H / G + 31) / 32;
  DSA_REQUIRE(entries < (1ll << 31) && B * R < (1ll << 31) && entries * ntiles < (1ll << 40),
              "%s: too many entries for int32 CSR keys", fn);
  DSA_REQUIRE(S_kv * G * D_qk * 2 <= (int64_t)kMaskedOff, "%s: kv rows of one batch exceed 4 GiB - 64 KiB", fn);
  const bool f8 = dtype == DSA_DTYPE_E4M3;
  const bool shape_ok = (D_qk == 128 && D_v == 64) || (D_qk == 128 && D_v == 128) || (D_qk == 192 && D_v == 128) ||
                        (D_qk == 64 && D_v == 32 && !f8) || wide_shape(D_qk, D_v);
  if (!shape_ok)
    return set_error(DSA_ERR_UNSUPPORTED, "%s: no kernel for d_qk=%lld d_v=%lld dtype=%d", fn, (long long)D_qk,
                     (long long)D_v, dtype);
  return DSA_OK;
}

// Main kernel, reduction (and, unless index_ready, the inverse index) of every pass.
static int bwd_run(const void *q, const void *kv, const void *o, const void *dO, const int32_t *indices,
                   const float *lse2, const float *delta, void *dq, void *dkv, unsigned char *ws, unsigned char *ix,
                   bool index_ready, int64_t B, int64_t S, int64_t S_kv, int64_t H, int64_t G, int64_t D_qk,
                   int64_t D_v, int64_t topk, float sm_scale, int dtype, const float *q_scale, const float *kv_scale,
                   int flags, const BwdWorkspace &L, hipStream_t st) {
  const int64_t R = S_kv * G;
  const int64_t hpg = H / G;
  const int ntiles = (int)((hpg + 31) / 32);
  const bool f8 = dtype == DSA_DTYPE_E4M3;
  const bool wide = wide_shape(D_qk, D_v);
  const bool f32p = (flags & DSA_BWD_FP32_PARTIALS) != 0;
  const BwdPlan &pl = L.plan;
  const int64_t npass = bwd_passes(pl, B);
  const size_t qel = f8 ? 1 : 2;  // bytes per q / kv element
  uint16_t *dkv16 = static_cast<uint16_t *>(dkv);
  float *carry = reinterpret_cast<float *>(ws + L.carry);
  // the main kernel addresses a pass's partial rows with 32-bit offsets
  DSA_REQUIRE(L.pexp <= 0xffffffffull, "sparse_mla_bwd: one pass's partial rows exceed 4 GiB (topk too large)");
  stage_begin(st);
  for (int64_t ps = 0; ps < npass; ++ps) {
    // this pass: batches [b0, b0 + nbp), tokens [t0, t0 + ctp) of each
    const int64_t b0 = pl.npb > 1 ? ps / pl.npb : ps * pl.nb;
    const int64_t nbp = pl.npb > 1 ? 1 : (B - b0 < pl.nb ? B - b0 : pl.nb);
    const int64_t t0 = pl.npb > 1 ? (ps % pl.npb) * pl.ct : 0;
    const int64_t ctp = pl.npb > 1 ? (S - t0 < pl.ct ? S - t0 : pl.ct) : S;
    const int64_t T0 = b0 * S + t0;  // first flattened token
    const int mode = pl.npb == 1 ? 0 : (ps % pl.npb == 0 ? 1 : (ps % pl.npb == pl.npb - 1 ? 3 : 2));
    const bool timed = npass == 1;

    const CsrParams cp = bwd_csr_params(indices, L, ix, T0, nbp, ctp, S_kv, G, topk, wide);
    int rc = DSA_OK;
    if (!index_ready) {
      rc = launch_csr(cp, nbp, st);
      if (rc) return rc;
    }
    if (timed) stage_mark(st);  // (a prebuilt index makes this stage empty)

    BwdParams p;
    p.q = static_cast<const unsigned char *>(q) + (size_t)T0 * H * D_qk * qel;
    p.kv = static_cast<const unsigned char *>(kv) + (size_t)b0 * S_kv * G * D_qk * qel;
    p.o = static_cast<const uint16_t *>(o) + T0 * H * D_v;
    p.dO = static_cast<const uint16_t *>(dO) + T0 * H * D_v;
    p.idx = cp.idx;
    p.lse = lse2 + T0 * H;
    p.delta = delta ? delta + T0 * H : nullptr;
    p.dq = static_cast<uint16_t *>(dq) + T0 * H * D_qk;
    p.q_scale = q_scale ? q_scale + T0 : nullptr;
    p.kv_scale = kv_scale ? kv_scale + b0 * S_kv : nullptr;
    p.pos_of = cp.pos_of;
    p.mask = cp.mask;
    p.base = cp.base;
    p.dup = cp.dupc;
    p.R = cp.R;
    p.rowstart = cp.rowstart;
    p.NC = cp.NC;
    p.partials = ws + L.partials;
    p.partial_exp = reinterpret_cast<int8_t *>(ws + L.pexp);
    p.B = nbp;
    p.S = ctp;
    p.S_kv = S_kv;
    p.H = H;
    p.G = G;
    p.topk = topk;
    p.hpg = (int)hpg;
    p.ntiles = ntiles;
    p.sl2 = sm_scale * kLog2e;
    p.scale = sm_scale;
    if (wide) rc = launch_bwd_main_wide(p, D_qk, D_v, f8, f32p, st);
    else if (D_qk == 128 && D_v == 64) rc = f8 ? launch_bwd_main_p<128, 64, true>(p, f32p, st) : launch_bwd_main_p<128, 64, false>(p, f32p, st);
    else if (D_qk == 128 && D_v == 128) rc = f8 ? launch_bwd_main_p<128, 128, true>(p, f32p, st) : launch_bwd_main_p<128, 128, false>(p, f32p, st);
    else if (D_qk == 192 && D_v == 128) rc = f8 ? launch_bwd_main_p<192, 128, true>(p, f32p, st) : launch_bwd_main_p<192, 128, false>(p, f32p, st);
    else rc = launch_bwd_main_p<64, 32, false>(p, f32p, st);
    if (rc) return rc;
    if (timed) stage_mark(st);

    uint16_t *dkv_p = dkv16 + b0 * R * D_qk;
    const int64_t prow = nbp * R;
    if (D_qk == 128) rc = launch_reduce<128>(cp, p.partials, p.partial_exp, dkv_p, carry, mode, prow, ntiles, f32p, st);
    else if (D_qk == 192) rc = launch_reduce<192>(cp, p.partials, p.partial_exp, dkv_p, carry, mode, prow, ntiles, f32p, st);
    else if (D_qk == 576) rc = launch_reduce<576>(cp, p.partials, p.partial_exp, dkv_p, carry, mode, prow, ntiles, f32p, st);
    else rc = launch_reduce<64>(cp, p.partials, p.partial_exp, dkv_p, carry, mode, prow, ntiles, f32p, st);
    if (rc) return rc;
  }
  stage_mark(st);  // several passes: one stage for the whole call
  return DSA_OK;
}

static int bwd_zero_dkv(void *dkv, int64_t rows, int64_t D_qk, hipStream_t st) {
  hipLaunchKernelGGL(fill_i32_kernel, dim3(256), dim3(256), 0, st, reinterpret_cast<int32_t *>(dkv),
                     (rows * D_qk) / 2, 0);
  return check_launch("sparse_mla_bwd(fill)");
}

extern "C" int dsa_sparse_mla_bwd(const void *q, const void *kv, const void *o, const void *dO,
                                  const int32_t *indices, const float *lse2, const float *delta, void *dq,
                                  void *dkv, void *workspace, size_t workspace_bytes, int64_t B, int64_t S,
                                  int64_t S_kv, int64_t H, int64_t G, int64_t D_qk, int64_t D_v, int64_t topk,
                                  float sm_scale, int dtype, const float *q_scale, const float *kv_scale,
                                  int flags, uint64_t pass_bytes, void *stream) {
  int rc = bwd_check("dsa_sparse_mla_bwd", B, S, S_kv, H, G, D_qk, D_v, topk, dtype, flags);
  if (rc) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (B == 0) return DSA_OK;
  DSA_REQUIRE(dkv, "dsa_sparse_mla_bwd: null dkv");
  DSA_REQUIRE(q && kv && o && dO && indices && lse2 && dq, "dsa_sparse_mla_bwd: null tensor pointer");
  if (dtype == DSA_DTYPE_E4M3)
    DSA_REQUIRE(q_scale && kv_scale, "dsa_sparse_mla_bwd: e4m3 input needs q_scale and kv_scale");
  const BwdWorkspace L = bwd_layout(B, S, S_kv, H, G, D_qk, topk, flags, pass_bytes);
  if (!workspace || workspace_bytes < L.total)
    return set_error(DSA_ERR_WORKSPACE, "dsa_sparse_mla_bwd: workspace %zu < required %zu", workspace_bytes,
                     L.total);
  if (S == 0) return bwd_zero_dkv(dkv, B * S_kv * G, D_qk, st);  // no queries: dKV is zero
  unsigned char *ws = static_cast<unsigned char *>(workspace);
  return bwd_run(q, kv, o, dO, indices, lse2, delta, dq, dkv, ws, ws + L.rows_total, false, B, S, S_kv, H, G, D_qk,
                 D_v, topk, sm_scale, dtype, q_scale, kv_scale, flags, L, st);
}

extern "C" size_t dsa_sparse_mla_bwd_index_size(int64_t B, int64_t S, int64_t S_kv, int64_t H, int64_t G,
                                                int64_t D_qk, int64_t D_v, int64_t topk, int flags,
                                                uint64_t pass_bytes) {
  (void)D_v;
  if (B <= 0 || S <= 0 || S_kv <= 0 || H <= 0 || G <= 0 || topk <= 0 || D_qk <= 0) return 0;
  const BwdWorkspace L = bwd_layout(B, S, S_kv, H, G, D_qk, topk, flags, pass_bytes);
  return bwd_passes(L.plan, B) == 1 ? L.index_total : 0;  // several passes rebuild it per pass
}

extern "C" size_t dsa_sparse_mla_bwd_indexed_workspace_size(int64_t B, int64_t S, int64_t S_kv, int64_t H,
                                                            int64_t G, int64_t D_qk, int64_t D_v, int64_t topk,
                                                            int flags, uint64_t pass_bytes) {
  (void)D_v;
  if (B <= 0 || S <= 0 || S_kv <= 0 || H <= 0 || G <= 0 || topk <= 0 || D_qk <= 0) return 0;
  return bwd_layout(B, S, S_kv, H, G, D_qk, topk, flags, pass_bytes).rows_total;
}

extern "C" int dsa_sparse_mla_bwd_build_index(const int32_t *indices, int64_t B, int64_t S, int64_t S_kv, int64_t H,
                                              int64_t G, int64_t D_qk, int64_t D_v, int64_t topk, int flags,
                                              uint64_t pass_bytes, void *index, size_t index_bytes,
                                              void *stream) {
  int rc = bwd_check("dsa_sparse_mla_bwd_build_index", B, S, S_kv, H, G, D_qk, D_v, topk, DSA_DTYPE_BF16, flags);
  if (rc) return rc;
  if (B == 0 || S == 0) return DSA_OK;
  const BwdWorkspace L = bwd_layout(B, S, S_kv, H, G, D_qk, topk, flags, pass_bytes);
  DSA_REQUIRE(bwd_passes(L.plan, B) == 1,
              "dsa_sparse_mla_bwd_build_index: this backward runs in several passes (no prebuilt index)");
  DSA_REQUIRE(indices, "dsa_sparse_mla_bwd_build_index: null indices");
  if (!index || index_bytes < L.index_total)
    return set_error(DSA_ERR_WORKSPACE, "dsa_sparse_mla_bwd_build_index: index buffer %zu < required %zu",
                     index_bytes, L.index_total);
  const CsrParams cp = bwd_csr_params(indices, L, static_cast<unsigned char *>(index), 0, B, S, S_kv, G, topk,
                                      wide_shape(D_qk, D_v));
  return launch_csr(cp, B, static_cast<hipStream_t>(stream));
}

extern "C" int dsa_sparse_mla_bwd_indexed(const void *q, const void *kv, const void *o, const void *dO,
                                          const int32_t *indices, const float *lse2, const float *delta, void *dq,
                                          void *dkv, const void *index, size_t index_bytes, void *workspace,
                                          size_t workspace_bytes, int64_t B, int64_t S, int64_t S_kv, int64_t H,
                                          int64_t G, int64_t D_qk, int64_t D_v, int64_t topk, float sm_scale,
                                          int dtype, const float *q_scale, const float *kv_scale, int flags,
                                          uint64_t pass_bytes, void *stream) {
  int rc = bwd_check("dsa_sparse_mla_bwd_indexed", B, S, S_kv, H, G, D_qk, D_v, topk, dtype, flags);
  if (rc) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (B == 0) return DSA_OK;
  DSA_REQUIRE(dkv, "dsa_sparse_mla_bwd_indexed: null dkv");
  DSA_REQUIRE(q && kv && o && dO && indices && lse2 && dq, "dsa_sparse_mla_bwd_indexed: null tensor pointer");
  if (dtype == DSA_DTYPE_E4M3)
    DSA_REQUIRE(q_scale && kv_scale, "dsa_sparse_mla_bwd_indexed: e4m3 input needs q_scale and kv_scale");
  const BwdWorkspace L = bwd_layout(B, S, S_kv, H, G, D_qk, topk, flags, pass_bytes);
  if (S == 0) return bwd_zero_dkv(dkv, B * S_kv * G, D_qk, st);
  DSA_REQUIRE(bwd_passes(L.plan, B) == 1,
              "dsa_sparse_mla_bwd_indexed: this backward runs in several passes (use dsa_sparse_mla_bwd)");
  if (!index || index_bytes < L.index_total)
    return set_error(DSA_ERR_WORKSPACE, "dsa_sparse_mla_bwd_indexed: index buffer %zu < required %zu", index_bytes,
                     L.index_total);
  if (!workspace || workspace_bytes < L.rows_total)
    return set_error(DSA_ERR_WORKSPACE, "dsa_sparse_mla_bwd_indexed: workspace %zu < required %zu", workspace_bytes,
                     L.rows_total);
  return bwd_run(q, kv, o, dO, indices, lse2, delta, dq, dkv, static_cast<unsigned char *>(workspace),
                 const_cast<unsigned char *>(static_cast<const unsigned char *>(index)), true, B, S, S_kv, H, G, D_qk,
                 D_v, topk, sm_scale, dtype, q_scale, kv_scale, flags, L, st);
}
