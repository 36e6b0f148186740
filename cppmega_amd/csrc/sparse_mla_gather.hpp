// Row gather shared by the SparseMLA forward and backward kernels.
//
// A wave gathers the 32 kv rows selected by one block of 32 top-k slots.  The
// work is split into units of (4 consecutive slots x one 16-byte chunk); lane
// u handles chunk u % NCH of slots 4*(u / NCH) .. +3, so 16 consecutive lanes
// read one 256-byte row contiguously.  gather_issue() only issues the loads
// (bounded buffer loads: masked slots read zeros, and the loads carry no
// branches); the stores to LDS happen later, so a block's loads overlap the
// previous block's compute.  Every tile is stored row-major: MFMA operands
// that need a transposed view read it with ds_read_b64_tr_b16 (tr_operand).
#pragma once

#include <type_traits>

#include "dsa_common.hpp"

namespace dsa {

// MX: e4m3 rows with one f32 scale per 32 consecutive channels (MXFP8 block
// scaling) instead of one scale per row.
template <int D_QK, int D_V, bool FP8, bool MX = false>
struct GatherCfg {
  static constexpr int kDqk = D_QK;
  static constexpr int kDv = D_V;
  static constexpr bool kFp8 = FP8;
  static constexpr bool kMx = MX;
  static constexpr int NBLK = D_QK / 32;           // MX scale blocks per row
  static constexpr int ELT = FP8 ? 1 : 2;          // bytes per element in HBM
  static constexpr int ROWB = D_QK * ELT;          // bytes per kv row
  static constexpr int CH = 16 / ELT;              // elements per 16-byte chunk
  static constexpr int NCH = D_QK / CH;            // chunks per row
  static constexpr int NCH_V = D_V / CH;           // chunks of the V prefix
  static constexpr int UNITS = 8 * NCH;            // (4 rows x 1 chunk) units per block
  static constexpr int UPL = (UNITS + 63) / 64;    // units per lane
  static constexpr int KL_STRIDE = ROWB + 32;      // LDS row stride: a 32-byte pad puts the 4 rows of a
                                                   // transposed read in distinct banks
  static_assert(NCH * CH == D_QK && NCH_V * CH == D_V, "head dims must be whole 16-byte chunks");
  static_assert(!MX || (FP8 && D_QK % 32 == 0), "MX block scales need e4m3 rows of whole 32-channel blocks");
  struct Regs {
    i32x4 v[UPL][4];
    float sc[UPL][4];
  };
};

// Raw index of slot blk*32 + l32 through a buffer resource covering the row's
// topk indices (0 past the end): an unconditional load, so the wait for it is
// counted exactly and never has to drain other outstanding memory operations
// (stores in particular).  slot_index() applies the mask when it is used.
__device__ __forceinline__ int load_slot_raw(__amdgpu_buffer_rsrc_t idx_rs, int blk, int l32) {
  return (int)__builtin_amdgcn_raw_buffer_load_b32(idx_rs, (blk * 32 + l32) * 4, 0, 0);
}
// topk and s_kv are below 2^31 (checked on the host), so unsigned 32-bit
// compares cover both bounds of each test.
__device__ __forceinline__ int slot_index(int raw, int blk, int l32, int64_t topk, int64_t s_kv) {
  const uint32_t sl = (uint32_t)blk * 32u + (uint32_t)l32;
  return (sl < (uint32_t)topk && (uint32_t)raw < (uint32_t)s_kv) ? raw : -1;
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t slot_rsrc(const int32_t *row, int64_t topk) {
  const int64_t nb = topk * 4;
  return make_buffer_rsrc(row, nb < 0x7fffffff ? (uint32_t)nb : 0x7fffffffu);
}

// Number of 32-slot blocks of this row up to its last valid slot (an index in
// [0, s_kv)), 0 when it has none: every later block is wholly masked and
// contributes nothing, so the block loops stop there.  One pass of unconditional
// bounded loads over the row's indices, then a wave maximum (the same value in
// every wave of a workgroup).
__device__ __forceinline__ int valid_blocks(__amdgpu_buffer_rsrc_t idx_rs, int64_t topk, int64_t s_kv) {
  const int lane = lane_id();
  int last = -1;
  for (int64_t s0 = 0; s0 < topk; s0 += 256) {
    int raw[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) raw[u] = (int)__builtin_amdgcn_raw_buffer_load_b32(idx_rs, (int)((s0 + 64 * u + lane) * 4), 0, 0);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t s = s0 + 64 * u + lane;
      last = (s < topk && raw[u] >= 0 && raw[u] < s_kv && (int)s > last) ? (int)s : last;
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const int o = __shfl_xor(last, off, 64);
    last = o > last ? o : last;
  }
  return __builtin_amdgcn_readfirstlane((last + 32) / 32);
}

// Index of slot blk*32 + l32 of this row, or -1 when masked / past topk.
__device__ __forceinline__ int load_slot_index(const int32_t *idx_row, int blk, int l32, int64_t topk,
                                               int64_t s_kv) {
  const int64_t sl = (int64_t)blk * 32 + l32;
  if (sl >= topk) return -1;
  const int v = idx_row[sl];
  return (v >= 0 && v < s_kv) ? v : -1;
}

// Byte offset at or past the end of every kv resource (the host keeps a
// batch's kv rows within it): a masked slot's loads start here and read
// zeros, and adding a chunk offset (below 64 KiB) cannot wrap.
constexpr uint32_t kMaskedOff = 0xffff0000u;

// Rows are read through buffer resources: kv_rs covers the kv rows of this
// (batch, kv group) (row r at byte r * row_pitch, row_pitch = G * ROWB), sc_rs
// their e4m3 scales (row r at byte r * sc_pitch; MX: the scale of 16-byte
// chunk c is block c / 2 of the row, 4 bytes apart).  A masked slot reads at an offset past the resource, which
// the hardware answers with zeros, so masked rows (and their scales) arrive as
// zeros without selects, and every load is issued on every path.  Each lane
// forms its own slot's row offset once (one multiply per block); a load takes
// its row's offset from the owner lane and adds its chunk's.
template <class Gat>
__device__ __forceinline__ void gather_issue(typename Gat::Regs &rg, __amdgpu_buffer_rsrc_t kv_rs,
                                             __amdgpu_buffer_rsrc_t sc_rs, int my_idx, uint32_t row_pitch,
                                             uint32_t sc_pitch = 4u) {
  const int lane = lane_id();
  const uint32_t my_off = my_idx >= 0 ? (uint32_t)my_idx * row_pitch : kMaskedOff;
  uint32_t my_soff = kMaskedOff;
  if constexpr (Gat::kFp8) my_soff = my_idx >= 0 ? (uint32_t)my_idx * sc_pitch : kMaskedOff;
#pragma unroll
  for (int uu = 0; uu < Gat::UPL; ++uu) {
    const int u = lane + 64 * uu;
    const int c = u % Gat::NCH;
    const int quad = (u / Gat::NCH) & 7;
    const bool in = u < Gat::UNITS;  // false only on the lanes past a ragged last unit
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t ro = (uint32_t)__shfl((int)my_off, quad * 4 + r, 64);
      const uint32_t off = in ? ro + (uint32_t)c * 16u : kMaskedOff;
      rg.v[uu][r] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(kv_rs, (int)off, 0, 0));
      if constexpr (Gat::kFp8) {
        const uint32_t so = (uint32_t)__shfl((int)my_soff, quad * 4 + r, 64) +
                            (Gat::kMx ? (uint32_t)(c / 2) * 4u : 0u);
        rg.sc[uu][r] = buffer_load_f32(sc_rs, in ? (int)so : (int)kMaskedOff, 0);
      }
    }
  }
}

// The same issue with the slots' row offsets exchanged through LDS instead of
// ds_bpermute (bf16 rows, no scales): gather_put_offsets writes each slot's
// row offset (lane l32 -> offs[l32], 32 ints of the wave's LDS), and after a
// wave sync gather_issue_offs reads the four offsets of a lane's rows with
// one broadcast 16-byte read per unit.  LDS time per block is about a third
// of eight bpermutes'.
__device__ __forceinline__ void gather_put_offsets(int *offs, int my_idx, uint32_t row_pitch) {
  const uint32_t my_off = my_idx >= 0 ? (uint32_t)my_idx * row_pitch : kMaskedOff;
  const int lane = lane_id();
  if (lane < 32) offs[lane] = (int)my_off;
}
template <class Gat>
__device__ __forceinline__ void gather_issue_offs(typename Gat::Regs &rg, __amdgpu_buffer_rsrc_t kv_rs,
                                                  const int *offs) {
  static_assert(!Gat::kFp8, "rows with scales take gather_issue");
  const int lane = lane_id();
#pragma unroll
  for (int uu = 0; uu < Gat::UPL; ++uu) {
    const int u = lane + 64 * uu;
    const int c = u % Gat::NCH;
    const int quad = (u / Gat::NCH) & 7;
    const bool in = u < Gat::UNITS;
    const i32x4 o4 = *reinterpret_cast<const i32x4 *>(offs + quad * 4);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t off = in ? (uint32_t)o4[r] + (uint32_t)c * 16u : kMaskedOff;
      rg.v[uu][r] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(kv_rs, (int)off, 0, 0));
    }
  }
}

// K rows, row-major (raw bf16 / e4m3 bytes): Kl[slot][chunk]; masked slots
// arrive as zeros from gather_issue.  SWZ: 16-byte chunk c of row R sits at
// chunk c ^ ((R >> 3) & 1), so rows R and R + 8 (which the 32-byte row pad
// puts on the same banks) hold a column on different 16-byte halves and the
// MFMA operand reads (lane = row) are free of bank conflicts; the row count
// of chunks must be even.
template <class Gat, bool SWZ = false>
__device__ __forceinline__ void gather_store_k(const typename Gat::Regs &rg, unsigned char *Kl) {
  static_assert(!SWZ || Gat::NCH % 2 == 0, "the swizzle pairs chunks");
  const int lane = lane_id();
#pragma unroll
  for (int uu = 0; uu < Gat::UPL; ++uu) {
    const int u = lane + 64 * uu;
    if (u >= Gat::UNITS) break;
    const int c = u % Gat::NCH, quad = u / Gat::NCH;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = quad * 4 + r;
      const int pc = SWZ ? (c ^ ((row >> 3) & 1)) : c;
      *reinterpret_cast<i32x4 *>(Kl + row * Gat::KL_STRIDE + pc * 16) = rg.v[uu][r];
    }
  }
}

// e4m3 only: rows dequantised to bf16 (value * kv_scale, RNE), row-major,
// for the chunks c < NCH_D (the V prefix or the whole row).
template <class Gat, int NCH_D>
__device__ __forceinline__ void gather_store_dequant(const typename Gat::Regs &rg, unsigned char *Kd, int stride) {
  static_assert(Gat::kFp8, "dequantised rows exist for e4m3 input only");
  const int lane = lane_id();
#pragma unroll
  for (int uu = 0; uu < Gat::UPL; ++uu) {
    const int u = lane + 64 * uu;
    if (u >= Gat::UNITS) break;
    const int c = u % Gat::NCH, quad = u / Gat::NCH;
    if (c < NCH_D) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float s = rg.sc[uu][r];  // 0 for a masked slot
        uint32_t w[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const f32x2 v2 = e4m3x2_to_f32((uint32_t)rg.v[uu][r][e >> 1], (e & 1) != 0);
          w[e] = pack_bf16x2(v2[0] * s, v2[1] * s);
        }
        unsigned char *dst = Kd + (quad * 4 + r) * stride + c * 32;
        *reinterpret_cast<i32x4 *>(dst) = i32x4{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
        *reinterpret_cast<i32x4 *>(dst + 16) = i32x4{(int)w[4], (int)w[5], (int)w[6], (int)w[7]};
      }
    }
  }
}

// e4m3 only: per-slot kv dequant scale (0 for masked slots); MX: per (block,
// slot), block-major (Ksc[block * 32 + slot]).
template <class Gat>
__device__ __forceinline__ void gather_store_scale(const typename Gat::Regs &rg, float *Ksc) {
  const int lane = lane_id();
#pragma unroll
  for (int uu = 0; uu < Gat::UPL; ++uu) {
    const int u = lane + 64 * uu;
    if (u >= Gat::UNITS) break;
    const int c = u % Gat::NCH, quad = u / Gat::NCH;
    if (Gat::kMx ? (c % 2 == 0) : (c == 0)) {
      float *dst = Gat::kMx ? Ksc + (c / 2) * 32 : Ksc;
#pragma unroll
      for (int r = 0; r < 4; ++r) dst[quad * 4 + r] = rg.sc[uu][r];
    }
  }
}

}  // namespace dsa
