// Kernel parameter blocks of the SparseMLA forward and backward, shared by
// the narrow-head kernels and the wide-head (d_qk = 576) kernels.
#pragma once

#include <stdint.h>

namespace dsa {

// Partial rows past the entries that masked slots of the backward write (their
// stores are unconditional); workgroup `item` uses row entries + item % kTrashRows,
// so the discarded stores spread over many rows (and memory channels) instead
// of all landing on one.
constexpr int kTrashRows = 64;

struct FwdParams {
  const unsigned char *q;
  const unsigned char *kv;
  const int32_t *idx;
  uint16_t *out;
  float *lse;
  const float *q_scale;
  const float *kv_scale;
  const uint16_t *v16;  // e4m3 / MX: V rows dequantised once to bf16 (v16_ld elements per row), or null
  int v16_ld;           // elements per row of v16: D_v, or D_qk when it holds whole kv rows
  // when set, the kernel computes only if *gate == gate_run (two kernels of one
  // call, one of which does the work, chosen on the device without a host sync)
  const int *gate;
  int gate_run;
  int64_t B, S, S_kv, H, G, topk;
  int hpg;     // heads per kv group
  int ntiles;  // ceil(hpg / 32)
  float sl2;   // sm_scale * log2(e)
};

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
  const int32_t *pos_of;  // narrow kernel: an entry's rank among its chunk's earlier entries of its
                          // row (chunks with repeats only); wide kernel: every entry's CSR
                          // position (-1: masked slot)
  const uint32_t *mask;   // inverse index: [B][NC][R] token bits per (chunk, kv row)
  const int32_t *base;    // [B][NC][R] first CSR position of a (chunk, kv row)
  const int32_t *dup;     // [B][NC] chunk has a token repeating a row
  const int32_t *rowstart;  // [B*R] first CSR position of each kv row
  int64_t R;              // kv rows per batch (S_kv * G)
  int NC;                 // token chunks per batch
  unsigned char *partials;
  int8_t *partial_exp;  // fp16 rows: power-of-two scale exponent per (position, tile)
  int64_t B, S, S_kv, H, G, topk;
  int hpg, ntiles;
  float sl2;    // sm_scale * log2(e)
  float scale;  // sm_scale
};

}  // namespace dsa
