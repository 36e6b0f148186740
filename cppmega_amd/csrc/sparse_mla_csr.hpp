// Inverse index (kv row -> entries) and the deterministic dKV reduction used
// by the SparseMLA backward.
#pragma once

#include "dsa_common.hpp"

namespace dsa {

// ---------------------------------------------------------------------------
// Inverse index: stable counting sort of entries by kv row
// ---------------------------------------------------------------------------
// Entry e = ((b*S + t)*G + g)*topk + slot; its row (within batch b) is
// r = j*G + g for a valid index j.  Tokens are grouped into chunks of 32
// within one batch (NC chunks per batch), and a chunk's rows into SPL parts
// of RP consecutive rows (one workgroup each, so a chunk's LDS holds RP words
// and short token ranges with long rows still fill the GPU).
//   csr_mask     mask[b][c][r]  = bit tl set when token 32c + tl references
//                                 row r; dup[b][c][part] = some (token, group)
//                                 references one row of the part twice, and
//                                 then the exact counts of the part's rows go
//                                 to base[b][c][r] (a bit cannot count
//                                 repeats); count(c, r) below is that count
//                                 or popcount(mask); such a part writes zero
//                                 masks.  With local ranks, it also writes
//                                 pos_of[e] = the entry's rank among the
//                                 chunk's earlier entries of its row (entry
//                                 order)
//   csr_colscan  base[b][c][r]  = entries of row r in the chunks before c
//                                 (exclusive prefix over chunks), tot = row
//                                 total; dupc[b][c] = any part of chunk c has
//                                 a repeat; rowstart = the row's first CSR
//                                 position: each workgroup reserves one
//                                 contiguous range for its rows with an
//                                 integer atomic and lays its rows out in
//                                 order inside it
//   csr_scatter  pos_of[e]      = rowstart + base + popcount of the earlier
//                                 tokens' bits: entries of a row in ascending
//                                 entry order (only for consumers that read
//                                 every position from pos_of)
// Where a row's range lies depends on the order of the reservations; the
// entries inside it, and so every dKV sum, do not.
// Without repeats a row's entries inside a chunk are ordered by token alone,
// so every entry's position is computed independently: the narrow SparseMLA
// backward's main kernel computes rowstart + base + popcount itself, and for
// a row whose part has a repeat (a zero mask word) rowstart + base + the
// local rank (the order the stable sort defines), so it needs no scatter.

constexpr int kChunkTokens = 32;  // tokens per chunk: one bit each in a 32-bit mask

struct CsrParams {
  const int32_t *idx;
  uint32_t *mask;   // [B][NC][R]
  int32_t *base;    // [B][NC][R]
  int32_t *dup;     // [B][NC][SPL]: the part's rows hold a repeat
  int32_t *dupc;    // [B][NC]: some part of the chunk does
  int32_t *tot;     // [B*R] entries of each row
  int32_t *rowstart;  // [B*R] first CSR position of each row
  int32_t *pos_of;  // [entries]: CSR position of each entry, -1 for a masked slot
  int64_t S, S_kv, G, topk;
  int64_t R;        // rows per batch = S_kv * G
  int NC;           // chunks per batch
  int SPL;          // row parts per chunk
  int64_t RP;       // rows per part (the last part may hold fewer)
  int local_ranks;  // 1: chunks with repeats get local ranks in pos_of and no scatter runs;
                    // 0: the scatter writes every entry's CSR position to pos_of
  int32_t *next;    // [B] CSR positions reserved so far in each batch's region of S * G * topk
                    // positions (zeroed by the mask kernel)
};

// Row parts per chunk: enough that a part's rows fit 64 KiB of LDS, and up to
// 16 when the chunks alone (nchunks over all batches) leave the GPU idle.
static int csr_split(int64_t nchunks, int64_t R) {
  int64_t spl = (R + 16383) / 16384;
  int64_t want = nchunks >= 256 ? 1 : (256 + nchunks - 1) / (nchunks > 0 ? nchunks : 1);
  want = want < 16 ? want : 16;
  spl = spl > want ? spl : want;
  return (int)(spl < R ? spl : (R > 0 ? R : 1));
}

__global__ void fill_i32_kernel(int32_t *p, int64_t n, int32_t v) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

// grid (NC * SPL, B), kMaskThreads threads, dynamic LDS = RP words: workgroup
// (c, part) reads every index of chunk c and records the rows [r_lo, r_hi) of
// its part.
constexpr int kMaskThreads = 1024;
__global__ void __launch_bounds__(kMaskThreads) csr_mask_kernel(const CsrParams p) {
  extern __shared__ uint32_t mk[];
  __shared__ int dflag;
  const int c = blockIdx.x / p.SPL, part = blockIdx.x % p.SPL;
  const int64_t b = blockIdx.y;
  const int tid = threadIdx.x;
  // the column scan that follows on the stream reserves CSR positions from here
  if (blockIdx.x == 0 && tid == 0) p.next[b] = 0;
  // parts past the last row (RP * SPL may exceed R) hold no rows
  const int64_t r_lo = part * p.RP, r_hi = r_lo + p.RP < p.R ? r_lo + p.RP : p.R;
  const uint32_t nr = r_hi > r_lo ? (uint32_t)(r_hi - r_lo) : 0u;
  for (int64_t r = tid; r < nr; r += kMaskThreads) mk[r] = 0u;
  if (tid == 0) dflag = 0;
  __syncthreads();
  const int64_t t0 = (int64_t)c * kChunkTokens;
  const int64_t t1 = t0 + kChunkTokens < p.S ? t0 + kChunkTokens : p.S;
  const int64_t nseg = (t1 - t0) * p.G;
  const int32_t *seg_idx = p.idx + ((b * p.S + t0) * p.G) * p.topk;
  // work item w = (segment w / spt, slots 256 (w % spt) + sl), taken by the
  // thread group ig = w % IG of 256 threads; a round issues U loads per thread
  // (U * IG work items) before any is used
  constexpr int IG = kMaskThreads / 256;
  const int sl = tid & 255, ig = tid >> 8;
  const int spt = (int)((p.topk + 255) / 256);
  const int nw = (int)nseg * spt;
  const int G = (int)p.G;
  int dup = 0;
  // unconditional bounded loads: invalid work items land past the resource
  constexpr int U = 16;
  const auto seg_rs = make_buffer_rsrc(seg_idx, (uint32_t)(nseg * p.topk * 4));
  for (int w0 = 0; w0 < nw; w0 += U * IG) {
    int32_t j[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int w = w0 + u * IG + ig, sg = spt == 1 ? w : w / spt, s = (spt == 1 ? 0 : w % spt) * 256 + sl;
      const bool ok = w < nw && s < p.topk;
      const uint32_t off = ok ? (uint32_t)((sg * p.topk + s) * 4) : 0xffffffffu;
      const int32_t v = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(seg_rs, (int)off, 0, 0);
      j[u] = ok ? v : -1;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int w = w0 + u * IG + ig, sg = spt == 1 ? w : w / spt;
      // rows of other parts (and invalid indices) fail the unsigned range test
      const uint32_t rr = (uint32_t)((int64_t)j[u] * G + (G == 1 ? 0 : sg % G) - r_lo);
      if (j[u] >= 0 && j[u] < p.S_kv && rr < nr) {
        const uint32_t bit = 1u << (G == 1 ? sg : sg / G);
        const uint32_t old = atomicOr(&mk[rr], bit);
        dup |= (old & bit) != 0u;
      }
    }
  }
  if (dup) dflag = 1;  // benign race: every writer stores 1
  __syncthreads();
  // a part with a repeat writes zero masks: a valid entry's own mask word is
  // never zero otherwise, so consumers tell such rows apart by it
  uint32_t *m = p.mask + (b * p.NC + c) * p.R + r_lo;
  for (int64_t r = tid; r < nr; r += kMaskThreads) m[r] = dflag ? 0u : mk[r];
  if (tid == 0) p.dup[(b * p.NC + c) * p.SPL + part] = dflag;
  if (dflag) {  // block-uniform: exact per-row counts of this part's rows
    __syncthreads();
    int32_t *cnt = reinterpret_cast<int32_t *>(mk);
    for (int64_t r = tid; r < nr; r += kMaskThreads) cnt[r] = 0;
    __syncthreads();
    for (int64_t e = tid; e < nseg * p.topk; e += kMaskThreads) {
      const int64_t g = (e / p.topk) % p.G;
      const int32_t j = seg_idx[e];
      const uint32_t rr = (uint32_t)(j * p.G + g - r_lo);
      if (j >= 0 && j < p.S_kv && rr < nr) atomicAdd(&cnt[rr], 1);
    }
    __syncthreads();
    int32_t *dst = p.base + (b * p.NC + c) * p.R + r_lo;
    for (int64_t r = tid; r < nr; r += kMaskThreads) dst[r] = cnt[r];
    if (p.local_ranks) {
      // each entry of this part's rows: its rank among the chunk's earlier
      // entries of the same row, walked in entry order by one thread (a
      // token that repeats a row is an unusual input; this path is serial)
      __syncthreads();
      for (int64_t r = tid; r < nr; r += kMaskThreads) cnt[r] = 0;
      __syncthreads();
      if (tid == 0) {
        int32_t *pos = p.pos_of + ((b * p.S + t0) * p.G) * p.topk;
        for (int64_t e = 0; e < nseg * p.topk; ++e) {
          const int64_t g = (e / p.topk) % p.G;
          const int32_t j = seg_idx[e];
          const uint32_t rr = (uint32_t)(j * p.G + g - r_lo);
          if (j >= 0 && j < p.S_kv && rr < nr) pos[e] = cnt[rr]++;
        }
      }
    }
  }
}

// Entries of row r in chunks c0 .. c0 + T - 1 (those below c_hi) of batch b:
// the mask popcount, or the exact count the mask kernel left in base[] where
// the row's part has a repeat.  The flags and masks load together; base only
// where a flag is set.
template <int T>
__device__ __forceinline__ void tile_counts(const CsrParams &p, int64_t b, int c0, int c_hi, int64_t r, bool rok,
                                            int part, int32_t (&v)[T]) {
  int32_t dv[T];
  uint32_t mv[T];
#pragma unroll
  for (int u = 0; u < T; ++u) {
    const bool ok = c0 + u < c_hi && rok;
    dv[u] = ok ? p.dup[(b * p.NC + c0 + u) * p.SPL + part] : 0;
    mv[u] = ok ? p.mask[(b * p.NC + c0 + u) * p.R + r] : 0u;
  }
#pragma unroll
  for (int u = 0; u < T; ++u) v[u] = dv[u] ? p.base[(b * p.NC + c0 + u) * p.R + r] : (int32_t)__popc(mv[u]);
}

// grid (ceil(R / 32), B), 512 threads: thread t takes row 32 blockIdx.x + t % 32
// and chunk group t / 32 (a contiguous sixteenth of the chunks).  Each thread
// totals its chunks of its row, the groups' totals are combined in LDS, and
// each thread then writes the exclusive prefix over chunks into base[b][c][r]
// (a chunk's exact count, kept in base for chunks with repeats, is read before
// the same thread overwrites it).  A group of at most TILE chunks (every group
// while NC <= 16 * TILE) keeps its counts in registers between the two steps;
// longer ranges re-read them.  Wave 0 reserves one contiguous range of CSR
// positions for the workgroup's rows (an atomic add of their total to the
// batch's counter p.next[b]; batch b's positions start at b * S * G * topk,
// past every entry of the batches before it) and gives each row its start
// inside it, in row order.  Few atomics to one address matter here: each is a
// round trip to the memory side, and they queue.
constexpr int kScanRows = 32, kScanGroups = 16;
__global__ void __launch_bounds__(kScanRows * kScanGroups) csr_colscan_kernel(const CsrParams p) {
  constexpr int TILE = 8;
  __shared__ int32_t gtot[kScanGroups][kScanRows];
  const int tid = threadIdx.x, rl = tid % kScanRows, cg = tid / kScanRows;
  const int64_t b = blockIdx.y;
  const int64_t r = (int64_t)blockIdx.x * kScanRows + rl;
  const bool rok = r < p.R;
  const int part = rok ? (int)(r / p.RP) : 0;
  const int c_lo = (int)((int64_t)p.NC * cg / kScanGroups), c_hi = (int)((int64_t)p.NC * (cg + 1) / kScanGroups);
  if (blockIdx.x == 0) {  // the chunks' combined repeat flags (read by the scatter and the main kernel)
    for (int c = tid; c < p.NC; c += kScanRows * kScanGroups) {
      int any = 0;
      for (int q = 0; q < p.SPL; ++q) any |= p.dup[(b * p.NC + c) * p.SPL + q];
      p.dupc[b * p.NC + c] = any;
    }
  }
  int32_t v[TILE];
  int32_t s = 0;
  for (int c0 = c_lo; c0 < c_hi; c0 += TILE) {
    tile_counts<TILE>(p, b, c0, c_hi, r, rok, part, v);
#pragma unroll
    for (int u = 0; u < TILE; ++u) s += v[u];
  }
  gtot[cg][rl] = s;
  __syncthreads();
  int32_t run = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < kScanGroups; ++i) {
    const int32_t t = gtot[i][rl];
    run += i < cg ? t : 0;
    tot += t;
  }
  // lanes 0..15 of wave 0 hold the rows' totals: their inclusive prefix over
  // the rows, and one reservation for all of them, issued here so that its
  // round trip overlaps the base stores below
  int32_t x = 0, at = 0;
  if (cg == 0) {
    x = tot;
#pragma unroll
    for (int off = 1; off < kScanRows; off <<= 1) {
      const int32_t o = __shfl_up(x, off, kScanRows);
      if (rl >= off) x += o;
    }
    if (rl == kScanRows - 1) at = atomicAdd(p.next + b, x);
  }
  const bool one_tile = c_hi - c_lo <= TILE;  // block-uniform
  for (int c0 = c_lo; c0 < c_hi; c0 += TILE) {
    if (!one_tile) tile_counts<TILE>(p, b, c0, c_hi, r, rok, part, v);
#pragma unroll
    for (int u = 0; u < TILE; ++u) {
      if (c0 + u < c_hi && rok) p.base[(b * p.NC + c0 + u) * p.R + r] = run;
      run += v[u];
    }
  }
  if (cg == 0) {
    at = __shfl(at, kScanRows - 1, kScanRows);
    if (rok) {
      p.tot[b * p.R + r] = tot;
      p.rowstart[b * p.R + r] = (int32_t)(b * p.S * p.G * p.topk) + at + x - tot;
    }
  }
}

// grid (NC * SPL, B), 256 threads; dynamic LDS = RP ints (cursors of the
// serial path).  Chunks without repeats: the SPL workgroups of a chunk split
// its entries, each entry placed independently.  A chunk with a repeat: each
// part's workgroup walks the chunk's entries in order with one thread and
// places those whose rows lie in its part.
__global__ void __launch_bounds__(256) csr_scatter_kernel(const CsrParams p) {
  extern __shared__ int32_t cur[];
  const int c = blockIdx.x / p.SPL, part = blockIdx.x % p.SPL;
  const int64_t b = blockIdx.y;
  const int tid = threadIdx.x;
  const int64_t t0 = (int64_t)c * kChunkTokens;
  const int64_t t1 = t0 + kChunkTokens < p.S ? t0 + kChunkTokens : p.S;
  const int64_t nseg = (t1 - t0) * p.G;
  const int64_t e_first = ((b * p.S + t0) * p.G) * p.topk;
  const uint32_t *m = p.mask + (b * p.NC + c) * p.R;
  const int32_t *bs = p.base + (b * p.NC + c) * p.R;
  const int32_t *rp = p.rowstart + b * p.R;
  if (p.dupc[b * p.NC + c] == 0) {
    // row r of (token t0 + tl, group g): position = base + earlier tokens of the chunk in r;
    // work items as in the mask kernel, this part's share of them, eight in flight
    const int spt = (int)((p.topk + 255) / 256);
    const int nw = (int)nseg * spt;
    const int w_lo = (int)((int64_t)nw * part / p.SPL), w_hi = (int)((int64_t)nw * (part + 1) / p.SPL);
    const int G = (int)p.G;
    for (int w0 = w_lo; w0 < w_hi; w0 += 8) {
      int32_t j[8];
      int64_t e[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int w = w0 + u, sg = spt == 1 ? w : w / spt, s = (spt == 1 ? 0 : w % spt) * 256 + tid;
        e[u] = (w < w_hi && s < p.topk) ? e_first + (int64_t)sg * p.topk + s : -1;
        j[u] = e[u] >= 0 ? p.idx[e[u]] : -1;
      }
      int32_t bv[8];
      uint32_t mv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int w = w0 + u, sg = spt == 1 ? w : w / spt;
        const bool ok = j[u] >= 0 && j[u] < p.S_kv;
        const int64_t r = ok ? (int64_t)j[u] * G + (G == 1 ? 0 : sg % G) : 0;
        bv[u] = ok ? rp[r] + bs[r] : -1;
        mv[u] = ok ? m[r] : 0u;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int w = w0 + u, sg = spt == 1 ? w : w / spt;
        if (e[u] >= 0) {
          const bool ok = j[u] >= 0 && j[u] < p.S_kv;
          const uint32_t below = (1u << (G == 1 ? sg : sg / G)) - 1u;
          p.pos_of[e[u]] = ok ? bv[u] + __popc(mv[u] & below) : -1;
        }
      }
    }
  } else {
    // a row repeats inside a (token, group): one thread per part walks the
    // entries in order (the part holding row 0 also marks the masked slots)
    const int64_t r_lo = part * p.RP, r_hi = r_lo + p.RP < p.R ? r_lo + p.RP : p.R;
    const uint32_t nr = r_hi > r_lo ? (uint32_t)(r_hi - r_lo) : 0u;
    for (int64_t r = tid; r < nr; r += 256) cur[r] = rp[r_lo + r] + bs[r_lo + r];
    __syncthreads();
    if (tid == 0) {
      for (int64_t sg = 0; sg < nseg; ++sg) {
        const int64_t g = sg % p.G;
        for (int64_t s = 0; s < p.topk; ++s) {
          const int64_t e = e_first + sg * p.topk + s;
          const int32_t j = p.idx[e];
          if (j >= 0 && j < p.S_kv) {
            const uint32_t rr = (uint32_t)(j * p.G + g - r_lo);
            if (rr < nr) p.pos_of[e] = cur[rr]++;
          } else if (part == 0) {
            p.pos_of[e] = -1;
          }
        }
      }
    }
  }
}

// One workgroup per kv row.  The main kernel wrote each entry's partial rows
// at its CSR position, so the row's items are the contiguous partial rows
// [rowstart[r] * ntiles, (rowstart[r] + cnt[r]) * ntiles) in CSR order; they are split
// into four contiguous quarters, one per wave.  A partial row is read as
// 16-byte chunks by a group of LPE lanes (rows over 1 KiB: all 64 lanes, CPL
// chunks each), so one load instruction covers EPI = 64 / LPE items and every
// lane keeps about 8 loads in flight.  Lane group g of a wave sums items g,
// g + EPI, ... of its quarter in order (fp32); the groups are combined by a
// fixed xor tree and the four waves as ((w0 + w1) + w2) + w3.  The association
// depends on the item count alone, so the result is bitwise reproducible.
// When one batch's tokens span several passes of the backward, the rows'
// sums are carried in an fp32 accumulator: mode 1 (first pass) stores the
// pass's sum there, mode 2 adds it to the carried sum, mode 3 (last pass)
// writes bf16(carried + pass sum); mode 0 (one pass) writes bf16(pass sum).
template <int D_QK, bool F32P>
__global__ void __launch_bounds__(256)
dkv_reduce_kernel(const int32_t *rowstart, const int32_t *cnt, const unsigned char *partials, const int8_t *partial_exp,
                  uint16_t *dkv, float *carry, int mode, int64_t nrows, int ntiles) {
  constexpr int ROWB = D_QK * (F32P ? 4 : 2);  // bytes per partial row
  constexpr int NCR = ROWB / 16;                // 16-byte chunks per partial row
  constexpr int LPE = NCR <= 8 ? 8 : (NCR <= 16 ? 16 : (NCR <= 32 ? 32 : 64));  // lanes per item
  constexpr int CPL = (NCR + 63) / 64;          // chunks per lane (rows over 1 KiB)
  constexpr int EPI = 64 / LPE;                 // items per load instruction
  constexpr int EPC = F32P ? 4 : 8;             // elements per chunk
  constexpr int U = CPL > 1 ? (8 + CPL - 1) / CPL : 8;  // items in flight per lane
  static_assert(NCR * 16 == ROWB, "partial rows must be whole 16-byte chunks");
  __shared__ float part[4][D_QK];
  const int lane = lane_id(), w = wave_id();
  const int grp = lane / LPE, c = lane % LPE;
  const int64_t r = blockIdx.x;
  if (r >= nrows) return;
  const int64_t base = rowstart[r], n = (int64_t)cnt[r] * ntiles;
  const int64_t k0 = base * ntiles + n * w / 4, k1 = base * ntiles + n * (w + 1) / 4;
  float acc[CPL][EPC];
#pragma unroll
  for (int q = 0; q < CPL; ++q)
#pragma unroll
    for (int x = 0; x < EPC; ++x) acc[q][x] = 0.0f;
  // Batches of EPI * U items: batch j+1 is loaded (unconditional streaming
  // buffer loads through a resource that ends at the wave's last item, so
  // items past it read zeros) while batch j is summed.
  constexpr int STEP = EPI * U;
  const int64_t nk = k1 - k0;
  auto issue = [&](int64_t off, i32x4 (&v)[U][CPL], int (&e)[U]) {
    const int64_t left = nk - off;
    const int64_t cnt = left <= 0 ? 0 : (left < STEP ? left : STEP);
    const int64_t first = left <= 0 ? k0 : k0 + off;
    const auto rs = make_buffer_rsrc(partials + first * ROWB, (uint32_t)(cnt * ROWB));
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int item = EPI * u + grp;
#pragma unroll
      for (int q = 0; q < CPL; ++q) {
        const int cc = c + 64 * q;
        const uint32_t o = cc < NCR ? (uint32_t)(item * ROWB + cc * 16) : 0xffffffffu;
        v[u][q] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)o, 0, 2));
      }
      e[u] = 0;
    }
    if constexpr (!F32P) {
      const auto es = make_buffer_rsrc(partial_exp + first, (uint32_t)cnt);
#pragma unroll
      for (int u = 0; u < U; ++u)
        e[u] = (int)(int8_t)(uint8_t)__builtin_amdgcn_raw_buffer_load_b8(es, EPI * u + grp, 0, 0);
    }
  };
  auto accumulate = [&](const i32x4 (&v)[U][CPL], const int (&e)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float sc = F32P ? 1.0f : exp2i(-e[u]);
#pragma unroll
      for (int q = 0; q < CPL; ++q) {
#pragma unroll
        for (int x = 0; x < EPC; ++x) {
          if constexpr (F32P) {
            acc[q][x] += __int_as_float(v[u][q][x]);
          } else {
            const uint32_t h = ((uint32_t)v[u][q][x >> 1] >> (16 * (x & 1))) & 0xffffu;
            acc[q][x] += f16_bits_to_f32(h) * sc;  // exact: sc is a power of two
          }
        }
      }
    }
  };
  i32x4 va[U][CPL], vb[U][CPL];
  int ea[U], eb[U];
  issue(0, va, ea);
  for (int64_t off = 0; off < nk; off += 2 * STEP) {
    issue(off + STEP, vb, eb);
    accumulate(va, ea);
    if (off + STEP >= nk) break;  // wave-uniform
    issue(off + 2 * STEP, va, ea);
    accumulate(vb, eb);
  }
#pragma unroll
  for (int off = LPE; off < 64; off *= 2) {
#pragma unroll
    for (int q = 0; q < CPL; ++q)
#pragma unroll
      for (int x = 0; x < EPC; ++x) acc[q][x] += __shfl_xor(acc[q][x], off, 64);
  }
  if (grp == 0) {
#pragma unroll
    for (int q = 0; q < CPL; ++q) {
      const int cc = c + 64 * q;
      if (cc < NCR) {
#pragma unroll
        for (int x = 0; x < EPC; ++x) part[w][cc * EPC + x] = acc[q][x];
      }
    }
  }
  __syncthreads();
  uint32_t *out = reinterpret_cast<uint32_t *>(dkv + r * D_QK);
  float *cr = carry + (mode != 0 ? r * D_QK : 0);
  for (int pi = threadIdx.x; pi < D_QK / 2; pi += 256) {
    float x0 = ((part[0][2 * pi] + part[1][2 * pi]) + part[2][2 * pi]) + part[3][2 * pi];
    float x1 = ((part[0][2 * pi + 1] + part[1][2 * pi + 1]) + part[2][2 * pi + 1]) + part[3][2 * pi + 1];
    if (mode >= 2) {  // earlier passes' sum first
      x0 = cr[2 * pi] + x0;
      x1 = cr[2 * pi + 1] + x1;
    }
    if (mode == 0 || mode == 3) {
      out[pi] = pack_bf16x2(x0, x1);
    } else {
      cr[2 * pi] = x0;
      cr[2 * pi + 1] = x1;
    }
  }
}

// Chunking of the inverse index: 32-token chunks (one mask bit per token).
static int csr_chunks(int64_t S) { return (int)((S + kChunkTokens - 1) / kChunkTokens); }

static int launch_csr(const CsrParams &cp, int64_t B, hipStream_t st) {
  const size_t lds = (size_t)cp.RP * 4;
  if (cp.SPL < 1 || cp.RP * cp.SPL < cp.R || lds > 64 * 1024 || (int64_t)cp.NC * cp.SPL >= (1ll << 31))
    return set_error(DSA_ERR_UNSUPPORTED, "sparse_mla_bwd: inverse index split %d x %lld rows of %lld", cp.SPL,
                     (long long)cp.RP, (long long)cp.R);
  const dim3 cgrid((unsigned)(cp.NC * cp.SPL), (unsigned)B);
  const dim3 sgrid((unsigned)((cp.R + kScanRows - 1) / kScanRows), (unsigned)B);
  hipLaunchKernelGGL(csr_mask_kernel, cgrid, dim3(kMaskThreads), lds, st, cp);
  hipLaunchKernelGGL(csr_colscan_kernel, sgrid, dim3(kScanRows * kScanGroups), 0, st, cp);
  if (!cp.local_ranks) hipLaunchKernelGGL(csr_scatter_kernel, cgrid, dim3(256), lds, st, cp);
  return check_launch("sparse_mla_bwd(csr)");
}

}  // namespace dsa
