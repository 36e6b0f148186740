/*
 * dsa_hip.h — C-ABI of the MI355X (gfx950) DeepSeek Sparse Attention hot path.
 *
 * Every entry point is stateless, stream-ordered and returns an int status
 * (DSA_OK == 0, negative on error; dsa_last_error() holds a per-thread
 * message).  All device buffers are caller-owned.  `stream` is a hipStream_t
 * passed as void* so that this header needs no HIP include; NULL means the
 * null stream.  Tensors are dense, row-major and contiguous in the shapes
 * given below.  No entry point allocates device memory; scratch space comes
 * from a caller-provided workspace sized by the matching *_workspace_size().
 *
 * Index convention (all SparseMLA entry points): indices are int32 and any
 * value outside [0, S_kv) — in particular the -1 sentinel — marks a masked
 * slot.  Duplicate indices are legal and counted once per occurrence.
 * LSE is returned in log2 units: lse2 = log2(sum_j exp(sm_scale * q.k_j)).
 * A (token, head) whose slots are all masked yields out = 0, lse2 = -inf and
 * zero gradients.
 */
#ifndef DSA_HIP_H_
#define DSA_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum dsa_status {
  DSA_OK = 0,
  DSA_ERR_INVALID_ARG = -1,  /* shape / pointer / range violation           */
  DSA_ERR_UNSUPPORTED = -2,  /* valid request this build has no kernel for  */
  DSA_ERR_HIP = -3,          /* HIP runtime error (launch, device query)    */
  DSA_ERR_WORKSPACE = -4     /* workspace missing or smaller than required  */
};

enum dsa_dtype {
  DSA_DTYPE_BF16 = 0,        /* bfloat16                                     */
  DSA_DTYPE_E4M3 = 1,        /* OCP float8 e4m3fn (max 448), gfx950 native   */
  DSA_DTYPE_F32 = 2,         /* float32                                      */
  DSA_DTYPE_I32 = 3,         /* int32 (index tensors)                        */
  DSA_DTYPE_I64 = 4,         /* int64 (index tensors)                        */
  DSA_DTYPE_MXFP8 = 5        /* e4m3 with one f32 scale per 32 channels      */
};

/* Per-thread message for the last non-zero status returned on this thread. */
const char *dsa_last_error(void);

/* ABI version (major * 100 + minor). */
int dsa_abi_version(void);

/* Returns DSA_OK when `device` is a gfx950 (MI355X-class) GPU, otherwise
 * DSA_ERR_UNSUPPORTED with the architecture named in dsa_last_error(). */
int dsa_device_check(int device);

/*
 * SparseMLA forward (MQA, packed latent KV).
 * Replaces sparse_mla_fwd_interface / the TileLang `sparse_mla_fwd` kernel
 *   (cppmega/megatron/sparse_mla_ops/tilelang_sparse_mla_fwd.py:128-290,293-391)
 * and, with dtype == DSA_DTYPE_E4M3, sparse_mla_fwd_fp8_interface
 *   (cppmega/megatron/sparse_mla_ops/tilelang_sparse_mla_fwd_fp8.py:178-393,415-559).
 *
 *   q       [B, S, H, D_qk]      bf16 or e4m3 (dtype)
 *   kv      [B, S_kv, G, D_qk]   bf16 or e4m3 (dtype); V = kv[..., :D_v]
 *   indices [B, S, G, topk]      int32
 *   out     [B, S, H, D_v]       bf16
 *   lse2    [B, S, H]            f32 (log2 units)
 *   q_scale [B, S], kv_scale [B, S_kv]  f32 dequant factors (real = fp8 * scale),
 *                                 required for e4m3, ignored (may be NULL) for bf16.
 * dtype DSA_DTYPE_MXFP8 (block-scaled e4m3): q / kv e4m3 with
 *   q_scale [B, S, H, D_qk / 32], kv_scale [B, S_kv, G, D_qk / 32], one f32
 *   factor per 32 consecutive channels; each block's q.k over the codes is
 *   multiplied by q_scale[block] * kv_scale[block] before the blocks are
 *   summed, and V is dequantised per block to bf16.  Replaces the block-scaled
 *   forward sparse_mla_blockscaled_mxfp8_fwd_interface
 *   (cppmega/megatron/sparse_mla_ops/tilelang_sparse_mla_blockscaled_fused.py:248-418,694-793).
 *   (d_qk, d_v) in {(128, 64), (128, 128), (192, 128)}.
 * Head h reads kv group h / (H / G).  sm_scale multiplies the raw q.k dot.
 */
int dsa_sparse_mla_fwd(const void *q, const void *kv, const int32_t *indices,
                       void *out, float *lse2, int64_t B, int64_t S,
                       int64_t S_kv, int64_t H, int64_t G, int64_t D_qk,
                       int64_t D_v, int64_t topk, float sm_scale, int dtype,
                       const float *q_scale, const float *kv_scale,
                       void *stream);

/*
 * The same forward with a workspace.  e4m3 input: the V rows (the first D_v
 * columns of kv) are dequantised to bf16 once per call into the workspace,
 * bit-identical to the per-gather dequantisation of dsa_sparse_mla_fwd, and
 * the kernel gathers those rows instead of converting every gathered row
 * again.  MXFP8 input (d_qk/d_v 128/64, 128/128, 192/128, 576/512): whole kv
 * rows are dequantised to bf16 (code times its block scale) and every q and kv
 * block scale is checked on the device; if each is zero or a power of two in
 * [2^-40, 2^40] (OCP MX scales are powers of two), every dequantised value is
 * exact and the bf16 kernel runs on those rows with q converted at load (the
 * block-scaled scores up to the order of the fp32 sums), otherwise the
 * block-scaled e4m3 kernel runs, with the same result as dsa_sparse_mla_fwd.
 * The choice is made on the device (no host synchronisation; graph capture
 * safe).  dsa_sparse_mla_fwd_workspace_size returns the bytes needed (e4m3:
 * B * S_kv * G * D_v bf16, 0 for the d_qk = 576 kernels, which keep converting
 * V in LDS; MXFP8: B * S_kv * G * D_qk bf16 plus 256; bf16 input: 0, and then
 * `workspace` may be NULL).  Replaces the same reference interfaces as
 * dsa_sparse_mla_fwd.
 */
size_t dsa_sparse_mla_fwd_workspace_size(int64_t B, int64_t S_kv, int64_t G,
                                         int64_t D_qk, int64_t D_v, int dtype);
int dsa_sparse_mla_fwd_ws(const void *q, const void *kv, const int32_t *indices,
                          void *out, float *lse2, int64_t B, int64_t S,
                          int64_t S_kv, int64_t H, int64_t G, int64_t D_qk,
                          int64_t D_v, int64_t topk, float sm_scale, int dtype,
                          const float *q_scale, const float *kv_scale,
                          void *workspace, size_t workspace_bytes, void *stream);

/* dsa_sparse_mla_bwd flags */
enum dsa_bwd_flags {
  /* Keep the per-(token, slot) dKV rows in fp32 instead of bf16 before the
   * deterministic fp32 reduction (2x the workspace traffic, fp32-exact rows). */
  DSA_BWD_FP32_PARTIALS = 1
};

/*
 * pass_bytes (every backward entry point below): the per-pass cap on the
 * backward's partial dKV rows, in bytes; 0 means the default of 4 GiB, and
 * every cap is lowered to at most 4 GiB - 1 MiB (a pass's rows are addressed
 * with 32-bit offsets).  The backward runs in passes over contiguous token ranges sized to this cap, so
 * its workspace stays bounded at any sequence length; a batch split over
 * passes carries its kv rows' sums in fp32 between them.  The workspace /
 * index size queries and the call they size must be given the same value.
 * No counterpart in the reference (whose backward scatters into one fp32 dKV
 * buffer with atomics).
 */

/* Bytes of workspace dsa_sparse_mla_bwd needs for these dimensions, flags and cap. */
size_t dsa_sparse_mla_bwd_workspace_size(int64_t B, int64_t S, int64_t S_kv,
                                         int64_t H, int64_t G, int64_t D_qk,
                                         int64_t D_v, int64_t topk, int flags,
                                         uint64_t pass_bytes);

/*
 * SparseMLA backward.
 * Replaces sparse_mla_bwd = preprocess + bwd + postprocess
 *   (cppmega/megatron/sparse_mla_ops/tilelang_sparse_mla_bwd.py:114-201,204-419,422-531)
 * and, with dtype == DSA_DTYPE_E4M3, sparse_mla_bwd_fp8
 *   (cppmega/megatron/sparse_mla_ops/tilelang_sparse_mla_bwd_fp8.py:191-489,492-630).
 *
 *   q, kv, indices, q_scale, kv_scale as in dsa_sparse_mla_fwd
 *   o   [B, S, H, D_v] bf16 (forward output), dO [B, S, H, D_v] bf16
 *   lse2 [B, S, H] f32 (forward LSE, log2 units)
 *   delta [B, S, H] f32 = sum_d o * dO, or NULL to compute it from o and dO
 *   dq  [B, S, H, D_qk] bf16 (written), dkv [B, S_kv, G, D_qk] bf16 (written)
 * dKV is reduced deterministically: every kv row sums its per-(token, slot)
 * contribution rows (fp16 with a per-row power-of-two scale taken from a bound
 * on the row, max|Q| sum|dS| + max|dO| sum P; fp32 with DSA_BWD_FP32_PARTIALS) in
 * ascending (token, kv group, slot) order in fp32, so repeated calls are
 * bitwise identical.  Gradients are with respect to the dequantised values
 * for e4m3 inputs.  The work runs in passes over token ranges whose partial
 * rows fit the per-pass cap pass_bytes, so the workspace is bounded; results
 * are deterministic for a given cap.
 * Limits: B * S_kv * G < 2^31, B * S * G * topk < 2^31.
 */
int dsa_sparse_mla_bwd(const void *q, const void *kv, const void *o,
                       const void *dO, const int32_t *indices,
                       const float *lse2, const float *delta, void *dq,
                       void *dkv, void *workspace,
                       size_t workspace_bytes, int64_t B, int64_t S,
                       int64_t S_kv, int64_t H, int64_t G, int64_t D_qk,
                       int64_t D_v, int64_t topk, float sm_scale, int dtype,
                       const float *q_scale, const float *kv_scale,
                       int flags, uint64_t pass_bytes, void *stream);

/*
 * The backward's inverse index (kv row -> entries) depends on the indices
 * alone, so a caller may build it ahead of the backward, e.g. on a second
 * stream while the forward runs, and pass it to dsa_sparse_mla_bwd_indexed,
 * which then runs only the main kernel and the dKV reduction (same results,
 * bit for bit, as dsa_sparse_mla_bwd).  Available when the backward runs in one
 * pass: dsa_sparse_mla_bwd_index_size returns 0 otherwise (then use
 * dsa_sparse_mla_bwd).  The index buffer must stay untouched between the two
 * calls and the build must be ordered before the backward (same stream, or an
 * event).  dsa_sparse_mla_bwd_indexed_workspace_size is the partial-row
 * workspace it needs besides the index.  No counterpart in the reference
 * (its backward has no inverse index).
 */
size_t dsa_sparse_mla_bwd_index_size(int64_t B, int64_t S, int64_t S_kv,
                                     int64_t H, int64_t G, int64_t D_qk,
                                     int64_t D_v, int64_t topk, int flags,
                                     uint64_t pass_bytes);
size_t dsa_sparse_mla_bwd_indexed_workspace_size(int64_t B, int64_t S,
                                                 int64_t S_kv, int64_t H,
                                                 int64_t G, int64_t D_qk,
                                                 int64_t D_v, int64_t topk,
                                                 int flags, uint64_t pass_bytes);
int dsa_sparse_mla_bwd_build_index(const int32_t *indices, int64_t B, int64_t S,
                                   int64_t S_kv, int64_t H, int64_t G,
                                   int64_t D_qk, int64_t D_v, int64_t topk,
                                   int flags, uint64_t pass_bytes, void *index,
                                   size_t index_bytes, void *stream);
int dsa_sparse_mla_bwd_indexed(const void *q, const void *kv, const void *o,
                               const void *dO, const int32_t *indices,
                               const float *lse2, const float *delta, void *dq,
                               void *dkv, const void *index, size_t index_bytes,
                               void *workspace, size_t workspace_bytes,
                               int64_t B, int64_t S, int64_t S_kv, int64_t H,
                               int64_t G, int64_t D_qk, int64_t D_v,
                               int64_t topk, float sm_scale, int dtype,
                               const float *q_scale, const float *kv_scale,
                               int flags, uint64_t pass_bytes, void *stream);

/*
 * DSA indexer scores: score[b, t, s] = sum_h w[t, b, h] * act(q[t, b, h, :] . k[s, b, :])
 * with act = ReLU when use_relu != 0, identity otherwise; fp32 accumulate.
 * Replaces Megatron `_compute_index_scores` as patched by
 *   compute_index_scores_fused_bf16 (cppmega/megatron/dsa_indexer_fused_patch.py:71-133).
 *
 *   q [Sq, B, H, D] (dtype), w [Sq, B, H] (w_dtype: bf16 or f32),
 *   k [Sk, B, D] (dtype), scores [B, Sq, Sk] f32.
 *   dtype e4m3: q_scale / k_scale point to one f32 each (per-tensor dequant).
 * causal: 0 = every (t, s) computed;
 *         1 = s > t written as -inf;
 *         2 = only s <= t written (the rest of each row is left untouched).
 */
int dsa_indexer_scores(const void *q, const void *w, const void *k,
                       float *scores, int64_t B, int64_t Sq, int64_t Sk,
                       int64_t H, int64_t D, int dtype, int w_dtype,
                       const float *q_scale, const float *k_scale, int causal,
                       int use_relu, void *stream);

/*
 * DSA indexer scores restricted to per-row windows, with Megatron's additive
 * mask: the scores fused_qk_topk_naive ranks when it is given a mask or varlen
 * windows (call shapes cppmega/megatron/lemyx_dsa_warmup.py:169-176,
 * cppmega/megatron/index_cache_patch.py:148-153):
 *   scores[b, t, s] = sum_h w * act(q . k) + mask[b, t, s]   for starts[b, t] <= s < ends[b, t]
 *                   = -inf                                    elsewhere.
 *   q, w, k, scores, dtype, w_dtype, q_scale, k_scale, use_relu as in
 *   dsa_indexer_scores; starts, ends [B, Sq] int32 (device);
 *   mask [Mb, Sq, Sk] f32 with batch stride mask_bstride elements (0: one mask
 *   shared by every batch) or NULL (no additive term);
 *   row_plain [B, Sq] int32 (device) or NULL: rows flagged nonzero have a mask
 *   of +0.0 on their whole window (dsa_mask_windows' plain flags), which is
 *   then not read (score + 0.0f: the same bits as score + mask).
 * Key tiles outside every window of a group of query tokens are not computed,
 * so a causal window costs the lower-triangle work.  Every element is written.
 */
int dsa_indexer_scores_masked(const void *q, const void *w, const void *k,
                              float *scores, int64_t B, int64_t Sq, int64_t Sk,
                              int64_t H, int64_t D, int dtype, int w_dtype,
                              const float *q_scale, const float *k_scale,
                              const int32_t *starts, const int32_t *ends,
                              const float *mask, int64_t mask_bstride,
                              const int32_t *row_plain, int use_relu,
                              void *stream);

/*
 * Per-row candidate windows of Megatron's additive mask (fused_qk_topk_naive's
 * mask argument, call shapes cppmega/megatron/lemyx_dsa_warmup.py:169-176):
 * for every row t of mask [mask_batches, Sq, Sk] f32 (mask_batches 1 = one
 * mask for every batch, or B), starts / ends [B, Sq] int32 get the first
 * finite column and one past the last ((0, 0) for a row without one), and
 * plain [B, Sq] int32 gets 1 when every entry in between is +0.0 (no finite
 * bias, no -inf / NaN hole), else 0.  One read of the mask, no host
 * synchronisation.  No counterpart in the reference (Megatron adds the mask
 * to the dense scores).
 */
int dsa_mask_windows(const float *mask, int64_t mask_batches, int64_t B,
                     int64_t Sq, int64_t Sk, int32_t *starts, int32_t *ends,
                     int32_t *plain, void *stream);

/*
 * Last step of the masked top-k: idx [rows, topk] int32 (dsa_topk output,
 * ascending, -1 padded) -> out [rows, topk] int64.  On rows not flagged in
 * plain [rows] (NULL: no row is), picks whose score in scores (rows of
 * row_stride f32) is -inf -- mask holes inside a window that held fewer
 * finite columns than topk -- become -1 and the remaining picks stay
 * ascending, padded with -1 at the end.  Megatron returns such picks as
 * indices (torch.topk over index_scores + mask); this build's contract
 * returns only the finite-mask columns.
 */
int dsa_topk_finalize(const float *scores, int64_t row_stride,
                      const int32_t *idx, int64_t rows, int64_t topk,
                      const int32_t *plain, int64_t *out, void *stream);

/*
 * Backward of dsa_indexer_scores (bf16 q / k): given grad_scores G [B, Sq, Sk] f32,
 *   dw[t, b, h]    = sum_s G[b, t, s] * act(L)
 *   dq[t, b, h, :] = w[t, b, h] * sum_s G[b, t, s] * act'(L) * k[s, b, :]
 *   dk[s, b, :]    = sum_{t, h} G[b, t, s] * w[t, b, h] * act'(L) * q[t, b, h, :]
 * with L = q[t, b, h, :] . k[s, b, :] recomputed on MFMA (act = ReLU when
 * use_relu, act' its 0/1 derivative; identity otherwise).  G * act'(L)
 * (times w for dk) is rounded to bf16 for the MFMA; sums are fp32.
 * Replaces the autograd backward of compute_index_scores_fused_bf16's
 * per-head loop (cppmega/megatron/dsa_indexer_fused_patch.py:71-133), the
 * gradient Megatron's indexer loss sends to the indexer's q, weights and k.
 *   q [Sq, B, H, D] bf16, w [Sq, B, H] (w_dtype), k [Sk, B, D] bf16;
 *   dq [Sq, B, H, D] bf16, dw [Sq, B, H] (w_dtype), dk [Sk, B, D] bf16 (written).
 * causal: 0 = every (t, s); 1 = only s <= t (G above the diagonal ignored).
 * starts / ends [B, Sq] int32 (device; both or neither): row windows, the
 * backward of dsa_indexer_scores_masked -- G outside [start, end) is ignored
 * (the masked forward writes -inf there whatever the raw score) and key tiles
 * outside every window of a group of rows are not computed, so a causal
 * window costs the lower-triangle work.
 * Deterministic (fixed summation orders, no atomics).  workspace >=
 * dsa_indexer_scores_backward_workspace_size() bytes (fp32 dk partials per
 * token chunk, and the windows' chunk flags).  Limits: Sq * Sk < 2^30,
 * H in {16, 32, 64}, D in {64, 128}.
 */
size_t dsa_indexer_scores_backward_workspace_size(int64_t B, int64_t Sq,
                                                  int64_t Sk, int64_t H,
                                                  int64_t D);
int dsa_indexer_scores_backward(const float *grad_scores, const void *q,
                                const void *w, const void *k, void *dq,
                                void *dw, void *dk, int64_t B, int64_t Sq,
                                int64_t Sk, int64_t H, int64_t D, int dtype,
                                int w_dtype, int causal, int use_relu,
                                const int32_t *starts, const int32_t *ends,
                                void *workspace, size_t workspace_bytes,
                                void *stream);

/*
 * Per-row top-k selection over fp32 scores.
 * Replaces the top-k of Megatron `fused_qk_topk_naive`
 *   (restated in scripts/modal_dsa_indexer_bench.py:188-194) with a stricter,
 * deterministic contract: the candidates of row r are columns [start, end);
 * the min(topk, end - start) largest are selected, ties break to the lower
 * column, NaN ranks as +inf, -0.0 equals +0.0; selected columns are written
 * in ascending order and the row is padded with -1.
 *
 *   scores  rows of `row_len` f32, row r at scores + r * row_stride
 *   out_idx [rows, topk] int32
 *   starts/ends: per-row int32 window; when NULL the window is
 *     causal != 0 : [0, min(row_len, (r % seq_q) + 1 + causal_offset))
 *     causal == 0 : [0, row_len)
 */
int dsa_topk(const float *scores, int64_t rows, int64_t row_len,
             int64_t row_stride, int64_t seq_q, int causal,
             int64_t causal_offset, const int32_t *starts,
             const int32_t *ends, int64_t topk, int32_t *out_idx,
             void *stream);

/*
 * dsa_topk for rows of any length up to 64 x 32768 columns (with
 * ceil(row_len / 32768) * topk <= 32768), the reach of the reference's
 * tl_topk, which streams rows of any seq_len (topk_selector.py:30-186).
 * dsa_topk takes rows of up to 32768 columns in one pass; longer rows run as
 * segments of at most 32768 columns, each segment's top-k, then one top-k
 * over the segments' picks (which hold the row's top-k), so the result
 * follows the same contract bit for bit.  Those passes use a workspace of
 * dsa_topk_workspace_size(rows, row_len, topk) bytes (0 for rows that fit
 * one pass, where workspace may be NULL).
 */
size_t dsa_topk_workspace_size(int64_t rows, int64_t row_len, int64_t topk);
int dsa_topk_ws(const float *scores, int64_t rows, int64_t row_len,
                int64_t row_stride, int64_t seq_q, int causal,
                int64_t causal_offset, const int32_t *starts,
                const int32_t *ends, int64_t topk, int32_t *out_idx,
                void *workspace, size_t workspace_bytes, void *stream);

/*
 * Streaming indexer + top-k: the top-k of the indexer scores of every query
 * row without the [B, Sq, Sk] score matrix, the target the reference states
 * for its indexer ("emit only [b, sq, topk] indices and optional top-k
 * scores", docs/status/cppmega_architecture_status.md:340-362).  Query rows
 * go through the workspace in chunks of as many rows as it holds
 * (workspace_bytes / (B * Sk * 4); causal chunks hold only keys up to their
 * last query row): per chunk the indexer kernel writes the chunk's scores
 * (causal: only s <= t) and the top-k kernel selects from them, so the
 * indices equal dsa_topk's on the same fp32 scores, bit for bit.  Rows over
 * 32768 keys also keep the top-k's segment passes in the workspace
 * (dsa_topk_workspace_size of the chunk's B * rows rows).
 *   q, w, k, dtype, w_dtype, q_scale, k_scale, use_relu as in dsa_indexer_scores;
 *   out_idx [B, Sq, topk] int32 (ascending, -1 padded; candidates s <= t when
 *   causal, every key otherwise); out_scores [B, Sq, topk] f32 (the selected
 *   scores, -inf for padding) or NULL.
 * workspace: >= dsa_indexer_topk_streaming_workspace_size(B, Sq, Sk, rows)
 * bytes for chunks of `rows` query rows (at least one row); for Sk > 32768
 * add 256 + dsa_topk_workspace_size(B * rows, Sk, topk).
 */
size_t dsa_indexer_topk_streaming_workspace_size(int64_t B, int64_t Sq, int64_t Sk,
                                                 int64_t chunk_rows);
int dsa_indexer_topk_streaming(const void *q, const void *w, const void *k,
                               int32_t *out_idx, float *out_scores, int64_t B,
                               int64_t Sq, int64_t Sk, int64_t H, int64_t D,
                               int dtype, int w_dtype, const float *q_scale,
                               const float *k_scale, int64_t topk, int causal,
                               int use_relu, void *workspace,
                               size_t workspace_bytes, void *stream);

/*
 * Fused indexer + top-k: the same indices (and selected scores) as
 * dsa_indexer_topk_streaming and as dsa_topk over dsa_indexer_scores, bit for
 * bit, with no score matrix and no workspace at all: each query row keeps a
 * bounded candidate list in on-chip memory while its keys are scored, and an
 * exact selection under the top-k contract (value descending, NaN as +inf,
 * -0 equal to +0, ties to the lower column) keeps its running top-k.  This is
 * the reference's stated target for its indexer ("fold top-k selection into
 * the per-head/tiled accumulation so the runtime emits only [b,sq,topk]",
 * docs/status/cppmega_architecture_status.md:358-359); the reference itself
 * materialises the scores (dsa_indexer_fused_patch.py:71-133 + topk).
 * Arguments as in dsa_indexer_topk_streaming (no workspace).  topk is at most
 * dsa_indexer_topk_fused_max_topk(H, D) (0: no kernel for that shape);
 * larger requests return DSA_ERR_UNSUPPORTED.
 */
int64_t dsa_indexer_topk_fused_max_topk(int64_t H, int64_t D);
int dsa_indexer_topk_fused(const void *q, const void *w, const void *k,
                           int32_t *out_idx, float *out_scores, int64_t B,
                           int64_t Sq, int64_t Sk, int64_t H, int64_t D,
                           int dtype, int w_dtype, const float *q_scale,
                           const float *k_scale, int64_t topk, int causal,
                           int use_relu, void *stream);

/*
 * Tensorwise (current-scaling) quantisation to OCP e4m3:
 *   amax = max|x|, scale = 448 / amax (1 when amax == 0),
 *   out = e4m3(RNE(x * scale)) saturated to +-448, scale_inv = 1 / scale.
 * Replaces the TE Float8CurrentScalingQuantizer call in per_token_cast_to_fp8
 *   (cppmega/megatron/sparse_mla_ops/tilelang_sparse_mla_fwd_fp8.py:74-99,396-412).
 *   x [n] (in_dtype bf16 or f32), out_fp8 [n] e4m3, scale_inv [1] f32,
 *   workspace >= dsa_fp8_quantize_workspace_size() bytes.
 */
size_t dsa_fp8_quantize_workspace_size(void);
int dsa_fp8_tensorwise_quantize(const void *x, int64_t n, int in_dtype,
                                uint8_t *out_fp8, float *scale_inv,
                                void *workspace, size_t workspace_bytes,
                                void *stream);

/*
 * dsa_fp8_tensorwise_quantize without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  No counterpart in the reference.
 * Same arguments, result and error behaviour as dsa_fp8_tensorwise_quantize;
 * the scratch comes from a static device array of
 * dsa_fp8_quantize_workspace_size() bytes (4352) that each GPU holds until
 * the process ends, so every n is accepted.  The call allocates nothing.
 * Calls that overlap on one GPU (different streams) share that scratch and
 * race; serialise them on one stream.
 */
int dsa_fp8_tensorwise_quantize_noalloc(const void *x, int64_t n, int in_dtype,
                                        uint8_t *out_fp8, float *scale_inv,
                                        void *stream);

/*
 * e4m3 dequantisation: out[i] = value(x_fp8[i]) * scale_inv[0] (bf16 RNE or f32).
 * Replaces Float8Tensor.dequantize() (the TE tensors whose _data / _scale_inv
 *   cppmega's SparseMLA_FP8 unpacks, cppmega/megatron/sparse_mla_ops/sparse_mla.py:310-353);
 *   decodes with the same hardware conversion the e4m3 SparseMLA kernels use.
 *   x_fp8 [n] OCP e4m3fn, scale_inv [1] f32 (device), out [n] (out_dtype bf16 or f32).
 */
int dsa_fp8_dequantize(const uint8_t *x_fp8, int64_t n, const float *scale_inv,
                       void *out, int out_dtype, void *stream);

/*
 * Block-scaled e4m3 dequantisation: out[i] = value(x_fp8[i]) * scales[i / block]
 * (block a positive multiple of 4; 32 for MXFP8 rows).  Replaces
 *   _dequantize_mxfp8_tensor (cppmega/megatron/sparse_mla_ops/tilelang_sparse_mla_blockscaled_fused.py:961-969),
 *   which the reference's block-scaled backward runs before a bf16 backward.
 *   x_fp8 [n] e4m3, scales [n / block] f32, out [n] bf16 (RNE) or f32.
 */
int dsa_fp8_dequantize_blockwise(const uint8_t *x_fp8, int64_t n, int64_t block,
                                 const float *scales, void *out, int out_dtype,
                                 void *stream);

/*
 * DSA indexer KL loss (the indexer's training signal):
 *   a_h[t, s] = softmax_scale * query[t, b, h] . key[s, b, h / (H / G)]
 *   P[t, s]   = mean_h softmax over s <= t of a_h[t, :]      (sparse: and s in
 *               the row's top-k set)
 *   Q[t, s]   = softmax over all s in [0, Sk) of index_scores[b, t, :] (sparse:
 *               over the top-k set)
 *   row_loss[b, t] = sum_s P (ln(P + 1e-10) - ln(Q + 1e-10)),
 *   loss = loss_coeff * mean over (b, t) of row_loss.
 * Replaces compute_dsa_indexer_loss_splitk
 *   (cppmega/megatron/dsa_splitk_indexer_loss.py:328-468), the Triton split-K
 *   form of Megatron's compute_dsa_indexer_loss
 *   (clone at tests/test_dsa_splitk_indexer_loss.py:29-83).
 *
 *   index_scores [B, Sq, Sk] f32
 *   topk_indices [B, Sq, topk] int32 / int64 (topk_dtype), used when sparse != 0;
 *                values outside [0, Sk) are ignored, duplicates count once
 *   query [Sq, B, H, D] bf16, key [Sk, B, G, D] bf16 (G divides H; G = H is
 *                the reference's per-head key), D in {64, 128, 192, 256}
 *   loss [1] f32 (written), row_loss [B, Sq] f32 (written; may be NULL)
 * A row with no admissible attention column (sparse: no top-k column <= t) or
 * whose index softmax is undefined (all -inf, any NaN or +inf) gets a NaN row
 * loss, as the reference's softmax does, and the mean is then NaN.
 * Deterministic: fixed summation orders, no global atomics.
 * Limits: softmax_scale > 0, B * Sq * Sk < 2^29; sparse mode Sk <= 32768.
 */
size_t dsa_indexer_kl_loss_workspace_size(int64_t B, int64_t Sq, int64_t Sk,
                                          int64_t H, int64_t D, int sparse);
int dsa_indexer_kl_loss(const float *index_scores, const void *topk_indices,
                        int topk_dtype, int64_t topk, const void *query,
                        const void *key, float *loss, float *row_loss,
                        int64_t B, int64_t Sq, int64_t Sk, int64_t H,
                        int64_t G, int64_t D, float softmax_scale,
                        float loss_coeff, int sparse, void *workspace,
                        size_t workspace_bytes, void *stream);

/*
 * Gradient of dsa_indexer_kl_loss's scalar with respect to index_scores:
 *   grad_index_scores[b, t, s] = grad_loss[0] * loss_coeff / (B * Sq)
 *                                * (Q_s * R - P_s * Q_s / (Q_s + 1e-10)),
 *   R = sum_j P_j * Q_j / (Q_j + 1e-10)
 * (P the detached head-mean attention target, Q the index softmax; 0 where
 * Q_s = 0, NaN over a row whose loss is NaN).  Replaces the autograd path
 * through Megatron's compute_dsa_indexer_loss that the reference's split-K
 * loss (cppmega/megatron/dsa_splitk_indexer_loss.py:328-468) does not provide,
 * and the gradient the lemyx fused indexer loss returns to the index scores
 * (cppmega/megatron/lemyx_dsa_warmup.py:78-178).  grad_loss is a device
 * pointer (no host synchronisation).  Same arguments, limits and workspace
 * size as dsa_indexer_kl_loss; grad_index_scores [B, Sq, Sk] f32 must not
 * alias index_scores.
 */
int dsa_indexer_kl_loss_backward(const float *index_scores,
                                 const void *topk_indices, int topk_dtype,
                                 int64_t topk, const void *query,
                                 const void *key, const float *grad_loss,
                                 float *grad_index_scores, int64_t B,
                                 int64_t Sq, int64_t Sk, int64_t H, int64_t G,
                                 int64_t D, float softmax_scale,
                                 float loss_coeff, int sparse, void *workspace,
                                 size_t workspace_bytes, void *stream);

/*
 * Top-k index mask of the sparse indexer loss.
 * Replaces Megatron's _scatter_topk_into_index_mask in the CUDA-graph-safe form
 *   cppmega patches in (cppmega/megatron/upstream_patches/apply_dsa_cg_patches.py:267-291;
 *   eager oracle upstream_prs/examples/01_dsa_cuda_graph_safety/reproducer.py:124-138).
 *
 *   topk_indices [B, rows, topk] int32 / int64 (topk_dtype): the top-k columns
 *                of mask rows [row0, row0 + rows); values outside [0, Sk) (the
 *                -1 sentinel) are skipped, duplicates are harmless
 *   mask [B, Sq, Sk] f32
 * fill_rows == 0: mask[b, row0 + r, s] = value for every listed s; nothing
 *                 else is written (the reference's in-place scatter).
 * fill_rows != 0: every element of rows [row0, row0 + rows) is written:
 *                 value on listed columns, fill elsewhere (Sk <= 262144).
 * One launch, no host synchronisation, idempotent: safe under graph capture.
 */
int dsa_topk_index_mask(const void *topk_indices, int topk_dtype, int64_t topk,
                        float *mask, int64_t B, int64_t Sq, int64_t Sk,
                        int64_t row0, int64_t rows, float value, float fill,
                        int fill_rows, void *stream);

/*
 * Stage timing (measurement aid; no counterpart in the reference, which
 * times whole calls with CUDA events in its benchmark scripts).  With
 * dsa_stage_timing(1) on a thread, every later dsa_sparse_mla_bwd call on
 * that thread records HIP events on its stream at its stage boundaries:
 * stage 0 = inverse index (CSR), 1 = main kernel (dQ + dKV partial rows),
 * 2 = dKV reduction.  Nothing synchronises until dsa_stage_times(back, ...)
 * reads the record of the call `back` calls ago (0 = most recent, up to 255)
 * and writes the elapsed milliseconds of its stages; it returns the number
 * of stages written (or a negative status).
 */
int dsa_stage_timing(int enable);
int dsa_stage_times(int back, float *ms, int max_stages);

#ifdef __cplusplus
}
#endif

#endif /* DSA_HIP_H_ */
