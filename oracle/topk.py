"""CPU restatement of the deterministic per-row top-k.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

The reference top-k is Megatron's `fused_qk_topk_naive`, inlined as
`index_scores.topk(min(topk, seqlen), dim=-1)[1]`
(scripts/modal_dsa_indexer_bench.py:188-194), with masked picks turned into
-1 (cppmega/megatron/upstream_patches/apply_dsa_cg_patches.py:267-291).
torch.topk leaves the order of ties unspecified; the contract restated here
fixes it: candidates of row r are the columns [start, end), the
min(topk, end - start) largest scores are selected, equal scores prefer the
lower column, NaN ranks as +inf, -0.0 equals +0.0, the chosen columns are
returned in ascending order and the row is padded with -1.
"""
from __future__ import annotations

import numpy as np


def causal_windows(rows, seq_q, row_len, offset=0):
    """Per-row [start, end) of the causal window: end = min(row_len, r % seq_q + 1 + offset)."""
    r = np.arange(rows)
    ends = np.minimum(row_len, (r % seq_q) + 1 + offset).astype(np.int64)
    return np.zeros(rows, dtype=np.int64), np.maximum(ends, 0)


def topk_ascending(scores, topk, starts=None, ends=None, admissible=None):
    """scores [rows, n] float32 -> idx [rows, topk] int32 (ascending, -1 padded).

    Vectorised: one stable descending sort by score keeps the lower column first
    among equal scores; the window is enforced by a second stable sort on an
    out-of-window flag.  `admissible` ([rows, n] bool, optional) further
    restricts the candidates to its True columns inside the window: the
    finite-mask columns of a row that Megatron's fused_qk_topk_naive ranks
    after adding its mask (call shape cppmega/megatron/lemyx_dsa_warmup.py:169-176).
    """
    scores = np.asarray(scores, dtype=np.float32)
    rows, n = scores.shape
    if starts is None:
        starts = np.zeros(rows, dtype=np.int64)
    if ends is None:
        ends = np.full(rows, n, dtype=np.int64)
    starts = np.asarray(starts, dtype=np.int64)
    ends = np.asarray(ends, dtype=np.int64)
    col = np.arange(n)[None, :]
    inwin = (col >= starts[:, None]) & (col < ends[:, None])
    if admissible is not None:
        inwin = inwin & np.asarray(admissible, dtype=bool)
    key = np.where(np.isnan(scores), np.float32(np.inf), scores).astype(np.float64)
    key = key + 0.0  # -0.0 -> +0.0
    order = np.argsort(-key, axis=1, kind="stable")
    flag = (~np.take_along_axis(inwin, order, axis=1)).astype(np.int8)
    order2 = np.argsort(flag, axis=1, kind="stable")
    order = np.take_along_axis(order, order2, axis=1)
    nvalid = inwin.sum(axis=1)
    count = np.minimum(nvalid, topk)
    out = np.full((rows, topk), -1, dtype=np.int32)
    kk = min(topk, n)
    sel = order[:, :kk]
    take = np.arange(kk)[None, :] < count[:, None]
    sel = np.where(take, sel, np.iinfo(np.int64).max)
    sel.sort(axis=1)
    sel = np.where(sel == np.iinfo(np.int64).max, -1, sel)
    out[:, :kk] = sel.astype(np.int32)
    return out


def topk_bruteforce_row(row, topk, start=0, end=None, admissible=None):
    """Pure-Python reference for one row (tiny rows only); `admissible` is an
    optional per-column bool list restricting the candidates."""
    n = len(row)
    end = n if end is None else end

    def k(i):
        v = float(row[i])
        if v != v:
            v = float("inf")
        return (-v, i)

    cols = [i for i in range(start, max(start, end)) if admissible is None or admissible[i]]
    cand = sorted(cols, key=k)[:topk]
    cand.sort()
    return cand + [-1] * (topk - len(cand))


def topk_bytes(b, s, topk):
    """Algorithmic HBM bytes of causal top-k: fp32 causal scores read + int32 indices written."""
    return 4 * b * s * (s + 1) // 2 + 4 * b * s * topk


def mask_windows(mask):
    """Candidate windows of an additive mask [R, sq, sk] (numpy, float32):
    (starts, ends, plain) int32 [R, sq] -- the first finite column of each row,
    one past its last ((0, 0) when the row has none), and 1 where every entry
    in between is +0.0 (bit pattern 0: no finite bias, no -inf / NaN hole).
    The windows are the candidate sets of fused_qk_topk_naive's masked rows
    (index_scores + mask, call shapes cppmega/megatron/lemyx_dsa_warmup.py:169-176);
    Megatron itself is not vendored, so this is this build's contract (parity
    unpinned against Megatron), pinned by a per-element brute force
    (``mask_windows_bruteforce``) and hypothesis in the CPU tests."""
    m = np.ascontiguousarray(mask, dtype=np.float32)
    R, sq, sk = m.shape
    fin = np.isfinite(m)
    has = fin.any(-1)
    first = np.argmax(fin, axis=-1)
    last = sk - 1 - np.argmax(fin[..., ::-1], axis=-1)
    starts = np.where(has, first, 0).astype(np.int32)
    ends = np.where(has, last + 1, 0).astype(np.int32)
    col = np.arange(sk)[None, None, :]
    inside = (col >= starts[..., None]) & (col < ends[..., None])
    pos_zero = m.view(np.uint32) == 0
    plain = np.all(~inside | pos_zero, axis=-1).astype(np.int32)
    return starts, ends, plain


def mask_windows_bruteforce(row):
    """One mask row (a list of floats) -> (start, end, plain) by a plain loop."""
    import struct

    cols = [i for i, v in enumerate(row) if v == v and abs(v) != float("inf")]
    if not cols:
        return 0, 0, 1
    st, en = cols[0], cols[-1] + 1
    plain = all(struct.pack("<f", row[i]) == b"\0\0\0\0" for i in range(st, en))
    return st, en, int(plain)


def drop_masked_picks(scores, idx, plain=None):
    """Picks whose score is -inf become -1, the rest stay ascending with the -1
    padding at the end, on every row not flagged in `plain` (those are
    returned as they are).  scores [rows, sk] float32, idx [rows, k] (ascending,
    -1 padded) -> int64 [rows, k].  The repair the sync-free Megatron top-k
    needs after ranking index_scores + mask (masked picks become -1 as in
    cppmega/megatron/upstream_patches/apply_dsa_cg_patches.py:267-291)."""
    scores = np.asarray(scores, dtype=np.float32)
    idx = np.asarray(idx, dtype=np.int64)
    out = np.full(idx.shape, -1, dtype=np.int64)
    for r in range(idx.shape[0]):
        if plain is not None and plain[r]:
            out[r] = idx[r]
            continue
        keep = [c for c in idx[r] if c >= 0 and scores[r, c] != -np.inf]
        out[r, :len(keep)] = keep
    return out
