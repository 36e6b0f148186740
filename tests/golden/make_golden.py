"""Writes the known-answer fixtures under tests/golden/ (run from the repo root:
``python tests/golden/make_golden.py``).

The reference ships no golden vectors for the DSA path, and its kernels
(TileLang, Megatron, Transformer Engine) cannot run here.  The expected values
below come from a float64 / pure-Python computation written directly from the
definitions, sharing no code with the oracle or the HIP path:

  sparse_mla_*.npz  out_j = sum_s p_s v_s with p = softmax over the valid
                    slots (index in [0, S_kv), duplicates counted) of
                    scale * q . k_s; lse2 = log2(sum_s exp(scale * q . k_s));
                    gradients from the hand-derived formulas
                    dS_s = p_s (dO . v_s - dO . out), dq = scale sum_s dS_s k_s,
                    dk_s += scale dS_s q, dv_s += p_s dO (v = first d_v dims of
                    the kv row).  All-masked rows give out 0, lse2 -inf.
  indexer.npz       scores[b, t, j] = sum_h w[t, b, h] relu(q[t, b, h] . k[j, b]).
  topk.npz          per row: columns [start, end) sorted by (score desc, index
                    asc) with NaN as +inf and -0 == +0, first min(topk, n)
                    taken, returned ascending, -1 padded.
  fp8.npz           e4m3fn code of x * (448 / amax(|x|)) chosen by a brute-force
                    nearest search over the 254 finite codes (ties to the code
                    with an even mantissa, saturation at +-448).
  indexer_loss_*.npz per-position KL of the DSA indexer loss from explicit loops:
                    per head, a softmax over the columns s <= t (and, sparse, in
                    the row's top-k set) of scale * q . k; the head mean P; the
                    index softmax Q over all columns (sparse: the top-k set); then
                    sum_s P (ln(P + 1e-10) - ln(Q + 1e-10)).  A row with no
                    admissible column is NaN.

Inputs are bf16-representable (stored as their uint16 bit patterns), so every
implementation reads exactly the same numbers.
"""
from __future__ import annotations

import math
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LOG2E = 1.0 / math.log(2.0)


def bf16_bits(x):
    """float32 -> bf16 bit pattern (round to nearest even), no NaN inputs."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def bf16_value(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


# ---------------------------------------------------------------------------
# SparseMLA
# ---------------------------------------------------------------------------
def sparse_mla_expected(q, kv, idx, do, scale, d_v):
    """q [B,S,H,D], kv [B,Skv,G,D], idx [B,S,G,K] int, do [B,S,H,d_v] (float64)."""
    B, S, H, D = q.shape
    Skv, G = kv.shape[1], kv.shape[2]
    hpg = H // G
    out = np.zeros((B, S, H, d_v))
    lse2 = np.full((B, S, H), -np.inf)
    dq = np.zeros((B, S, H, D))
    dkv = np.zeros((B, Skv, G, D))
    for b in range(B):
        for t in range(S):
            for h in range(H):
                g = h // hpg
                slots = [int(j) for j in idx[b, t, g] if 0 <= int(j) < Skv]
                if not slots:
                    continue
                qv = q[b, t, h]
                logits = [scale * float(np.dot(qv, kv[b, j, g])) for j in slots]
                m = max(logits)
                e = [math.exp(x - m) for x in logits]
                z = sum(e)
                p = [x / z for x in e]
                o = np.zeros(d_v)
                for ps, j in zip(p, slots):
                    o += ps * kv[b, j, g, :d_v]
                out[b, t, h] = o
                lse2[b, t, h] = (m + math.log(z)) * LOG2E
                dov = do[b, t, h]
                base = float(np.dot(dov, o))
                for ps, j in zip(p, slots):
                    ds = ps * (float(np.dot(dov, kv[b, j, g, :d_v])) - base)
                    dq[b, t, h] += scale * ds * kv[b, j, g]
                    dkv[b, j, g] += scale * ds * qv
                    dkv[b, j, g, :d_v] += ps * dov
    return out, lse2, dq, dkv


def causal_topk_indices(rng, S, Skv, K):
    idx = np.full((S, K), -1, dtype=np.int32)
    for t in range(S):
        n = min(t + 1, Skv)
        pick = np.sort(rng.choice(n, size=min(K, n), replace=False))
        idx[t, :len(pick)] = pick
    return idx


def make_sparse_mla(name, seed, B, S, Skv, H, G, D, d_v, K, std=0.5):
    rng = np.random.default_rng(seed)
    qb = bf16_bits(rng.standard_normal((B, S, H, D)) * std)
    kvb = bf16_bits(rng.standard_normal((B, Skv, G, D)) * std)
    dob = bf16_bits(rng.standard_normal((B, S, H, d_v)))
    idx = np.stack([np.stack([causal_topk_indices(rng, S, Skv, K) for _ in range(G)], axis=1)
                    for _ in range(B)])                       # [B,S,G,K]
    # edge cases the reference's adapter and kernels see: a fully masked row,
    # duplicated indices, out-of-range values (masked like -1), unsorted slots
    idx[0, S - 1, 0, :] = -1
    idx[0, S - 2, 0, :4] = [3, 3, 1, 3]
    idx[0, S - 3, 0, :3] = [Skv + 5, -7, 2 ** 31 - 1]
    idx[-1, S - 4, -1, :] = idx[-1, S - 4, -1, ::-1].copy()
    scale = D ** -0.5
    out, lse2, dq, dkv = sparse_mla_expected(bf16_value(qb), bf16_value(kvb), idx, bf16_value(dob), scale, d_v)
    np.savez_compressed(os.path.join(HERE, name), q_bits=qb, kv_bits=kvb, do_bits=dob, indices=idx,
                        scale=np.float32(scale), d_v=np.int32(d_v),
                        out=out.astype(np.float32), lse2=lse2.astype(np.float32),
                        dq=dq.astype(np.float32), dkv=dkv.astype(np.float32))


# ---------------------------------------------------------------------------
# Indexer
# ---------------------------------------------------------------------------
def make_indexer(name, seed, Sq, Sk, B, H, D):
    rng = np.random.default_rng(seed)
    qb = bf16_bits(rng.standard_normal((Sq, B, H, D)))
    kb = bf16_bits(rng.standard_normal((Sk, B, D)))
    w = (rng.standard_normal((Sq, B, H)) / 4.0).astype(np.float32)
    q, k = bf16_value(qb), bf16_value(kb)
    scores = np.zeros((B, Sq, Sk))
    for b in range(B):
        for t in range(Sq):
            for j in range(Sk):
                acc = 0.0
                for h in range(H):
                    acc += float(w[t, b, h]) * max(0.0, float(np.dot(q[t, b, h], k[j, b])))
                scores[b, t, j] = acc
    np.savez_compressed(os.path.join(HERE, name), q_bits=qb, k_bits=kb, w=w, scores=scores)


# ---------------------------------------------------------------------------
# Top-k
# ---------------------------------------------------------------------------
def topk_row(row, k, start, end):
    def key(i):
        v = float(row[i])
        if v != v:
            v = math.inf
        if v == 0.0:
            v = 0.0
        return (-v, i)
    cand = sorted(range(start, max(start, end)), key=key)[:k]
    cand.sort()
    return cand + [-1] * (k - len(cand))


def make_topk(name, seed, rows, n, k):
    rng = np.random.default_rng(seed)
    s = rng.standard_normal((rows, n)).astype(np.float32)
    s[0::4] = np.round(s[0::4] * 2) / 2              # heavy ties
    s[1] = 0.0
    s[1, 1::3] = -0.0                                # signed zeros are equal
    s[2, ::7] = np.nan                               # NaN ranks as +inf
    s[3, ::5] = -np.inf
    s[5, :] = 1.0                                    # all equal
    s[6, 10:20] = np.inf
    starts = np.zeros(rows, dtype=np.int32)
    ends = np.full(rows, n, dtype=np.int32)
    ends[8:] = rng.integers(0, n + 1, size=rows - 8)
    starts[8:] = np.minimum(rng.integers(0, n // 2, size=rows - 8), ends[8:])
    ends[9] = starts[9]                              # empty window
    ends[10] = starts[10] + k // 2                   # shorter than k
    out = np.array([topk_row(s[r], k, int(starts[r]), int(ends[r])) for r in range(rows)], dtype=np.int32)
    np.savez_compressed(os.path.join(HERE, name), scores=s, starts=starts, ends=ends, topk=np.int32(k), out=out)


# ---------------------------------------------------------------------------
# FP8 e4m3fn tensorwise quantisation
# ---------------------------------------------------------------------------
def e4m3_table():
    vals = []
    for c in range(256):
        s = -1.0 if c & 0x80 else 1.0
        e, m = (c >> 3) & 0xF, c & 7
        if e == 0xF and m == 7:
            vals.append(math.nan)
        elif e == 0:
            vals.append(s * m * 2.0 ** -9)
        else:
            vals.append(s * (1 + m / 8.0) * 2.0 ** (e - 7))
    return vals


def e4m3_nearest(v, table):
    if v != v:
        return 0x7F
    best, best_err = None, None
    for c, tv in enumerate(table):
        if tv != tv:
            continue
        err = abs(tv - v)
        if best is None or err < best_err or (err == best_err and (c & 1) == 0 and (best & 1) == 1):
            best, best_err = c, err
    if abs(v) > 448.0:
        best = 0x7E | (0x80 if v < 0 else 0)
    if best in (0x00, 0x80):  # zero keeps the input's sign
        best = 0x80 if math.copysign(1.0, v) < 0 else 0x00
    return best


def make_fp8(name, seed, n):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(n).astype(np.float32)
    x[rng.random(n) < 0.01] *= 20.0
    x = np.clip(x, -27.5, 27.5)
    x[0] = 28.0                                      # amax 28 -> scale exactly 16
    x[1:9] = [0.0, -0.0, 1e-30, -1e-30, 3.0e-3, -5.5e-4, 7.0, -7.0]
    # exact halfway points between neighbouring codes after scaling (ties to
    # even mantissa): 1.0|1.125, 1.125|1.25, 16|18, 18|20, 416|448, 0|2^-9,
    # 2^-9|2^-8, 2^-6|2^-6+2^-9, largest subnormal|2^-6
    ties = np.array([1.0625, 1.1875, 17.0, 19.0, 432.0, 2.0 ** -10, 3 * 2.0 ** -10,
                     0.0166015625, 0.0146484375], dtype=np.float32)
    x[9:9 + len(ties)] = ties / np.float32(16.0)
    x[9 + len(ties):9 + 2 * len(ties)] = -ties / np.float32(16.0)
    amax = np.float32(np.max(np.abs(x)))
    scale = np.float32(448.0) / amax
    assert scale == np.float32(16.0)
    y = (x * scale).astype(np.float32)
    table = e4m3_table()
    codes = np.array([e4m3_nearest(float(v), table) for v in y], dtype=np.uint8)
    np.savez_compressed(os.path.join(HERE, name), x=x, scale=np.float32(scale),
                        scale_inv=np.float32(np.float32(1.0) / scale), codes=codes)


# ---------------------------------------------------------------------------
# DSA indexer KL loss
# ---------------------------------------------------------------------------
def indexer_loss_rows_expected(idx_scores, topk, q, k, scale, sparse):
    """idx_scores [B,Sq,Sk], topk [B,Sq,K], q [Sq,B,H,D], k [Sk,B,G,D] (float64) -> [B,Sq]."""
    Sq, B, H, D = q.shape
    Sk, G = k.shape[0], k.shape[2]
    rows = np.zeros((B, Sq))
    for b in range(B):
        for t in range(Sq):
            chosen = set(int(j) for j in topk[b, t] if 0 <= j < Sk) if sparse else set(range(Sk))
            att_cols = [s for s in range(Sk) if s <= t and s in chosen]
            if not att_cols or not chosen:
                rows[b, t] = math.nan
                continue
            P = [0.0] * Sk
            for h in range(H):
                g = h // (H // G)
                logit = {s: scale * sum(float(q[t, b, h, d]) * float(k[s, b, g, d]) for d in range(D))
                         for s in att_cols}
                mx = max(logit.values())
                z = sum(math.exp(v - mx) for v in logit.values())
                for s in att_cols:
                    P[s] += math.exp(logit[s] - mx) / z / H
            idx_cols = sorted(chosen)
            mx = max(float(idx_scores[b, t, s]) for s in idx_cols)
            z = sum(math.exp(float(idx_scores[b, t, s]) - mx) for s in idx_cols)
            tot = 0.0
            for s in range(Sk):
                if P[s] == 0.0:
                    continue
                Qs = math.exp(float(idx_scores[b, t, s]) - mx) / z if s in chosen else 0.0
                tot += P[s] * (math.log(P[s] + 1e-10) - math.log(Qs + 1e-10))
            rows[b, t] = tot
    return rows


def make_indexer_loss(name, seed, B, Sq, Sk, H, G, D, K):
    rng = np.random.default_rng(seed)
    qb = bf16_bits(rng.standard_normal((Sq, B, H, D)))
    kb = bf16_bits(rng.standard_normal((Sk, B, G, D)))
    idx_scores = rng.standard_normal((B, Sq, Sk)).astype(np.float32)
    # reference-test style: K distinct columns drawn from all of [0, Sk) (rows
    # with no column <= t exist), and a causal set with one column <= t per row
    topk_any = np.stack([rng.permutation(Sk)[:K] for _ in range(B * Sq)]).reshape(B, Sq, K).astype(np.int64)
    topk_causal = topk_any.copy()
    for b in range(B):
        for t in range(Sq):
            if not any(0 <= j <= t for j in topk_causal[b, t]):
                topk_causal[b, t, 0] = rng.integers(0, t + 1)
                if len(set(topk_causal[b, t].tolist())) < K:  # keep the set distinct
                    free = [j for j in range(Sk) if j not in set(topk_causal[b, t].tolist())]
                    topk_causal[b, t, 1:] = np.array(free[:K - 1])
    scale = 1.0 / math.sqrt(D)
    q, k = bf16_value(qb), bf16_value(kb)
    sc = idx_scores.astype(np.float64)
    dense = indexer_loss_rows_expected(sc, topk_any, q, k, scale, False)
    sparse_any = indexer_loss_rows_expected(sc, topk_any, q, k, scale, True)
    sparse_causal = indexer_loss_rows_expected(sc, topk_causal, q, k, scale, True)
    np.savez_compressed(os.path.join(HERE, name), q_bits=qb, k_bits=kb, index_scores=idx_scores,
                        topk_any=topk_any, topk_causal=topk_causal, scale=np.float64(scale),
                        rows_dense=dense, rows_sparse_any=sparse_any, rows_sparse_causal=sparse_causal)
    print(f"wrote {name}")


# ---------------------------------------------------------------------------
# Top-k index mask
# ---------------------------------------------------------------------------
def make_index_mask(name, seed, b, s_q, s_kv, topk, s0, s1):
    """The reference reproducer's fixture shape (b=2, s_q=64, s_kv=256, topk=8,
    ~15% -1 sentinels), plus out-of-range columns; expected mask by loops."""
    rng = np.random.default_rng(seed)
    idx = rng.integers(0, s_kv, size=(b, s1 - s0, topk)).astype(np.int64)
    idx[rng.random(idx.shape) < 0.15] = -1
    idx[0, 0, :] = -1                      # a row of sentinels only
    idx[1, 1, 0] = s_kv + 3                # past the row: skipped
    idx[1, 2, :2] = 0                      # a real column 0 next to sentinels
    idx[1, 2, 2] = -1
    mask = np.full((b, s_q, s_kv), -np.inf, dtype=np.float32)
    for bb in range(b):
        for r in range(s1 - s0):
            for j in range(topk):
                c = int(idx[bb, r, j])
                if 0 <= c < s_kv:
                    mask[bb, s0 + r, c] = 0.0
    np.savez_compressed(os.path.join(HERE, name), idx=idx, s0=np.int64(s0), s1=np.int64(s1),
                        s_kv=np.int64(s_kv), mask=mask)
    print(f"wrote {name}")


FIXTURES = {
    "indexer_loss": lambda: (
        make_indexer_loss("indexer_loss_h4.npz", 16, B=1, Sq=24, Sk=24, H=4, G=4, D=64, K=8),
        make_indexer_loss("indexer_loss_g2.npz", 17, B=2, Sq=20, Sk=28, H=8, G=2, D=32, K=6)),
    "index_mask": lambda: make_index_mask("index_mask.npz", 18, b=2, s_q=64, s_kv=256, topk=8, s0=8, s1=40),
}


def main():
    import sys
    if len(sys.argv) > 1:  # regenerate only the named fixture families
        for name in sys.argv[1:]:
            FIXTURES[name]()
        return
    make_sparse_mla("sparse_mla_d128.npz", 11, B=1, S=16, Skv=16, H=16, G=1, D=128, d_v=64, K=16)
    make_sparse_mla("sparse_mla_d64_g2.npz", 12, B=2, S=8, Skv=20, H=32, G=2, D=64, d_v=32, K=40)
    make_indexer("indexer.npz", 13, Sq=20, Sk=28, B=2, H=16, D=64)
    make_topk("topk.npz", 14, rows=40, n=300, k=32)
    make_fp8("fp8.npz", 15, n=4096)
    for make in FIXTURES.values():
        make()


if __name__ == "__main__":
    main()
