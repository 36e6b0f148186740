"""CPU restatement of SparseMLA forward / backward (bf16 and FP8 tensorwise).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Semantics follow the reference kernels:
  forward  cppmega/megatron/sparse_mla_ops/tilelang_sparse_mla_fwd.py:137-290
           (gather kv rows per slot, QK^T over d_qk, masked -inf for the -1
           sentinel, exp2 softmax with log2(e) folded into the scale,
           P rounded to bf16 before PV, LSE2 = log2(sumexp) + m * scale')
  backward cppmega/megatron/sparse_mla_ops/tilelang_sparse_mla_bwd.py:123-167
           (Delta = sum O*dO), :204-419 (P = exp2(s*scale' - LSE2),
           dP = dO V^T, dS = P (dP - Delta) scale, P/dS rounded to bf16,
           dQ = dS K, dKV[:, :dv] += dS^T Q[:, :dv] + P^T dO,
           dKV[:, dv:] += dS^T Q_tail, fp32 accumulation cast to bf16)
  fp8 fwd  cppmega/megatron/sparse_mla_ops/tilelang_sparse_mla_fwd_fp8.py:341-375
           (QK^T on e4m3 codes times q_scale * kv_scale[row]; V dequantised
           to bf16 per row)
  fp8 bwd  cppmega/megatron/sparse_mla_ops/tilelang_sparse_mla_bwd_fp8.py:316-434
           (Q and KV dequantised to bf16 for the dP / dQ / dKV GEMMs)

Index convention: a slot is masked when its index is outside [0, S_kv)
(the reference masks exactly -1; its adapter maps every out-of-range index
to -1 first, cppmega/megatron/sparse_mla_ops/sparse_mla.py:670-678).
All-masked (token, head) rows give out = 0, lse2 = -inf, zero gradients
(the reference yields 0/0 there, tilelang_sparse_mla_fwd.py:225,281).
"""
from __future__ import annotations

import torch

LOG2E = 1.4426950408889634


def _as4(x):
    return x if x.dim() == 4 else x.unsqueeze(0)


def _default_scale(sm_scale, d_qk):
    # tilelang_sparse_mla_fwd.py:157-160 / tilelang_sparse_mla_bwd.py:236-238
    return float(d_qk) ** -0.5 if sm_scale is None else float(sm_scale)


def _bf16r(x):
    """Round an fp32 tensor to bf16 and back (RNE)."""
    return x.to(torch.bfloat16).to(torch.float32)


def _gather_rows(kv_bg, idx, s_kv):
    """kv_bg [S_kv, D] float, idx [T, topk] int -> rows [T, topk, D], valid [T, topk]."""
    valid = (idx >= 0) & (idx < s_kv)
    safe = torch.where(valid, idx, torch.zeros_like(idx)).long()
    return kv_bg[safe], valid


def sparse_mla_fwd(q, kv, indices, sm_scale=None, d_v=None, round_p_bf16=True,
                   chunk=256, q_scale=None, kv_scale=None):
    """Returns (out fp32 [B,S,H,d_v], lse2 fp32 [B,S,H]); 3-D inputs keep 3-D outputs.

    When q/kv are float8_e4m3fn, q_scale [B,S] and kv_scale [B,S_kv] dequantise
    them as in the FP8 kernel (scores from e4m3 codes times both scales, V
    dequantised to bf16 per row).
    """
    squeeze = q.dim() == 3
    q, kv, indices = _as4(q), _as4(kv), _as4(indices)
    fp8 = q.dtype == torch.float8_e4m3fn
    B, S, H, Dqk = q.shape
    _, Skv, G, _ = kv.shape
    d_v = Dqk if d_v is None else int(d_v)
    hpg = H // G
    scale = _default_scale(sm_scale, Dqk)
    sl2 = scale * LOG2E
    if fp8:
        q_scale = q_scale.reshape(B, S).float()
        kv_scale = kv_scale.reshape(B, Skv).float()
    out = torch.zeros(B, S, H, d_v, dtype=torch.float32)
    lse = torch.full((B, S, H), float("-inf"), dtype=torch.float32)
    for b in range(B):
        for g in range(G):
            kv_bg = kv[b, :, g, :].float()
            for s0 in range(0, S, chunk):
                s1 = min(S, s0 + chunk)
                idx = indices[b, s0:s1, g, :]
                rows, valid = _gather_rows(kv_bg, idx, Skv)        # [T,k,D]
                qh = q[b, s0:s1, g * hpg:(g + 1) * hpg, :].float()  # [T,h,D]
                s = torch.bmm(qh, rows.transpose(1, 2))            # [T,h,k]
                if fp8:
                    safe = torch.where(valid, idx, torch.zeros_like(idx)).long()
                    ks = kv_scale[b][safe]                          # [T,k]
                    s = s * q_scale[b, s0:s1, None, None] * ks[:, None, :]
                    vrows = _bf16r(rows[..., :d_v] * ks[..., None])
                else:
                    vrows = rows[..., :d_v]
                s = s.masked_fill(~valid[:, None, :], float("-inf"))
                m = s.amax(-1, keepdim=True)
                m_safe = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
                p = torch.exp2((s - m_safe) * sl2)
                sumexp = p.sum(-1)
                p_mm = _bf16r(p) if round_p_bf16 else p
                o = torch.bmm(p_mm, vrows)
                nz = sumexp > 0
                o = torch.where(nz[..., None], o / sumexp.clamp_min(1e-38)[..., None],
                                torch.zeros_like(o))
                l2 = torch.where(nz, torch.log2(sumexp.clamp_min(1e-38)) + m_safe[..., 0] * sl2,
                                 torch.full_like(sumexp, float("-inf")))
                out[b, s0:s1, g * hpg:(g + 1) * hpg] = o
                lse[b, s0:s1, g * hpg:(g + 1) * hpg] = l2
    if squeeze:
        return out[0], lse[0]
    return out, lse


def sparse_mla_bwd(q, kv, o, do, indices, lse2, sm_scale=None, d_v=None,
                   round_bf16=True, chunk=256, q_scale=None, kv_scale=None):
    """Returns (dq fp32 [B,S,H,Dqk], dkv fp32 [B,S_kv,G,Dqk]); grad_lse is ignored
    as in cppmega/megatron/sparse_mla_ops/sparse_mla.py:395-411."""
    squeeze = q.dim() == 3
    q, kv, o, do, indices = _as4(q), _as4(kv), _as4(o), _as4(do), _as4(indices)
    lse2 = lse2 if lse2.dim() == 3 else lse2.unsqueeze(0)
    fp8 = q.dtype == torch.float8_e4m3fn
    B, S, H, Dqk = q.shape
    _, Skv, G, _ = kv.shape
    d_v = o.shape[-1] if d_v is None else int(d_v)
    hpg = H // G
    scale = _default_scale(sm_scale, Dqk)
    sl2 = scale * LOG2E
    rb = _bf16r if round_bf16 else (lambda x: x)
    if fp8:
        q_scale = q_scale.reshape(B, S).float()
        kv_scale = kv_scale.reshape(B, Skv).float()
    # preprocess: Delta = sum_d O * dO in fp32 (tilelang_sparse_mla_bwd.py:123-167)
    delta = (o.float() * do.float()).sum(-1)
    dq = torch.zeros(B, S, H, Dqk, dtype=torch.float32)
    dkv = torch.zeros(B, Skv, G, Dqk, dtype=torch.float32)
    for b in range(B):
        for g in range(G):
            kv_bg = kv[b, :, g, :].float()
            for s0 in range(0, S, chunk):
                s1 = min(S, s0 + chunk)
                idx = indices[b, s0:s1, g, :]
                rows, valid = _gather_rows(kv_bg, idx, Skv)
                hs = slice(g * hpg, (g + 1) * hpg)
                qh = q[b, s0:s1, hs, :].float()
                doh = do[b, s0:s1, hs, :].float()
                s = torch.bmm(qh, rows.transpose(1, 2))
                if fp8:
                    safe = torch.where(valid, idx, torch.zeros_like(idx)).long()
                    ks = kv_scale[b][safe]
                    qs = q_scale[b, s0:s1]
                    s = s * qs[:, None, None] * ks[:, None, :]
                    krows = _bf16r(rows * ks[..., None])            # K/V dequant
                    qmm = _bf16r(qh * qs[:, None, None])            # Q dequant
                else:
                    krows = rows
                    qmm = qh
                s = s.masked_fill(~valid[:, None, :], float("-inf"))
                l2 = lse2[b, s0:s1, hs].float()
                l2_safe = torch.where(torch.isfinite(l2), l2, torch.zeros_like(l2))
                p = torch.exp2(s * sl2 - l2_safe[..., None])
                p = torch.where(torch.isfinite(l2)[..., None], p, torch.zeros_like(p))
                dp = torch.bmm(doh, krows[..., :d_v].transpose(1, 2))
                ds = p * (dp - delta[b, s0:s1, hs][..., None]) * scale
                p_b, ds_b = rb(p), rb(ds)
                dq[b, s0:s1, hs] = torch.bmm(ds_b, krows)
                contrib = torch.bmm(ds_b.transpose(1, 2), qmm)       # [T,k,Dqk]
                contrib[..., :d_v] += torch.bmm(p_b.transpose(1, 2), doh)
                contrib = contrib * valid[..., None]
                safe = torch.where(valid, idx, torch.zeros_like(idx)).long()
                dkv[b, :, g, :].index_add_(0, safe.reshape(-1),
                                           contrib.reshape(-1, Dqk))
    if squeeze:
        return dq[0], dkv[0]
    return dq, dkv


def sparse_mla_autograd_f64(q, kv, indices, sm_scale=None, d_v=None):
    """Closed-form masked sparse attention in float64 built from differentiable
    torch ops: out = softmax_j(scale q.k_j) V_j over valid slots (duplicates
    counted per occurrence), lse2 = logsumexp * log2(e).  Used to pin the
    explicit forward / backward above (autograd gives the exact gradient)."""
    B, S, H, Dqk = q.shape
    _, Skv, G, _ = kv.shape
    d_v = Dqk if d_v is None else int(d_v)
    hpg = H // G
    scale = _default_scale(sm_scale, Dqk)
    outs, lses = [], []
    for g in range(G):
        idx = indices[:, :, g, :]
        valid = (idx >= 0) & (idx < Skv)
        safe = torch.where(valid, idx, torch.zeros_like(idx)).long()
        kvg = kv[:, :, g, :]                                   # [B,Skv,D]
        rows = torch.stack([kvg[b][safe[b]] for b in range(B)])  # [B,S,k,D]
        qg = q[:, :, g * hpg:(g + 1) * hpg, :]                 # [B,S,h,D]
        s = torch.einsum("bshd,bskd->bshk", qg, rows) * scale
        s = s.masked_fill(~valid[:, :, None, :], float("-inf"))
        lse_nat = torch.logsumexp(s, dim=-1)                   # [B,S,h]
        p = torch.softmax(s, dim=-1)
        p = torch.nan_to_num(p, nan=0.0)
        outs.append(torch.einsum("bshk,bskd->bshd", p, rows[..., :d_v]))
        lses.append(lse_nat * LOG2E)
    return torch.cat(outs, dim=2), torch.cat(lses, dim=2)


def delta_f32(o, do):
    """Delta = sum_d O * dO (tilelang_sparse_mla_bwd.py:123-167)."""
    return (o.float() * do.float()).sum(-1)


def flops_fwd(B, S, H, topk, d_qk, d_v):
    """Reference FLOP convention (cppmega/megatron/tilelang_sparse_mla/sparse_mla_fwd.py:276-277)."""
    return 2 * B * S * H * topk * (d_qk + d_v)


def flops_bwd(B, S, H, topk, d_qk, d_v):
    """Reference FLOP convention (cppmega/megatron/tilelang_sparse_mla/sparse_mla_bwd.py:327-344)."""
    return 2 * B * S * H * topk * (3 * d_qk + 2 * d_v)


__all__ = [
    "LOG2E", "sparse_mla_fwd", "sparse_mla_bwd", "sparse_mla_autograd_f64",
    "delta_f32", "flops_fwd", "flops_bwd",
]


# ---------------------------------------------------------------------------
# MXFP8 block-scaled forward
# ---------------------------------------------------------------------------
MX_BLOCK = 32


def mxfp8_quantize(x, block=MX_BLOCK):
    """OCP Microscaling (MX v1.0) E4M3 quantisation along the last dim: per block
    of `block` elements the shared scale is 2^(floor(log2(amax)) - 8) (8 = the
    largest e4m3 exponent), elements are x / scale cast to e4m3fn with
    round-to-nearest-even, saturating at +-448; an all-zero block has scale 1.
    Returns (data e4m3fn [..., D], scale f32 [..., D / block]).  The reference
    probe quantises with quack's to_mx (not vendored): its exact scale rule is
    parity unpinned here; the kernels take any f32 block scales."""
    xf = x.float()
    shp = xf.shape
    blocks = xf.reshape(*shp[:-1], shp[-1] // block, block)
    amax = blocks.abs().amax(-1)
    exp = torch.where(amax > 0, torch.floor(torch.log2(amax.clamp_min(1e-38))) - 8, torch.zeros_like(amax))
    scale = torch.exp2(exp)
    data = (blocks / scale[..., None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return data.reshape(shp), scale.float()


def dequantize_blockwise(data, scale, block=MX_BLOCK, out_dtype=torch.bfloat16):
    """value * scale[block], as _dequantize_mxfp8_tensor
    (cppmega/megatron/sparse_mla_ops/tilelang_sparse_mla_blockscaled_fused.py:961-969)."""
    shp = data.shape
    v = data.float().reshape(*shp[:-1], shp[-1] // block, block) * scale.float()[..., None]
    return v.reshape(shp).to(out_dtype)


def sparse_mla_fwd_mxfp8(q8, kv8, q_scale, kv_scale, indices, sm_scale=None, d_v=None, chunk=256):
    """MXFP8 block-scaled SparseMLA forward, restating the reference kernel
    sparse_mla_blockscaled_mxfp8_fwd (tilelang_sparse_mla_blockscaled_fused.py:337-415):
    for every 32-channel block the q.k product over the e4m3 codes is scaled by
    q_scale[b,s,h,blk] * kv_scale[b,row,g,blk] and summed over blocks; exp2
    softmax; V = bf16(code * kv_scale[row, d // 32]); P rounded to bf16; LSE in
    log2 units.  q8 [B,S,H,D], kv8 [B,S_kv,G,D] e4m3fn, scales f32 [..., D/32].
    Returns (out fp32 [B,S,H,d_v], lse2 [B,S,H])."""
    B, S, H, D = q8.shape
    _, Skv, G, _ = kv8.shape
    nb = D // MX_BLOCK
    d_v = D if d_v is None else int(d_v)
    hpg = H // G
    scale = _default_scale(sm_scale, D)
    sl2 = scale * LOG2E
    out = torch.zeros(B, S, H, d_v, dtype=torch.float32)
    lse = torch.full((B, S, H), float("-inf"), dtype=torch.float32)
    qf = q8.float().reshape(B, S, H, nb, MX_BLOCK)
    for b in range(B):
        for g in range(G):
            kv_bg = kv8[b, :, g, :].float()                          # [Skv, D]
            ks_bg = kv_scale[b, :, g, :].float()                     # [Skv, nb]
            for s0 in range(0, S, chunk):
                s1 = min(S, s0 + chunk)
                idx = indices[b, s0:s1, g, :]
                rows, valid = _gather_rows(kv_bg, idx, Skv)          # [T,k,D]
                safe = torch.where(valid, idx, torch.zeros_like(idx)).long()
                ks = ks_bg[safe]                                     # [T,k,nb]
                qs = q_scale[b, s0:s1, g * hpg:(g + 1) * hpg, :].float()  # [T,h,nb]
                qb = qf[b, s0:s1, g * hpg:(g + 1) * hpg]             # [T,h,nb,32]
                rb = rows.reshape(*rows.shape[:2], nb, MX_BLOCK)     # [T,k,nb,32]
                part = torch.einsum("thcd,tkcd->thkc", qb, rb)       # per-block partials
                s = (part * qs[:, :, None, :] * ks[:, None, :, :]).sum(-1)   # [T,h,k]
                vblk = rows[..., :d_v].reshape(*rows.shape[:2], d_v // MX_BLOCK, MX_BLOCK)
                vrows = _bf16r((vblk * ks[..., : d_v // MX_BLOCK, None]).reshape(*rows.shape[:2], d_v))
                s = s.masked_fill(~valid[:, None, :], float("-inf"))
                m = s.amax(-1, keepdim=True)
                m_safe = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
                p = torch.exp2((s - m_safe) * sl2)
                sumexp = p.sum(-1)
                o = torch.bmm(_bf16r(p), vrows)
                nz = sumexp > 0
                o = torch.where(nz[..., None], o / sumexp.clamp_min(1e-38)[..., None], torch.zeros_like(o))
                l2 = torch.where(nz, torch.log2(sumexp.clamp_min(1e-38)) + m_safe[..., 0] * sl2,
                                 torch.full_like(sumexp, float("-inf")))
                out[b, s0:s1, g * hpg:(g + 1) * hpg] = o
                lse[b, s0:s1, g * hpg:(g + 1) * hpg] = l2
    return out, lse
