"""DSA indexer scores on gfx950 and the Megatron ``_compute_index_scores`` patch.

Drop-in for cppmega/megatron/dsa_indexer_fused_patch.py:
  * ``compute_index_scores_fused_bf16(q, weights, k, use_relu=True)`` (:71-133)
    -> [b, sq, sk] fp32 with score = sum_h w * ReLU(q_h . k), fp32 accumulate;
  * ``apply_dsa_indexer_fused_patch(force=False)`` (:136-173) installs it as
    ``megatron...dsa._compute_index_scores``.

The reference loops over heads with one fp32 bmm + 3 elementwise passes per
head; here one MFMA kernel computes every head and reduces over heads in
registers, writing each score once.  ``index_scores`` adds the causal modes the
fused top-k path uses (entries above the diagonal written as -inf or not at
all) and the e4m3 form with per-tensor scales.

The reference's loop is plain torch, so autograd carries the indexer's
gradient (from Megatron's KL loss) back to q, weights and k.  Here
``compute_index_scores_fused_bf16`` returns a tensor with that history whenever
grad mode is on and an input requires grad: ``IndexScores`` runs the forward
kernel and, in backward, ``index_scores_backward`` (two MFMA kernels that
recompute q.k, dsa_indexer_scores_backward).
"""
from __future__ import annotations

import logging

import torch

from . import _lib

log = logging.getLogger(__name__)

__all__ = ["IndexScores", "apply_dsa_indexer_fused_patch", "compute_index_scores_fused_bf16", "index_scores",
           "index_scores_backward"]

_PATCH_MARKER = "__cppmega_amd_dsa_indexer_fused_patched__"

CAUSAL_NONE = 0       # every (t, s)
CAUSAL_NEG_INF = 1    # s > t written as -inf
CAUSAL_LOWER = 2      # only s <= t written
CAUSAL_WINDOW = 3     # per-row [start, end) windows plus an additive mask, -inf elsewhere


def index_scores(q, weights, k, use_relu=True, causal=CAUSAL_NONE, q_scale=None, k_scale=None, out=None,
                 starts=None, ends=None, mask=None, row_plain=None):
    """q [sq,b,h,d] (bf16 or e4m3), weights [sq,b,h] (f32 or bf16), k [sk,b,d] -> [b,sq,sk] f32.

    For e4m3 q / k, q_scale and k_scale are one-element f32 tensors (per-tensor
    dequant factors, real = fp8 * scale).  causal=CAUSAL_WINDOW keeps, for row t
    of batch b, the columns [starts[b, t], ends[b, t]) (int32 device tensors
    broadcastable to [b, sq]) and adds ``mask`` there (f32, broadcastable to
    [b, sq, sk], or None); every other element is -inf.  ``row_plain`` (int32
    [b, sq], optional; ``mask_windows``' third output) flags rows whose mask is
    +0.0 on the whole window: their mask is not read (same result).
    """
    assert q.dim() == 4, f"q must be [sq,b,h,d], got {tuple(q.shape)}"
    assert k.dim() == 3, f"k must be [sk,b,d], got {tuple(k.shape)}"
    assert weights.dim() == 3, f"weights must be [sq,b,h], got {tuple(weights.shape)}"
    sq, b, h, d = q.shape
    sk, bk, dk = k.shape
    assert bk == b and dk == d, f"shape mismatch q={tuple(q.shape)} k={tuple(k.shape)}"
    assert tuple(weights.shape) == (sq, b, h), f"weights {tuple(weights.shape)} != {(sq, b, h)}"
    fp8 = q.dtype == torch.float8_e4m3fn
    if fp8:
        assert k.dtype == torch.float8_e4m3fn, "q and k must both be e4m3"
        assert q_scale is not None and k_scale is not None, "e4m3 indexer inputs need q_scale and k_scale"
        q_scale = q_scale.reshape(-1)[:1].to(torch.float32).contiguous()
        k_scale = k_scale.reshape(-1)[:1].to(torch.float32).contiguous()
    else:
        if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16:
            raise TypeError(f"indexer q/k must be bf16 or float8_e4m3fn, got {q.dtype}/{k.dtype}")
    if weights.dtype not in (torch.float32, torch.bfloat16):
        weights = weights.float()
    q, k, weights = q.contiguous(), k.contiguous(), weights.contiguous()
    if out is None:
        out = torch.empty((b, sq, sk), dtype=torch.float32, device=q.device)
    else:
        assert out.shape == (b, sq, sk) and out.dtype == torch.float32 and out.is_contiguous()
    dev = _lib.ensure_device(q)
    if causal == CAUSAL_WINDOW:
        assert starts is not None and ends is not None, "window mode needs starts and ends"
        starts = starts.to(device=q.device, dtype=torch.int32).expand(b, sq).contiguous()
        ends = ends.to(device=q.device, dtype=torch.int32).expand(b, sq).contiguous()
        bstride = 0
        if mask is not None:
            mask = mask.to(device=q.device, dtype=torch.float32)
            mask = mask.reshape(-1, *mask.shape[-2:]) if mask.dim() >= 3 else mask.reshape(1, *mask.shape)
            assert mask.shape[-2:] == (sq, sk) and mask.shape[0] in (1, b), \
                f"mask {tuple(mask.shape)} does not broadcast to {(b, sq, sk)}"
            mask = mask.contiguous()
            bstride = 0 if mask.shape[0] == 1 else sq * sk
        if row_plain is not None:
            row_plain = row_plain.to(device=q.device, dtype=torch.int32).expand(b, sq).contiguous()
        rc = _lib.load().dsa_indexer_scores_masked(
            q.data_ptr(), weights.data_ptr(), k.data_ptr(), out.data_ptr(), b, sq, sk, h, d,
            _lib.DTYPE_E4M3 if fp8 else _lib.DTYPE_BF16,
            _lib.DTYPE_F32 if weights.dtype == torch.float32 else _lib.DTYPE_BF16,
            _lib.ptr(q_scale), _lib.ptr(k_scale), starts.data_ptr(), ends.data_ptr(), _lib.ptr(mask), bstride,
            _lib.ptr(row_plain), 1 if use_relu else 0, _lib.stream_ptr(dev))
        _lib.check(rc, "dsa_indexer_scores_masked")
        return out
    rc = _lib.load().dsa_indexer_scores(
        q.data_ptr(), weights.data_ptr(), k.data_ptr(), out.data_ptr(), b, sq, sk, h, d,
        _lib.DTYPE_E4M3 if fp8 else _lib.DTYPE_BF16,
        _lib.DTYPE_F32 if weights.dtype == torch.float32 else _lib.DTYPE_BF16,
        _lib.ptr(q_scale), _lib.ptr(k_scale), int(causal), 1 if use_relu else 0, _lib.stream_ptr(dev))
    _lib.check(rc, "dsa_indexer_scores")
    return out


def index_scores_backward(grad, q, weights, k, use_relu=True, causal=False, starts=None, ends=None):
    """Gradients of ``index_scores`` (bf16 q / k) for grad = d loss / d scores
    [b, sq, sk]: returns (dq [sq,b,h,d] bf16, dweights [sq,b,h] in weights'
    dtype, dk [sk,b,d] bf16).  causal=True ignores grad above the diagonal
    (the entries a lower-triangle forward never wrote).  starts / ends (int32,
    broadcastable to [b, sq]; both or neither): the window-mode forward's row
    windows; grad outside them is ignored (the forward wrote -inf there
    whatever the raw score) and key tiles outside every window are skipped."""
    sq, b, h, d = q.shape
    sk = k.shape[0]
    assert q.dtype == torch.bfloat16 and k.dtype == torch.bfloat16, \
        f"the indexer backward takes bf16 q / k, got {q.dtype}/{k.dtype}"
    assert tuple(grad.shape) == (b, sq, sk), f"grad {tuple(grad.shape)} != {(b, sq, sk)}"
    if weights.dtype not in (torch.float32, torch.bfloat16):
        weights = weights.float()
    grad = grad.to(torch.float32).contiguous()
    q, k, weights = q.contiguous(), k.contiguous(), weights.contiguous()
    if (starts is None) != (ends is None):
        raise ValueError("give both starts and ends, or neither")
    if starts is not None:
        starts = starts.to(device=q.device, dtype=torch.int32).expand(b, sq).contiguous()
        ends = ends.to(device=q.device, dtype=torch.int32).expand(b, sq).contiguous()
    dq = torch.empty_like(q)
    dw = torch.empty_like(weights)
    dk = torch.empty_like(k)
    dev = _lib.ensure_device(q)
    lib = _lib.load()
    ws_bytes = int(lib.dsa_indexer_scores_backward_workspace_size(b, sq, sk, h, d))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
    rc = lib.dsa_indexer_scores_backward(
        grad.data_ptr(), q.data_ptr(), weights.data_ptr(), k.data_ptr(), dq.data_ptr(), dw.data_ptr(),
        dk.data_ptr(), b, sq, sk, h, d, _lib.DTYPE_BF16,
        _lib.DTYPE_F32 if weights.dtype == torch.float32 else _lib.DTYPE_BF16,
        1 if causal else 0, 1 if use_relu else 0, _lib.ptr(starts), _lib.ptr(ends), ws.data_ptr(), ws_bytes,
        _lib.stream_ptr(dev))
    _lib.check(rc, "dsa_indexer_scores_backward")
    return dq, dw, dk


class IndexScores(torch.autograd.Function):
    """Indexer scores with a backward to q, weights and k.

    forward(q, weights, k, use_relu, causal, starts, ends, mask, row_plain) ->
    [b, sq, sk] f32 with ``index_scores``' modes (CAUSAL_NONE, CAUSAL_NEG_INF,
    CAUSAL_LOWER, CAUSAL_WINDOW).  The lower-triangle modes write constants
    above the diagonal, which carry no gradient (causal backward).  The window
    mode is Megatron's ``scores + mask`` inside the row windows and the
    constant -inf outside them: inside, the raw scores receive the upstream
    gradient as autograd through the add gives it (mask holes included);
    outside, the output does not depend on the raw scores, so the gradient
    there is ignored and the backward computes only the key tiles inside the
    windows (a causal mask costs the lower-triangle backward).  Megatron's
    torch add would pass a gradient at -inf entries on to the raw scores; a
    finite loss of the scores (softmax, KL) gives exactly zero there.
    """

    @staticmethod
    def forward(ctx, q, weights, k, use_relu=True, causal=CAUSAL_NONE, starts=None, ends=None, mask=None,
                row_plain=None):
        out = index_scores(q, weights, k, use_relu=use_relu, causal=causal, starts=starts, ends=ends, mask=mask,
                           row_plain=row_plain)
        win = causal == CAUSAL_WINDOW
        ctx.save_for_backward(q, weights, k, *((starts, ends) if win else ()))
        ctx.win = win
        ctx.use_relu = use_relu
        ctx.causal = causal in (CAUSAL_NEG_INF, CAUSAL_LOWER)
        ctx.wdtype = weights.dtype
        return out

    @staticmethod
    def backward(ctx, grad):
        q, weights, k, *win = ctx.saved_tensors
        starts, ends = win if ctx.win else (None, None)
        dq, dw, dk = index_scores_backward(grad, q, weights, k, use_relu=ctx.use_relu, causal=ctx.causal,
                                           starts=starts, ends=ends)
        return dq, dw.to(ctx.wdtype), dk, None, None, None, None, None, None


def _needs_grad(*ts):
    return torch.is_grad_enabled() and any(t.requires_grad for t in ts)


def compute_index_scores_fused_bf16(q, weights, k, use_relu: bool = True):
    """Drop-in for Megatron DSA ``_compute_index_scores`` (bf16): [b, sq, sk] fp32,
    unmasked; differentiable with respect to q, weights and k like the
    reference's torch loop when grad mode is on and any of them requires grad."""
    if _needs_grad(q, weights, k):
        return IndexScores.apply(q, weights, k, use_relu, CAUSAL_NONE)
    return index_scores(q, weights, k, use_relu=use_relu, causal=CAUSAL_NONE)


def apply_dsa_indexer_fused_patch(*, force: bool = False, dsa_module=None) -> bool:
    """Install ``compute_index_scores_fused_bf16`` as Megatron's ``dsa._compute_index_scores``.

    Idempotent; raises if the Megatron DSA module or the attribute is absent.
    """
    dsa_mod = dsa_module
    if dsa_mod is None:
        from megatron.core.transformer.experimental_attention_variant import dsa as dsa_mod

    existing = getattr(dsa_mod, "_compute_index_scores", None)
    if existing is None:
        raise RuntimeError(
            "megatron.core.transformer.experimental_attention_variant.dsa."
            "_compute_index_scores not found — Megatron version mismatch?")
    if getattr(existing, _PATCH_MARKER, False) and not force:
        log.info("cppmega_amd DSA indexer patch already applied")
        return True

    def _compute_index_scores_fused(q, weights, k, use_relu: bool = True, **kwargs):
        return compute_index_scores_fused_bf16(q, weights, k, use_relu=use_relu)

    setattr(_compute_index_scores_fused, _PATCH_MARKER, True)
    dsa_mod._compute_index_scores = _compute_index_scores_fused
    log.info("cppmega_amd DSA indexer patch applied (gfx950 MFMA, heads reduced in registers)")
    return True
