"""AdaSplash (alpha-entmax attention) on the gfx950 HIP kernels.

Drop-ins for ``adasplash.adasplash(q, k, v, alpha=1.5, niter=10, is_causal=False,
varlen=None)`` (block-masked) and ``adasplash.adasplash_no_block_mask(...)``
(reference README.md:39-58; behaviour pinned by tests/test_adasplash.py and
tests/test_adasplash_no_block_mask.py).

q: [B, H, L, D], k, v: [B, H_kv, L, D] with H_kv dividing H (grouped-query attention: query
head h attends to K/V head h // (H / H_kv), read in place); float32 / float16 / bfloat16 on the
GPU, D <= 128.
varlen: optional [B] true lengths; keys j >= varlen[b] are masked and output rows
i >= varlen[b] are exactly zero.  The softmax scale is 1/sqrt(D).
The block-masked variant also records which (128-query x 64-key) tiles hold any p > 0
and skips the empty ones in the forward P V product and in both backward kernels.
"""
import torch

from ._lib import (
    DTYPE_CODE,
    check,
    check_inputs,
    kernel_head_dim,
    lib,
    prep_bhld,
    prep_varlen,
    ptr,
    stream_of,
    t4,
)


def _forward(q, k, v, alpha, niter, is_causal, varlen, use_mask, need_grad_state):
    D, scale = check_inputs(q, k, v)
    alpha = float(alpha)
    if not (1.0 < alpha <= 2.0):
        raise ValueError("alpha must lie in (1, 2]")
    Dk = kernel_head_dim(D)
    qp, kp, vp = (prep_bhld(x, Dk) for x in (q, k, v))
    B, H, L, _ = qp.shape
    vl = prep_varlen(varlen, B, q.device)
    out = torch.empty((B, H, L, Dk), device=q.device, dtype=q.dtype)
    tau = torch.empty((B, H, L), device=q.device, dtype=torch.float32)
    wn = torch.empty((B, H, L, Dk), device=q.device, dtype=torch.float32) if need_grad_state else None
    mask = None
    if use_mask:
        mw = lib().fla_adasplash_mask_words(L)
        mask = torch.empty((B, H, (L + 127) // 128, mw), device=q.device, dtype=torch.int32)
    rc = lib().fla_adasplash_fwd(
        t4(qp), t4(kp), t4(vp), t4(out), ptr(tau), ptr(wn), ptr(mask), ptr(vl),
        B, H, kp.shape[1], L, Dk, DTYPE_CODE[q.dtype], alpha, int(niter), int(bool(is_causal)), int(bool(use_mask)), scale,
        stream_of(q),
    )
    check(rc, "fla_adasplash_fwd")
    return out, tau, wn, mask, vl, (qp, kp, vp), D, Dk, scale


class AdaSplashFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, alpha, niter, is_causal, varlen, use_mask):
        out, tau, wn, mask, vl, (qp, kp, vp), D, Dk, scale = _forward(
            q, k, v, alpha, niter, is_causal, varlen, use_mask, True
        )
        ctx.save_for_backward(qp, kp, vp, tau, wn, mask, vl)
        ctx.cfg = (float(alpha), bool(is_causal), D, Dk, scale)
        return out[..., :D] if Dk != D else out

    @staticmethod
    def backward(ctx, do):
        qp, kp, vp, tau, wn, mask, vl = ctx.saved_tensors
        alpha, is_causal, D, Dk, scale = ctx.cfg
        B, H, L, _ = qp.shape
        dop = prep_bhld(do.to(qp.dtype), Dk)
        dq = torch.empty_like(qp)
        dk = torch.empty_like(kp)
        dv = torch.empty_like(vp)
        delta = torch.empty((B, H, L), device=qp.device, dtype=torch.float32)
        rc = lib().fla_adasplash_bwd(
            t4(qp), t4(kp), t4(vp), t4(dop), t4(dq), t4(dk), t4(dv), ptr(tau), ptr(wn), ptr(mask), ptr(vl),
            ptr(delta), B, H, kp.shape[1], L, Dk, DTYPE_CODE[qp.dtype], alpha, int(is_causal), scale, stream_of(qp),
        )
        check(rc, "fla_adasplash_bwd")
        if Dk != D:
            dq, dk, dv = dq[..., :D], dk[..., :D], dv[..., :D]
        return dq, dk, dv, None, None, None, None, None


def adasplash(q, k, v, alpha=1.5, niter=10, is_causal=False, varlen=None):
    """Block-masked AdaSplash attention (see module docstring)."""
    if torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v)):
        return AdaSplashFunction.apply(q, k, v, alpha, niter, is_causal, varlen, True)
    out, *_rest = _forward(q, k, v, alpha, niter, is_causal, varlen, True, False)
    D = q.shape[-1]
    return out[..., :D] if out.shape[-1] != D else out


def adasplash_stats(q, k, v, alpha=1.5, niter=10, is_causal=False, varlen=None, use_mask=True):
    """Forward only, returning (out, tau, block_mask): tau [B, H, L] in (alpha-1)*score units
    (+inf on padded rows), block_mask int32 [B, H, ceil(L/128), words] (None if use_mask is False)."""
    out, tau, _wn, mask, *_rest = _forward(q, k, v, alpha, niter, is_causal, varlen, use_mask, False)
    D = q.shape[-1]
    return (out[..., :D] if out.shape[-1] != D else out), tau, mask
