"""Lazy attention (elastic softmax with a windowed head-wise bias) on the gfx950 HIP kernels.

Drop-in for ``lazy_attention_triton(q, k, v, bias, tau, window_size=None, varlen=None)``
and ``LazyAttentionTritonFunc`` (reference lazy_attention_triton.py:503-541):

    out_i = sum_{j <= i} relu(softmax_j(q_i.k_j/sqrt(D) + bias[h, i-j]*1[0 <= i-j < W]) + tau_h/(i+1)) v_j

q: [B, H, L, D], k, v: [B, H_kv, L, D] (RoPE already applied; H_kv dividing H, query head h
reading K/V head h // (H / H_kv) in place, with no repeat_interleave), bias [H, >= W], tau [H],
varlen optional [B].
Gradients: dq, dk, dv in the input dtype; dbias / dtau in float32 and only when bias / tau
require grad (lazy_attention_triton.py:523-539).  Rows i >= varlen[b] are zero in the output
and in every gradient.

``return_mask=True`` (the block sparsity planned at CURSOR_TASKS.md:214-312) also returns
``bmask`` bool [B, H, ceil(L/64), ceil(L/64)]: block (r, c) is True iff some weight
relu(p + tau/i) > 0 links a query of rows 64r.. to a key of 64c..; the forward then skips the
P V products of empty tiles.  ``get_sparsity_stats(bmask)`` summarises it.
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


def _params(bias, tau, H, window_size):
    if bias.dim() != 2 or bias.shape[0] != H:
        raise ValueError(f"bias must be [H={H}, W], got {tuple(bias.shape)}")
    if tau.numel() != H:
        raise ValueError(f"tau must have H={H} entries")
    W = int(window_size)
    if W <= 0 or W > bias.shape[1]:
        raise ValueError(f"window_size={W} must lie in [1, bias.shape[1]={bias.shape[1]}]")
    b32 = bias.detach().to(torch.float32).contiguous()
    t32 = tau.detach().reshape(H).to(torch.float32).contiguous()
    return b32, t32, W


def _forward(q, k, v, bias, tau, window_size, varlen, need_w, want_mask=False):
    D, scale = check_inputs(q, k, v)
    Dk = kernel_head_dim(D)
    qp, kp, vp = (prep_bhld(x, Dk) for x in (q, k, v))
    B, H, L, _ = qp.shape
    b32, t32, W = _params(bias, tau, H, window_size)
    vl = prep_varlen(varlen, B, q.device)
    out = torch.empty((B, H, L, Dk), device=q.device, dtype=q.dtype)
    lse = torch.empty((B, H, L), device=q.device, dtype=torch.float32)
    wd = torch.empty((B, H, L, Dk), device=q.device, dtype=torch.float32) if need_w else None
    # the forward writes the boolean block mask directly (one byte per 64x64 block)
    nrb = (L + 63) // 64
    bmask = torch.empty((B, H, nrb, nrb), device=q.device, dtype=torch.bool) if want_mask else None
    rc = lib().fla_lazy_fwd(
        t4(qp), t4(kp), t4(vp), t4(out), ptr(b32), b32.shape[1], ptr(t32), W, ptr(lse), ptr(wd),
        None, ptr(bmask), int(want_mask), ptr(vl),
        B, H, kp.shape[1], L, Dk, DTYPE_CODE[q.dtype], scale, stream_of(q),
    )
    check(rc, "fla_lazy_fwd")
    return out, lse, wd, (qp, kp, vp), b32, t32, W, vl, D, Dk, scale, bmask


class LazyAttentionTritonFunc(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, bias, tau, window_size, varlen=None, want_mask=False):
        out, lse, wd, (qp, kp, vp), b32, t32, W, vl, D, Dk, scale, bmask = _forward(
            q, k, v, bias, tau, window_size, varlen, True, want_mask
        )
        ctx.save_for_backward(qp, kp, vp, b32, t32, lse, wd, vl)
        ctx.cfg = (W, D, Dk, scale, tuple(bias.shape))
        ctx.tau_shape = tuple(tau.shape)
        out = out[..., :D] if Dk != D else out
        if want_mask:
            ctx.mark_non_differentiable(bmask)
            return out, bmask
        return out

    @staticmethod
    def backward(ctx, do, *_dmask):
        qp, kp, vp, b32, t32, lse, wd, vl = ctx.saved_tensors
        W, D, Dk, scale, bshape = ctx.cfg
        B, H, L, _ = qp.shape
        need = ctx.needs_input_grad[3] or ctx.needs_input_grad[4]
        dop = prep_bhld(do.to(qp.dtype), Dk)
        dq = torch.empty_like(qp)
        dk = torch.empty_like(kp)
        dv = torch.empty_like(vp)
        dbias = torch.empty((H, W), device=qp.device, dtype=torch.float32) if need else None
        dtau = torch.empty((H,), device=qp.device, dtype=torch.float32) if need else None
        nbytes = int(lib().fla_lazy_bwd_workspace_size(B, H, L, W))
        ws = torch.empty((nbytes,), device=qp.device, dtype=torch.uint8)
        rc = lib().fla_lazy_bwd(
            t4(qp), t4(kp), t4(vp), t4(dop), t4(dq), t4(dk), t4(dv), ptr(b32), b32.shape[1], ptr(t32), W,
            ptr(lse), ptr(wd), ptr(vl), ptr(dbias), ptr(dtau), ptr(ws), nbytes, B, H, kp.shape[1], L, Dk,
            DTYPE_CODE[qp.dtype], scale, stream_of(qp),
        )
        check(rc, "fla_lazy_bwd")
        if Dk != D:
            dq, dk, dv = dq[..., :D], dk[..., :D], dv[..., :D]
        if need and bshape[1] != W:
            full = torch.zeros(bshape, device=qp.device, dtype=torch.float32)
            full[:, :W] = dbias
            dbias = full
        if need:
            dtau = dtau.reshape(ctx.tau_shape)
        return dq, dk, dv, dbias, dtau, None, None, None


def _decode_forward(q, k, v, bias, tau, window_size, varlen):
    """q [B, H, Lq, D] at the last Lq positions of each sequence against the cache k, v
    [B, H_kv, Lk, D] (Lq < Lk); varlen = cache lengths [B].  Inference only."""
    D, scale = check_inputs(q, k, v, kv_longer=True)
    Dk = kernel_head_dim(D)
    qp, kp, vp = (prep_bhld(x, Dk) for x in (q, k, v))
    B, H, Lq, _ = qp.shape
    Hkv, Lk = kp.shape[1], kp.shape[2]
    b32, t32, W = _params(bias, tau, H, window_size)
    vl = prep_varlen(varlen, B, q.device)
    out = torch.empty((B, H, Lq, Dk), device=q.device, dtype=q.dtype)
    nbytes = int(lib().fla_lazy_decode_workspace_size(B, H, Hkv, Lq, Lk, Dk))
    if nbytes == 0:
        raise ValueError(f"unsupported decode shape q {tuple(q.shape)}, k {tuple(k.shape)}")
    ws = torch.empty((nbytes,), device=q.device, dtype=torch.uint8)
    rc = lib().fla_lazy_decode_fwd(
        t4(qp), t4(kp), t4(vp), t4(out), ptr(b32), b32.shape[1], ptr(t32), W, ptr(vl), ptr(ws), nbytes,
        B, H, Hkv, Lq, Lk, Dk, DTYPE_CODE[q.dtype], scale, stream_of(q),
    )
    check(rc, "fla_lazy_decode_fwd")
    return out[..., :D] if Dk != D else out


def lazy_attention_triton(q, k, v, bias, tau, window_size=None, varlen=None, return_mask=False):
    """See the module docstring.  With q shorter than k, v (a KV cache: q holds the last
    q.shape[2] positions of each sequence, varlen the cache lengths) the inference-only decode
    kernels run instead; they produce no gradient."""
    if window_size is None:
        window_size = bias.shape[1]
    if q.dim() == 4 and k.dim() == 4 and q.shape[2] < k.shape[2]:
        if return_mask:
            raise ValueError("return_mask is not available on the KV-cache path")
        if torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v, bias, tau)):
            raise NotImplementedError("the KV-cache (Lq < Lk) path is inference only; wrap it in torch.no_grad()")
        return _decode_forward(q, k, v, bias, tau, window_size, varlen)
    if torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v, bias, tau)):
        return LazyAttentionTritonFunc.apply(q, k, v, bias, tau, window_size, varlen, bool(return_mask))
    res = _forward(q, k, v, bias, tau, window_size, varlen, False, bool(return_mask))
    out, bmask = res[0], res[-1]
    D = q.shape[-1]
    out = out[..., :D] if out.shape[-1] != D else out
    return (out, bmask) if return_mask else out


def get_sparsity_stats(bmask):
    """Block statistics of a ``return_mask`` mask (CURSOR_TASKS.md:246-258): ``block_density``
    (fraction of all blocks that are non-empty), ``visible_density`` (fraction of the causally
    visible blocks c <= r that are non-empty) and ``theoretical_speedup`` = 1 / block_density."""
    R, C = bmask.shape[-2:]
    vis = torch.ones(R, C, dtype=torch.bool, device=bmask.device).tril()
    density = bmask.float().mean().item()
    nvis = vis.sum().item() * (bmask.numel() // (R * C))
    return {
        "block_density": density,
        "visible_density": (bmask & vis).sum().item() / max(nvis, 1),
        "theoretical_speedup": 1.0 / max(density, 0.01),
    }
