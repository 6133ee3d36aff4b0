"""Row-wise alpha-entmax over the last dimension on the gfx950 HIP kernel.

Drop-in for ``adasplash.triton_entmax.triton_entmax(x, alpha=1.5, n_iter=10,
fast_math=True)`` (reference README.md:28-35; behaviour pinned by
tests/test_triton_entmax.py).  The threshold is solved to fp32 convergence (Newton from
below plus the closed forms for alpha = 1.5 and 2); ``n_iter`` and ``fast_math`` are
accepted for signature compatibility.
"""
import torch

from ._lib import DTYPE_CODE, check, lib, ptr, stream_of


def _forward(x, alpha, n_iter, fast_math):
    if not x.is_cuda:
        raise ValueError("triton_entmax expects a GPU tensor")
    if x.dtype not in DTYPE_CODE:
        raise TypeError(f"unsupported dtype {x.dtype}")
    alpha = float(alpha)
    if not (1.0 < alpha <= 2.0):
        raise ValueError("alpha must lie in (1, 2]")
    shape = x.shape
    n = shape[-1]
    x2 = x.reshape(-1, n).contiguous()
    y = torch.empty_like(x2)
    rc = lib().fla_entmax_fwd(
        ptr(x2), ptr(y), x2.shape[0], n, n, n, DTYPE_CODE[x.dtype], alpha, int(n_iter), int(bool(fast_math)),
        stream_of(x2),
    )
    check(rc, "fla_entmax_fwd")
    return y, alpha, shape


class EntmaxFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, alpha, n_iter, fast_math):
        y, alpha, shape = _forward(x, alpha, n_iter, fast_math)
        ctx.alpha = alpha
        ctx.save_for_backward(y)
        return y.reshape(shape)

    @staticmethod
    def backward(ctx, dy):
        (y,) = ctx.saved_tensors
        n = y.shape[-1]
        dy2 = dy.reshape(-1, n).to(y.dtype).contiguous()
        dx = torch.empty_like(y)
        rc = lib().fla_entmax_bwd(
            ptr(y), ptr(dy2), ptr(dx), y.shape[0], n, n, n, n, DTYPE_CODE[y.dtype], ctx.alpha, stream_of(y)
        )
        check(rc, "fla_entmax_bwd")
        return dx.reshape(dy.shape), None, None, None


def triton_entmax(x, alpha=1.5, n_iter=10, fast_math=True):
    if torch.is_grad_enabled() and x.requires_grad:
        return EntmaxFunction.apply(x, alpha, n_iter, fast_math)
    y, _alpha, shape = _forward(x, alpha, n_iter, fast_math)  # no autograd node needed
    return y.reshape(shape)
