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
    if not x.is_contiguous():
        x = x.contiguous()
    # Rows are the leading dims flattened; y has x's shape, so no reshapes are needed.
    y = torch.empty(shape, dtype=x.dtype, device=x.device)
    rows = x.numel() // n if n else 0
    rc = lib().fla_entmax_fwd(
        ptr(x), ptr(y), rows, n, n, n, DTYPE_CODE[x.dtype], alpha, int(n_iter), int(bool(fast_math)), stream_of(x),
    )
    check(rc, "fla_entmax_fwd")
    return y, alpha, shape


class EntmaxFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, alpha, n_iter, fast_math):
        y, alpha, shape = _forward(x, alpha, n_iter, fast_math)
        ctx.alpha = alpha
        ctx.save_for_backward(y)
        return y

    @staticmethod
    def backward(ctx, dy):
        (y,) = ctx.saved_tensors
        n = y.shape[-1]
        dy2 = dy.to(y.dtype).contiguous()
        dx = torch.empty(y.shape, dtype=y.dtype, device=y.device)
        rows = y.numel() // n if n else 0
        rc = lib().fla_entmax_bwd(
            ptr(y), ptr(dy2), ptr(dx), rows, n, n, n, n, DTYPE_CODE[y.dtype], ctx.alpha, stream_of(y)
        )
        check(rc, "fla_entmax_bwd")
        return dx, None, None, None


def triton_entmax(x, alpha=1.5, n_iter=10, fast_math=True):
    if torch.is_grad_enabled() and x.requires_grad:
        return EntmaxFunction.apply(x, alpha, n_iter, fast_math)
    return _forward(x, alpha, n_iter, fast_math)[0]  # no autograd node needed
