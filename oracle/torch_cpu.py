"""The reference's PyTorch CPU path, in float32 torch.  TEST / BASELINE INFRASTRUCTURE ONLY.

The reference checks its kernels against ``reference_attention`` (tests/test_adasplash.py:22-60):
scores q k^T / sqrt(D), masked entries -inf, ``entmax_bisect`` of the third-party ``entmax``
package (version unpinned, requirements-dev.txt:5; default n_iter = 50, renormalised), p v, and
autograd for the gradients, whose entmax backward is dX = U dY - (sum U dY / sum U) U with
U = Y^(2-alpha).  ``attention_rows`` restates that path for a block of query rows of one
(b, h) slice, float32 on the CPU, forward and backward, so that ``bench.py`` can time it on the
host cores as the CPU baseline.  Pinned against the float64 oracle (oracle.adasplash) at float32
tolerance in tests/test_oracle_rows.py.
"""
import math

import torch


def entmax_bisect(x, alpha, n_iter=50):
    """Bisection alpha-entmax over the last dim (the entmax package's algorithm, float32)."""
    d = x.shape[-1]
    z = x * (alpha - 1.0)
    mx = z.max(-1, keepdim=True).values
    tau_lo = mx - 1.0
    tau_hi = mx - (1.0 / d) ** (alpha - 1.0)
    beta = 1.0 / (alpha - 1.0)
    f_lo = torch.clamp(z - tau_lo, min=0).pow(beta).sum(-1, keepdim=True) - 1.0
    dm = tau_hi - tau_lo
    p = None
    for _ in range(n_iter):
        dm = dm / 2
        tau_m = tau_lo + dm
        p = torch.clamp(z - tau_m, min=0).pow(beta)
        f_m = p.sum(-1, keepdim=True) - 1.0
        tau_lo = torch.where(f_m * f_lo >= 0, tau_m, tau_lo)
    return p / p.sum(-1, keepdim=True)


def attention_rows(q, k, v, do, rows, alpha, is_causal=True, n_iter=50):
    """Forward and backward contributions of query rows ``rows`` (a contiguous range) of one
    (b, h) slice: returns out [R, D], dq [R, D], and the rows' contributions to dk, dv [L, D]."""
    L, D = k.shape
    sc = 1.0 / math.sqrt(D)
    r0, r1 = int(rows[0]), int(rows[-1]) + 1
    s = (q[r0:r1] @ k.T) * sc
    if is_causal:
        j = torch.arange(L)[None, :]
        i = torch.arange(r0, r1)[:, None]
        s = s.masked_fill(j > i, float("-inf"))
    p = entmax_bisect(s, alpha, n_iter)
    out = p @ v
    g = do[r0:r1]
    dP = g @ v.T
    u = torch.where(p > 0, p.clamp_min(1e-30).pow(2.0 - alpha), torch.zeros_like(p))
    delta = (u * dP).sum(-1, keepdim=True) / u.sum(-1, keepdim=True)
    ds = u * (dP - delta)
    dq = (ds @ k) * sc
    dk = (ds.T @ q[r0:r1]) * sc
    dv = p.T @ g
    return out, dq, dk, dv
