"""Row-wise alpha-entmax oracle (numpy, float64).  TEST INFRASTRUCTURE ONLY.

alpha-entmax of a row x (Peters, Niculae & Martins 2019):

    p_j = [(alpha-1) x_j - tau]_+ ^ (1/(alpha-1)),   with tau chosen so sum_j p_j = 1.

Functions
---------
entmax_bisect      restates the bisection solver of the third-party ``entmax``
                   package (``entmax.root_finding.EntmaxBisectFunction``, version
                   unpinned at requirements-dev.txt:5; called by the reference's
                   tests at tests/test_adasplash.py:53 and
                   tests/test_triton_entmax.py:24,95).  Pinned by: the exact
                   sort-based closed forms below (alpha=1.5, 2), the softmax limit
                   (alpha -> 1), the known answers of tests/test_triton_entmax.py:66-85
                   and brute-force support enumeration on tiny rows.
sparsemax_sort     alpha=2 closed form (Martins & Astudillo 2016, sort + cumsum).
entmax15_sort      alpha=1.5 closed form (Peters et al. 2019, Alg. 2: per support
                   size k the threshold is the smaller root of a quadratic).
entmax_support_brute  brute force over support sizes (tiny rows only).
entmax_backward    Jacobian-vector product of the entmax package's backward:
                   U = p^(2-alpha) on the support, dx = U*dy - (sum U*dy / sum U) U.
                   Pinned by float64 finite differences and by torch autograd
                   through the sort-based closed forms (tests/test_oracle_entmax.py).
"""
import numpy as np


def _p(x, alpha):
    return np.maximum(x, 0.0) ** (1.0 / (alpha - 1.0))


def entmax_bisect(x, alpha=1.5, axis=-1, n_iter=50, ensure_sum_one=True):
    """Bisection entmax along ``axis`` (float64).

    Same bracket and update rule as the ``entmax`` package: start from
    tau_lo = max - 1 and tau_hi = max - (1/d)^(alpha-1) where d is the length
    of the axis (masked ``-inf`` entries count towards d), halve the bracket
    ``n_iter`` times, then renormalise so the row sums to one.
    """
    x = np.asarray(x, dtype=np.float64)
    x = np.moveaxis(x, axis, -1)
    d = x.shape[-1]
    z = x * (alpha - 1.0)
    mx = np.max(z, axis=-1, keepdims=True)
    tau_lo = mx - 1.0
    tau_hi = mx - (1.0 / d) ** (alpha - 1.0)
    f_lo = _p(z - tau_lo, alpha).sum(-1, keepdims=True) - 1.0
    dm = tau_hi - tau_lo
    p = None
    for _ in range(n_iter):
        dm = dm / 2.0
        tau_m = tau_lo + dm
        p = _p(z - tau_m, alpha)
        f_m = p.sum(-1, keepdims=True) - 1.0
        tau_lo = np.where(f_m * f_lo >= 0, tau_m, tau_lo)
    if ensure_sum_one:
        p = p / p.sum(-1, keepdims=True)
    return np.moveaxis(p, -1, axis)


def entmax_threshold(x, alpha, axis=-1, n_iter=200):
    """Threshold tau (in z = (alpha-1) x units) to float64 precision by bisection."""
    x = np.asarray(x, dtype=np.float64)
    x = np.moveaxis(x, axis, -1)
    d = x.shape[-1]
    z = x * (alpha - 1.0)
    mx = np.max(z, axis=-1, keepdims=True)
    lo = mx - 1.0
    hi = mx - (1.0 / d) ** (alpha - 1.0)
    for _ in range(n_iter):
        mid = 0.5 * (lo + hi)
        f = _p(z - mid, alpha).sum(-1, keepdims=True) - 1.0
        lo = np.where(f >= 0, mid, lo)
        hi = np.where(f >= 0, hi, mid)
    return np.moveaxis(0.5 * (lo + hi), -1, axis)


def sparsemax_sort(x, axis=-1):
    """alpha=2 entmax (sparsemax) by sorting: tau = (sum_{top k} x - 1) / k."""
    x = np.moveaxis(np.asarray(x, dtype=np.float64), axis, -1)
    zs = -np.sort(-x, axis=-1)
    k = np.arange(1, x.shape[-1] + 1, dtype=np.float64)
    cs = np.cumsum(zs, axis=-1)
    cond = 1.0 + k * zs > cs
    ksup = cond.sum(-1, keepdims=True)
    tau = (np.take_along_axis(cs, ksup - 1, -1) - 1.0) / ksup
    return np.moveaxis(np.maximum(x - tau, 0.0), -1, axis)


def entmax15_sort(x, axis=-1):
    """alpha=1.5 entmax by sorting.

    With z = x/2 sorted descending and support size k, sum_{j<k} (z_j - tau)^2 = 1
    gives tau_k = mean_k - sqrt((1 - k*var_k)/k); the support is the largest k
    with tau_k <= z_k.
    """
    x = np.moveaxis(np.asarray(x, dtype=np.float64), axis, -1)
    z = x / 2.0
    zs = -np.sort(-z, axis=-1)
    k = np.arange(1, x.shape[-1] + 1, dtype=np.float64)
    mean = np.cumsum(zs, -1) / k
    mean_sq = np.cumsum(zs * zs, -1) / k
    ss = k * (mean_sq - mean * mean)
    delta = np.maximum((1.0 - ss) / k, 0.0)
    tau = mean - np.sqrt(delta)
    ksup = (tau <= zs).sum(-1, keepdims=True)
    tau_star = np.take_along_axis(tau, ksup - 1, -1)
    return np.moveaxis(np.maximum(z - tau_star, 0.0) ** 2, -1, axis)


def entmax_support_brute(x, alpha):
    """Tiny 1-D rows only: try every support = top-k set, bisect tau on it, keep the consistent one."""
    x = np.asarray(x, dtype=np.float64)
    z = (alpha - 1.0) * x
    order = np.argsort(-z)
    beta = 1.0 / (alpha - 1.0)
    for k in range(1, len(z) + 1):
        s = z[order[:k]]
        lo, hi = s.min() - 1.0 - abs(s.min()), s.min()
        lo = min(lo, s.max() - 1.0)
        for _ in range(300):
            mid = 0.5 * (lo + hi)
            f = (np.maximum(s - mid, 0.0) ** beta).sum() - 1.0
            if f >= 0:
                lo = mid
            else:
                hi = mid
        tau = 0.5 * (lo + hi)
        rest_ok = k == len(z) or z[order[k]] <= tau + 1e-12
        if np.all(s > tau - 1e-12) and rest_ok:
            return np.maximum(z - tau, 0.0) ** beta
    raise AssertionError("no consistent support found")


def entmax_backward(y, dy, alpha, axis=-1):
    """d x for y = entmax(x): U = y^(2-alpha) on y>0; dx = U*dy - (sum U dy / sum U) U."""
    y = np.asarray(y, dtype=np.float64)
    dy = np.asarray(dy, dtype=np.float64)
    u = np.where(y > 0, np.where(y > 0, y, 1.0) ** (2.0 - alpha), 0.0)
    gx = u * dy
    q = gx.sum(axis, keepdims=True) / u.sum(axis, keepdims=True)
    return gx - q * u


def softmax(x, axis=-1):
    x = np.asarray(x, dtype=np.float64)
    e = np.exp(x - x.max(axis, keepdims=True))
    return e / e.sum(axis, keepdims=True)
