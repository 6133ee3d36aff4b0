"""Row-sampled and row-chunked AdaSplash oracle for full-size parity.  TEST INFRASTRUCTURE ONLY.

The same mathematics as ``oracle.adasplash.reference_attention`` /
``reference_attention_backward`` (tests/test_adasplash.py:22-60 of the reference), organised so
that one 8192-key row costs O(L*D) on the host:

* ``entmax_tau_topk`` solves the alpha-entmax threshold of each row on its K largest entries
  (``np.partition``), by bisection to float64 precision, and accepts the result only when the
  (K+1)-th largest entry lies at or below it -- the root over any superset of the support is the
  root over the whole row.  Rows that fail the check are solved again on the whole row.
* ``ada_rows`` gives, for a set of query rows of one (b, h) slice: scores, threshold, p, the
  output row, delta and the dq row.
* ``ada_slice`` walks all rows of one slice in chunks and also accumulates dk and dv.

Pinned against ``oracle.adasplash`` (itself pinned by closed forms, brute force, finite
differences and torch autograd) on causal, bidirectional and varlen slices, and against the
sort-based closed forms of ``oracle.entmax`` (tests/test_oracle_rows.py).
"""
import math

import numpy as np


def _bisect_tau(z, alpha, iters=64):
    """Threshold of rows z [R, n] (may hold -inf) by bisection on [max - 1, max]."""
    beta = 1.0 / (alpha - 1.0)
    mx = z.max(-1, keepdims=True)
    lo, hi = mx - 1.0, mx.copy()
    for _ in range(iters):
        mid = 0.5 * (lo + hi)
        f = (np.maximum(z - mid, 0.0) ** beta).sum(-1, keepdims=True) - 1.0
        ge = f >= 0
        lo = np.where(ge, mid, lo)
        hi = np.where(ge, hi, mid)
    return 0.5 * (lo + hi)[:, 0]


def entmax_tau_topk(z, alpha, kmax=1024):
    """tau [R] (z units) of rows z [R, n]; rows with no finite entry get +inf."""
    z = np.asarray(z, dtype=np.float64)
    R, n = z.shape
    tau = np.full(R, np.inf)
    live = np.isfinite(z).any(-1)
    if not live.any():
        return tau
    zl = z[live]
    if n <= kmax:
        tau[live] = _bisect_tau(zl, alpha)
        return tau
    part = -np.partition(-zl, kmax, axis=-1)  # [:, :kmax] = the kmax largest, [:, kmax] = the next
    t = _bisect_tau(part[:, :kmax], alpha)
    bad = part[:, kmax] > t
    if bad.any():
        t[bad] = _bisect_tau(zl[bad], alpha)
    tau[live] = t
    return tau


def ada_rows(q, k, v, do, rows, alpha, is_causal, n_valid, scale=None, tie_window=None, unit_round=None):
    """Oracle quantities of query rows ``rows`` of one (b, h) slice.

    q, k, v, do: [L, D] (float64-convertible); n_valid: the sequence length (keys j >= n_valid
    are masked, rows >= n_valid have zero output and gradient).  Returns a dict with
    s [R, L] scores (-inf where masked), z = (alpha-1) s, tau [R], p [R, L], out [R, D],
    delta [R], dq [R, D], u [R, L] = p^(2-alpha), ds [R, L] and the row validity [R].

    tie_window(z, tau) -> [R, L], optional: entries with |z - tau| within it are near-ties whose
    side of the threshold float32 rounding decides.  p is continuous there, but U = p^(2-alpha)
    jumps at alpha = 2 (from 0 to 1), and so do delta, dS, dq and dk.  With a window the result
    also holds ``ds_flip`` (dS with every near-tie entry moved to the other side; U on the
    boundary is its one-sided limit: 1 at alpha = 2, 0 below) and ``dq_slack`` [R, D] =
    |dq(flipped) - dq|: a float32 computation may legitimately land on either side.

    unit_round, optional: relative rounding of the matrix-product operands (2^-8 for bf16).  A
    kernel that feeds p and dS to the matrix cores in that type carries, on top of its float32
    rounding, errors bounded by ``out_round`` = u |p| |v| and ``dq_round`` = u |dS| |k| scale.
    """
    q, k, v = (np.asarray(t, dtype=np.float64) for t in (q, k, v))
    rows = np.asarray(rows, dtype=np.int64)
    L, D = k.shape
    sc = 1.0 / math.sqrt(D) if scale is None else scale
    s = (q[rows] @ k.T) * sc
    j = np.arange(L)[None, :]
    ok = j < n_valid
    if is_causal:
        ok = ok & (j <= rows[:, None])
    rowv = rows < n_valid
    ok = ok & rowv[:, None]
    s = np.where(ok, s, -np.inf)
    z = (alpha - 1.0) * s
    tau = entmax_tau_topk(z, alpha)
    beta = 1.0 / (alpha - 1.0)
    with np.errstate(invalid="ignore"):
        p = np.where(ok, np.maximum(z - tau[:, None], 0.0), 0.0) ** beta
    tot = p.sum(-1, keepdims=True)
    p = np.where(tot > 0, p / np.where(tot > 0, tot, 1.0), 0.0)
    out = p @ v
    res = {"s": s, "z": z, "tau": tau, "p": p, "out": out, "row_valid": rowv}
    if unit_round is not None:
        res["out_round"] = unit_round * (p @ np.abs(v))
    if do is not None:
        do = np.asarray(do, dtype=np.float64)
        g = np.where(rowv[:, None], do[rows], 0.0)
        dP = g @ v.T
        u = np.where(p > 0, np.where(p > 0, p, 1.0) ** (2.0 - alpha), 0.0)
        den = u.sum(-1)
        delta = np.where(den > 0, (u * dP).sum(-1) / np.where(den > 0, den, 1.0), 0.0)
        ds = u * (dP - delta[:, None])
        res.update(u=u, delta=delta, ds=ds, dq=(ds @ k) * sc, g=g)
        if unit_round is not None:
            res["dq_round"] = unit_round * (np.abs(ds) @ np.abs(k)) * sc
        if tie_window is not None:
            with np.errstate(invalid="ignore"):
                near = (np.abs(z - tau[:, None]) <= tie_window(z, tau)) & ok
            u_edge = 1.0 if alpha == 2.0 else 0.0
            uf = np.where(near, np.where(p > 0, 0.0, u_edge), u)
            denf = uf.sum(-1)
            deltaf = np.where(denf > 0, (uf * dP).sum(-1) / np.where(denf > 0, denf, 1.0), 0.0)
            dsf = uf * (dP - deltaf[:, None])
            res.update(near=near, ds_flip=dsf, dq_slack=np.abs((dsf - ds) @ k) * sc)
    return res


def ada_slice(q, k, v, do, alpha, is_causal, n_valid, chunk=256, scale=None, tie_window=None, unit_round=None):
    """Whole-slice forward and gradients of one (b, h) slice in row chunks (float64):
    out [L, D], tau [L], dq, dk, dv [L, D].  Rows >= n_valid are skipped (zero).
    With ``tie_window`` (see ada_rows) also dq_slack and dk_slack [L, D]: how far dq and dk move
    when the near-tie entries change side (|change| summed over the rows that hold them).
    With ``unit_round`` (see ada_rows) also the operand-rounding bounds out_round, dq_round,
    dk_round = u |dS|^T |q| scale and dv_round = u p^T |dO|."""
    q, k, v, do = (np.asarray(t, dtype=np.float64) for t in (q, k, v, do))
    L, D = q.shape
    sc = 1.0 / math.sqrt(D) if scale is None else scale
    out = np.zeros((L, D))
    dq = np.zeros((L, D))
    dk = np.zeros((L, D))
    dv = np.zeros((L, D))
    tau = np.full(L, np.inf)
    dq_slack = np.zeros((L, D))
    dk_slack = np.zeros((L, D))
    rnd = {n: np.zeros((L, D)) for n in ("out_round", "dq_round", "dk_round", "dv_round")}
    for r0 in range(0, min(L, n_valid), chunk):
        rows = np.arange(r0, min(r0 + chunk, L, n_valid))
        r = ada_rows(q, k, v, do, rows, alpha, is_causal, n_valid, sc, tie_window, unit_round)
        if unit_round is not None:
            rnd["out_round"][rows] = r["out_round"]
            rnd["dq_round"][rows] = r["dq_round"]
            rnd["dk_round"] += unit_round * (np.abs(r["ds"]).T @ np.abs(q[rows])) * sc
            rnd["dv_round"] += unit_round * (r["p"].T @ np.abs(r["g"]))
        out[rows] = r["out"]
        tau[rows] = r["tau"]
        dq[rows] = r["dq"]
        dk += r["ds"].T @ q[rows] * sc
        dv += r["p"].T @ r["g"]
        if tie_window is not None:
            dq_slack[rows] = r["dq_slack"]
            dk_slack += np.abs(r["ds_flip"] - r["ds"]).T @ np.abs(q[rows]) * sc
    res = {"out": out, "tau": tau, "dq": dq, "dk": dk, "dv": dv}
    if tie_window is not None:
        res.update(dq_slack=dq_slack, dk_slack=dk_slack)
    if unit_round is not None:
        res.update(rnd)
    return res


def mask_row_words(p_tile, block_k=64):
    """Packed block-mask word row (uint32 [ceil(ceil(L/block_k)/32)]) of one 128-row query tile
    from its p [rows, L]: bit c%32 of word c//32 set iff some p > 0 among keys of key tile c."""
    _, L = p_tile.shape
    tc = -(-L // block_k)
    pad = np.zeros((p_tile.shape[0], tc * block_k), dtype=bool)
    pad[:, :L] = p_tile > 0
    occ = pad.reshape(-1, tc, block_k).any(axis=(0, 2))
    nw = -(-tc // 32)
    words = np.zeros(nw, dtype=np.uint64)
    for c in np.nonzero(occ)[0]:
        words[c // 32] |= np.uint64(1) << np.uint64(c % 32)
    return words.astype(np.uint32)
