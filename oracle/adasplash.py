"""AdaSplash attention oracle (numpy, float64).  TEST INFRASTRUCTURE ONLY.

``reference_attention`` restates tests/test_adasplash.py:22-60 (the reference's
own torch oracle): scores q k^T / sqrt(D), keys j >= varlen[b] and (causal)
j > i set to -inf, row-wise alpha-entmax, p @ v, rows i >= varlen[b] zeroed
(:56-58).  The reference's tests feed ``entmax_bisect`` (50 bisection steps,
renormalised); ``method="bisect"`` reproduces that, ``method="exact"``
solves tau to float64 precision (64 bisection steps on a bracket of width
<= 1, then renormalisation) and is the default because it is the fixed point
both solvers approach.

``reference_attention_backward`` gives dq, dk, dv by the chain rule through the
entmax Jacobian (entmax package backward; tests/test_adasplash.py:94-122 compares
against autograd through the same oracle):
    dP = dO v^T,  U = p^(2-alpha) on the support,
    delta_i = sum_j U_ij dP_ij / sum_j U_ij,  dS = U (dP - delta),
    dq = dS k / sqrt(D),  dk = dS^T q / sqrt(D),  dv = p^T dO.
Rows i >= varlen[b] carry no gradient (their output is masked to zero).

``block_mask`` is the per-(128 query x 64 key) tile occupancy that the
block-masked forward stores: bit (r, c) is set iff some row i < varlen of
query tile r has p_ij > 0 for some key j of key tile c.

Pinned by: brute-force per-row loops over the sort-based closed forms
(alpha = 1.5, 2), the known answer of tests/test_adasplash.py:148-158 (zero q, k
and v = 1 give out = 1), padded rows exactly zero (:161-174), and for the
backward float64 finite differences plus torch autograd through a torch
restatement of the forward built on the sort-based entmax (tests/test_oracle_adasplash.py).
"""
import math

import numpy as np

from .entmax import entmax_bisect, entmax_threshold

BLOCK_Q = 128
BLOCK_K = 64


def _masks(B, L, varlen, is_causal):
    """valid[b, i, j]: key j visible from query i in batch row b."""
    valid = np.ones((B, L, L), dtype=bool)
    if varlen is not None:
        vl = np.asarray(varlen).reshape(B)
        valid &= (np.arange(L)[None, None, :] < vl[:, None, None])
    if is_causal:
        valid &= np.tril(np.ones((L, L), dtype=bool))[None]
    return valid


def _row_valid(B, L, varlen):
    if varlen is None:
        return np.ones((B, L), dtype=bool)
    vl = np.asarray(varlen).reshape(B)
    return np.arange(L)[None, :] < vl[:, None]


def entmax_rows(s, alpha, method="exact", n_iter=50):
    """p and tau (z units) for score rows s[..., L] that may hold -inf."""
    if method == "bisect":
        p = entmax_bisect(s, alpha, n_iter=n_iter)
        tau = None
    else:
        tau = entmax_threshold(s, alpha, n_iter=64)
        z = (alpha - 1.0) * s
        p = np.maximum(z - tau, 0.0) ** (1.0 / (alpha - 1.0))
        p = p / p.sum(-1, keepdims=True)
    return p, tau


def reference_attention(q, k, v, alpha=1.5, varlen=None, is_causal=False, method="exact", return_aux=False):
    """Forward of tests/test_adasplash.py:22-60 in float64, processed per (b, h) slice."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    B, H, L, D = q.shape
    valid = _masks(B, L, varlen, is_causal)
    rowv = _row_valid(B, L, varlen)
    out = np.zeros_like(q)
    P = np.zeros((B, H, L, L)) if return_aux else None
    TAU = np.zeros((B, H, L)) if return_aux else None
    for b in range(B):
        for h in range(H):
            s = q[b, h] @ k[b, h].T / math.sqrt(D)
            s = np.where(valid[b], s, -np.inf)
            p, tau = entmax_rows(s, alpha, method)
            # rows past the length hold no probability (a length-0 sequence has no finite
            # score at all, where entmax of an all -inf row is undefined)
            p = np.where(rowv[b][:, None], p, 0.0)
            o = p @ v[b, h]
            o[~rowv[b]] = 0.0
            out[b, h] = o
            if return_aux:
                P[b, h] = p
                TAU[b, h] = tau[:, 0] if tau is not None else np.nan
    if not return_aux:
        return out
    return out, {"p": P, "tau": TAU, "row_valid": rowv}


def reference_attention_backward(q, k, v, do, alpha=1.5, varlen=None, is_causal=False, method="exact"):
    """(dq, dk, dv) of ``reference_attention`` for upstream gradient ``do`` (float64)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    do = np.asarray(do, dtype=np.float64)
    B, H, L, D = q.shape
    valid = _masks(B, L, varlen, is_causal)
    rowv = _row_valid(B, L, varlen)
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    sc = 1.0 / math.sqrt(D)
    for b in range(B):
        for h in range(H):
            s = q[b, h] @ k[b, h].T * sc
            s = np.where(valid[b], s, -np.inf)
            p, _ = entmax_rows(s, alpha, method)
            p = np.where(rowv[b][:, None], p, 0.0)
            g = np.where(rowv[b][:, None], do[b, h], 0.0)
            dP = g @ v[b, h].T
            u = np.where(p > 0, np.where(p > 0, p, 1.0) ** (2.0 - alpha), 0.0)
            den = u.sum(-1, keepdims=True)  # 0 only on rows past the length
            delta = np.where(den > 0, (u * dP).sum(-1, keepdims=True) / np.where(den > 0, den, 1.0), 0.0)
            dS = u * (dP - delta)
            dq[b, h] = dS @ k[b, h] * sc
            dk[b, h] = dS.T @ q[b, h] * sc
            dv[b, h] = p.T @ g
    return dq, dk, dv


def block_mask(p, row_valid, block_q=BLOCK_Q, block_k=BLOCK_K):
    """bool [B, H, ceil(L/block_q), ceil(L/block_k)] tile occupancy of p > 0 over valid rows."""
    B, H, L, _ = p.shape
    Tr = -(-L // block_q)
    Tc = -(-L // block_k)
    nz = (p > 0) & row_valid[:, None, :, None]
    pad = np.zeros((B, H, Tr * block_q, Tc * block_k), dtype=bool)
    pad[:, :, :L, :L] = nz
    return pad.reshape(B, H, Tr, block_q, Tc, block_k).any(axis=(3, 5))


def pack_block_mask(m):
    """bool [..., Tr, Tc] -> uint32 [..., Tr, ceil(Tc/32)], bit c%32 of word c//32."""
    *lead, Tr, Tc = m.shape
    W = -(-Tc // 32)
    pad = np.zeros((*lead, Tr, W * 32), dtype=np.uint64)
    pad[..., :Tc] = m
    pad = pad.reshape(*lead, Tr, W, 32)
    return (pad << np.arange(32, dtype=np.uint64)).sum(-1).astype(np.uint32)
