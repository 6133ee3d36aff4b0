"""Lazy-Attention oracle (numpy, float64).  TEST INFRASTRUCTURE ONLY.

Restates the maths of lazy_attention_triton.py in closed form:

forward (:9-174)
    s_ij  = q_i . k_j / sqrt(D) + bias[h, i-j] * 1[0 <= i-j < W]     (:58-73)
    valid = j <= i  and  j < varlen[b]                                (:74-78)
    LSE_i = logsumexp_{valid j} s_ij                                  (:80-88)
    p_ij  = exp(s_ij - LSE_i)
    e_ij  = relu(p_ij + tau_h / (i+1)) on j <= i, 0 above the diagonal (:158-168)
    out_i = sum_{j < varlen} e_ij v_j; rows i >= varlen are zero      (:172-174)

backward (:180-497)
    dP_ij = dO_i . v_j;  m_ij = 1[p_ij + tau_h/(i+1) > 0] * 1[j <= i]
    delta_i = sum_j m_ij p_ij dP_ij                                   (:253-268)
    dS_ij = p_ij (m_ij dP_ij - delta_i)                               (:376-377)
    dq = dS k / sqrt(D);  dk = dS^T q / sqrt(D);  dv = e^T dO          (:379, :487-494)
    dbias[h, d] = sum_{b, i-j=d} dS_ij for 0 <= d < W                 (:384-386, :645-647)
    dtau[h] = sum_{b,i,j} m_ij dP_ij / (i+1)                          (:389-395, :648-649)
Keys j >= varlen contribute nothing (the kernels load v_j = 0 there) and rows
i >= varlen carry no gradient.

The bias window is 0 <= d < W as in the kernel (lazy_attention_triton.py:62) and
compare_scratch_flash.py:52, not 0 <= d <= W as in tests/test_lazy_attention_triton.py:65.

Pinned by: torch float64 autograd through a restatement of
compare_scratch_flash.py:45-71 (forward values and every gradient), tau = 0
reducing to causal softmax attention with bias, tau = -100 giving zero output
(tests/test_lazy_attention.py:28-52), and finite differences (tests/test_oracle_lazy.py).
"""
import math

import numpy as np


def _scores(q, k, bias, window, varlen, b, h, L):
    D = q.shape[-1]
    s = q[b, h] @ k[b, h].T / math.sqrt(D)
    i = np.arange(L)[:, None]
    j = np.arange(L)[None, :]
    d = i - j
    inwin = (d >= 0) & (d < window)
    s = s + np.where(inwin, bias[h, np.clip(d, 0, window - 1)], 0.0)
    valid = d >= 0
    keyok = np.ones((1, L), dtype=bool)
    if varlen is not None:
        keyok = j < int(varlen[b])
    return s, valid, keyok, d, inwin


def _softmax_rows(sm, ok):
    """p = exp(sm - LSE) per row and LSE; a row with no visible key (a length-0 sequence) has
    p = 0 and LSE = -inf."""
    mx = sm.max(-1, keepdims=True)
    mx = np.where(np.isfinite(mx), mx, 0.0)
    with np.errstate(divide="ignore", invalid="ignore"):
        lse = mx + np.log(np.exp(sm - mx).sum(-1, keepdims=True))
        p = np.where(ok & np.isfinite(lse), np.exp(sm - lse), 0.0)
    return p, lse


def lazy_forward(q, k, v, bias, tau, window=None, varlen=None, return_aux=False):
    q, k, v = (np.asarray(t, dtype=np.float64) for t in (q, k, v))
    bias = np.asarray(bias, dtype=np.float64)
    tau = np.asarray(tau, dtype=np.float64)
    if window is None:
        window = bias.shape[1]
    B, H, L, D = q.shape
    out = np.zeros_like(q)
    lse_all = np.zeros((B, H, L))
    for b in range(B):
        n = L if varlen is None else int(varlen[b])
        for h in range(H):
            s, valid, keyok, _, _ = _scores(q, k, bias, window, varlen, b, h, L)
            sm = np.where(valid & keyok, s, -np.inf)
            p, lse = _softmax_rows(sm, valid & keyok)
            ti = tau[h] / np.arange(1, L + 1)[:, None]
            e = np.where(valid, np.maximum(p + ti, 0.0), 0.0)
            e = np.where(keyok, e, 0.0)
            o = e @ v[b, h]
            o[n:] = 0.0
            out[b, h] = o
            lse_all[b, h] = lse[:, 0]
    if return_aux:
        return out, lse_all
    return out


def lazy_backward(q, k, v, bias, tau, do, window=None, varlen=None):
    """Returns dq, dk, dv, dbias [H, bias.shape[1]], dtau [H] in float64."""
    q, k, v, do = (np.asarray(t, dtype=np.float64) for t in (q, k, v, do))
    bias = np.asarray(bias, dtype=np.float64)
    tau = np.asarray(tau, dtype=np.float64)
    if window is None:
        window = bias.shape[1]
    B, H, L, D = q.shape
    sc = 1.0 / math.sqrt(D)
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    dbias = np.zeros_like(bias)
    dtau = np.zeros_like(tau)
    for b in range(B):
        n = L if varlen is None else int(varlen[b])
        for h in range(H):
            s, valid, keyok, d, inwin = _scores(q, k, bias, window, varlen, b, h, L)
            sm = np.where(valid & keyok, s, -np.inf)
            p, lse = _softmax_rows(sm, valid & keyok)
            inv_i = 1.0 / np.arange(1, L + 1)[:, None]
            m = (p + tau[h] * inv_i > 0) & valid & keyok
            e = np.where(valid & keyok, np.maximum(p + tau[h] * inv_i, 0.0), 0.0)
            g = do[b, h].copy()
            g[n:] = 0.0
            dP = g @ v[b, h].T
            delta = (np.where(m, p * dP, 0.0)).sum(-1, keepdims=True)
            dS = p * (np.where(m, dP, 0.0) - delta)
            dq[b, h] = dS @ k[b, h] * sc
            dk[b, h] = dS.T @ q[b, h] * sc
            dv[b, h] = e.T @ g
            dS_w = np.where(inwin, dS, 0.0)
            for dd in range(min(window, L)):
                dbias[h, dd] += np.trace(dS_w, offset=-dd)
            dtau[h] += (np.where(m, dP, 0.0) * inv_i).sum()
    if varlen is not None:
        for b in range(B):
            n = int(varlen[b])
            dq[b, :, n:] = 0.0
            dk[b, :, n:] = 0.0
            dv[b, :, n:] = 0.0
    return dq, dk, dv, dbias, dtau


def lazy_weights(q, k, bias, tau, window=None, varlen=None):
    """e [B, H, L, L] = relu(p + tau/(i+1)) on valid (j <= i, j < varlen) entries, 0 elsewhere
    and on rows i >= varlen; with `margin` [B, H, L, L] = |p + tau/(i+1)| for tie detection."""
    q, k = (np.asarray(t, dtype=np.float64) for t in (q, k))
    bias = np.asarray(bias, dtype=np.float64)
    tau = np.asarray(tau, dtype=np.float64)
    if window is None:
        window = bias.shape[1]
    B, H, L, _ = q.shape
    e = np.zeros((B, H, L, L))
    margin = np.full((B, H, L, L), np.inf)
    for b in range(B):
        n = L if varlen is None else int(varlen[b])
        for h in range(H):
            s, valid, keyok, _, _ = _scores(q, k, bias, window, varlen, b, h, L)
            ok = valid & keyok
            sm = np.where(ok, s, -np.inf)
            mx = sm.max(-1, keepdims=True)
            lse = mx + np.log(np.exp(sm - mx).sum(-1, keepdims=True))
            pt = np.exp(sm - lse) + tau[h] / np.arange(1, L + 1)[:, None]
            w = np.where(ok, np.maximum(pt, 0.0), 0.0)
            w[n:] = 0.0
            e[b, h] = w
            margin[b, h] = np.where(ok, np.abs(pt), np.inf)
            margin[b, h, n:] = np.inf
    return e, margin


def lazy_block_mask(e, block=64):
    """bool [B, H, ceil(L/block), ceil(L/block)]: block (r, c) holds some e > 0 -- the block
    sparsity planned at CURSOR_TASKS.md:214-245 (BLOCK_M = BLOCK_N = 64)."""
    B, H, L, _ = e.shape
    nb = -(-L // block)
    pad = nb * block - L
    ep = np.pad(e > 0, ((0, 0), (0, 0), (0, pad), (0, pad)))
    return ep.reshape(B, H, nb, block, nb, block).any(axis=(3, 5))
