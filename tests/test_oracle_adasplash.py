"""Pins the AdaSplash attention oracle (forward, backward, block mask).

Checks: brute-force per-row loops over the sort-based closed forms, the reference's
known answers (tests/test_adasplash.py:148-174), the bisect/exact agreement, torch
autograd through a torch restatement of tests/test_adasplash.py:22-60 built on the
sort-based (differentiable) entmax, and finite differences.
"""
import math

import numpy as np
import pytest
import torch

from oracle.adasplash import (
    block_mask,
    pack_block_mask,
    reference_attention,
    reference_attention_backward,
)
from oracle.entmax import entmax15_sort, sparsemax_sort
from test_oracle_entmax import _torch_entmax15, _torch_sparsemax


def _rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


@pytest.mark.parametrize("alpha", [1.5, 2.0])
@pytest.mark.parametrize("causal", [False, True])
def test_forward_vs_row_loops(alpha, causal):
    B, H, L, D = 2, 2, 40, 16
    q, k, v = _rand((B, H, L, D), 0), _rand((B, H, L, D), 1), _rand((B, H, L, D), 2)
    varlen = np.array([40, 27])
    out = reference_attention(q, k, v, alpha, varlen, causal)
    ref = np.zeros_like(out)
    ent = entmax15_sort if alpha == 1.5 else sparsemax_sort
    for b in range(B):
        for h in range(H):
            for i in range(varlen[b]):
                n = min(varlen[b], i + 1) if causal else varlen[b]
                s = np.array([q[b, h, i] @ k[b, h, j] / math.sqrt(D) for j in range(n)])
                p = ent(s)
                ref[b, h, i] = sum(p[j] * v[b, h, j] for j in range(n))
    np.testing.assert_allclose(out, ref, atol=1e-10)


def test_bisect_and_exact_agree():
    q, k, v = _rand((1, 2, 64, 32), 3), _rand((1, 2, 64, 32), 4), _rand((1, 2, 64, 32), 5)
    a = reference_attention(q, k, v, 1.333, None, True, method="bisect")
    b = reference_attention(q, k, v, 1.333, None, True, method="exact")
    np.testing.assert_allclose(a, b, atol=1e-10)


def test_known_answers():
    # zero q, k and v = 1 give out = 1 (tests/test_adasplash.py:148-158)
    z = np.zeros((1, 1, 64, 64))
    out = reference_attention(z, z, np.ones_like(z), 1.5)
    np.testing.assert_allclose(out, 1.0, atol=1e-12)
    # padded rows are exactly zero (tests/test_adasplash.py:161-174)
    q, k, v = _rand((2, 1, 64, 16), 6), _rand((2, 1, 64, 16), 7), _rand((2, 1, 64, 16), 8)
    out = reference_attention(q, k, v, 1.5, np.array([40, 17]))
    assert (out[0, :, 40:] == 0).all() and (out[1, :, 17:] == 0).all()


def _torch_forward(q, k, v, alpha, varlen, causal):
    B, H, L, D = q.shape
    s = q @ k.transpose(-1, -2) / math.sqrt(D)
    valid = torch.ones(B, 1, L, L, dtype=torch.bool)
    if varlen is not None:
        valid &= (torch.arange(L)[None, :] < torch.as_tensor(varlen)[:, None])[:, None, None, :]
    if causal:
        valid &= torch.tril(torch.ones(L, L, dtype=torch.bool))
    s = s.masked_fill(~valid, -1e30)
    p = (_torch_entmax15 if alpha == 1.5 else _torch_sparsemax)(s)
    out = p @ v
    if varlen is not None:
        rowv = (torch.arange(L)[None, :] < torch.as_tensor(varlen)[:, None])[:, None, :, None]
        out = out.masked_fill(~rowv, 0)
    return out


@pytest.mark.parametrize("alpha", [1.5, 2.0])
@pytest.mark.parametrize("causal,varlen", [(False, None), (True, None), (True, [48, 30]), (False, [20, 48])])
def test_backward_vs_autograd(alpha, causal, varlen):
    B, H, L, D = 2, 2, 48, 16
    g = torch.Generator().manual_seed(9)
    q, k, v, do = (torch.randn(B, H, L, D, dtype=torch.float64, generator=g) for _ in range(4))
    q.requires_grad_(), k.requires_grad_(), v.requires_grad_()
    out = _torch_forward(q, k, v, alpha, varlen, causal)
    out.backward(do)
    vl = None if varlen is None else np.array(varlen)
    ref_out = reference_attention(q.detach().numpy(), k.detach().numpy(), v.detach().numpy(), alpha, vl, causal)
    np.testing.assert_allclose(ref_out, out.detach().numpy(), atol=1e-10)
    dq, dk, dv = reference_attention_backward(
        q.detach().numpy(), k.detach().numpy(), v.detach().numpy(), do.numpy(), alpha, vl, causal
    )
    np.testing.assert_allclose(dq, q.grad.numpy(), atol=1e-9)
    np.testing.assert_allclose(dk, k.grad.numpy(), atol=1e-9)
    np.testing.assert_allclose(dv, v.grad.numpy(), atol=1e-9)


def test_backward_finite_differences_general_alpha():
    alpha = 1.333
    B, H, L, D = 1, 1, 12, 8
    q, k, v, do = (_rand((B, H, L, D), s) for s in (10, 11, 12, 13))
    dq, dk, dv = reference_attention_backward(q, k, v, do, alpha, None, True)
    eps = 1e-6

    def loss(qq, kk, vv):
        return (reference_attention(qq, kk, vv, alpha, None, True) * do).sum()

    for arr, grad, which in ((q, dq, 0), (k, dk, 1), (v, dv, 2)):
        for idx in [(0, 0, 3, 1), (0, 0, 7, 5), (0, 0, 11, 0)]:
            args = [q.copy(), k.copy(), v.copy()]
            args[which][idx] += eps
            lp = loss(*args)
            args[which][idx] -= 2 * eps
            lm = loss(*args)
            assert abs((lp - lm) / (2 * eps) - grad[idx]) < 1e-5


def test_block_mask_and_packing():
    B, H, L = 1, 1, 300
    p = np.zeros((B, H, L, L))
    p[0, 0, 5, 70] = 0.3  # tile (0, 1)
    p[0, 0, 200, 299] = 0.1  # tile (1, 4)
    p[0, 0, 290, 0] = 0.2  # tile (2, 0) but row 290 is padding when varlen = 250
    rowv = np.arange(L)[None, :] < 250
    m = block_mask(p, rowv)
    assert m.shape == (1, 1, 3, 5)
    assert set(zip(*np.nonzero(m[0, 0]))) == {(0, 1), (1, 4)}
    w = pack_block_mask(m)
    assert w.shape == (1, 1, 3, 1)
    assert w[0, 0, 0, 0] == 2 and w[0, 0, 1, 0] == 16 and w[0, 0, 2, 0] == 0
