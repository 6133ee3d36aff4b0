"""Pins the Lazy-Attention oracle.

Checks: torch float64 autograd through a restatement of compare_scratch_flash.py:45-71
(the reference's vectorised scratch implementation, with the kernel's 0 <= d < W bias
window, lazy_attention_triton.py:62), tau = 0 reducing to causal softmax attention with
bias, tau = -100 giving zero output (tests/test_lazy_attention.py:28-52), varlen zero rows.
Block mask: the attention weights agree with the torch restatement, tau = -100 gives an
empty mask, tau > 0 gives exactly the causally visible blocks of the valid rows/keys (every
visible weight is then > 0), and the output recomputed from the masked blocks alone is the
full output (no non-zero weight lies outside the mask).
"""
import math

import numpy as np
import pytest
import torch

from oracle.lazy import lazy_backward, lazy_block_mask, lazy_forward, lazy_weights


def _torch_lazy(q, k, v, bias, tau, W, varlen=None):
    B, H, L, D = q.shape
    s = q @ k.transpose(-1, -2) * D ** -0.5
    rel = torch.arange(L)[:, None] - torch.arange(L)[None, :]
    valid = (0 <= rel) & (rel < W)
    idx = rel.clamp(0, bias.shape[1] - 1)
    s = s + bias[:, idx] * valid
    causal = torch.tril(torch.ones(L, L, dtype=torch.bool))
    keep = causal[None, None].expand(B, H, L, L).clone()
    if varlen is not None:
        keep &= (torch.arange(L)[None, :] < torch.as_tensor(varlen)[:, None])[:, None, None, :]
    s = s.masked_fill(~keep, float("-inf"))
    w = torch.softmax(s, -1)
    i = torch.arange(1, L + 1, dtype=q.dtype).view(1, 1, -1, 1)
    w = torch.relu(w + tau.view(1, H, 1, 1) / i)
    w = w.masked_fill(~keep, 0)
    out = w @ v
    if varlen is not None:
        rowv = (torch.arange(L)[None, :] < torch.as_tensor(varlen)[:, None])[:, None, :, None]
        out = out.masked_fill(~rowv, 0)
    return out


@pytest.mark.parametrize("tauval", [-1.0, -0.3, 0.5])
@pytest.mark.parametrize("varlen", [None, [32, 21]])
def test_forward_backward_vs_autograd(tauval, varlen):
    B, H, L, D, W = 2, 2, 32, 16, 8
    g = torch.Generator().manual_seed(0)
    q, k, v, do = (torch.randn(B, H, L, D, dtype=torch.float64, generator=g) for _ in range(4))
    bias = torch.randn(H, W, dtype=torch.float64, generator=g)
    tau = torch.full((H,), tauval, dtype=torch.float64)
    tau[1] = tauval * 0.5
    ts = [q, k, v, bias, tau]
    for t in ts:
        t.requires_grad_()
    out = _torch_lazy(q, k, v, bias, tau, W, varlen)
    out.backward(do)
    n = lambda t: t.detach().numpy()
    vl = None if varlen is None else np.array(varlen)
    o = lazy_forward(n(q), n(k), n(v), n(bias), n(tau), W, vl)
    np.testing.assert_allclose(o, n(out), atol=1e-11)
    grads = lazy_backward(n(q), n(k), n(v), n(bias), n(tau), n(do), W, vl)
    for ours, t in zip(grads, ts):
        np.testing.assert_allclose(ours, t.grad.numpy(), atol=1e-9)


def test_tau_zero_is_softmax_attention():
    B, H, L, D, W = 1, 2, 24, 8, 6
    rng = np.random.default_rng(1)
    q, k, v = (rng.standard_normal((B, H, L, D)) for _ in range(3))
    bias = rng.standard_normal((H, W))
    out = lazy_forward(q, k, v, bias, np.zeros(H), W)
    tq, tk, tv = (torch.from_numpy(x) for x in (q, k, v))
    mask = torch.zeros(L, L, dtype=torch.float64)
    for i in range(L):
        for j in range(L):
            if j > i:
                mask[i, j] = float("-inf")
            elif i - j < W:
                mask[:, :][i, j] = 0.0
    bm = torch.zeros(H, L, L, dtype=torch.float64)
    for h in range(H):
        for i in range(L):
            for j in range(max(0, i - W + 1), i + 1):
                bm[h, i, j] = bias[h, i - j]
    ref = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, attn_mask=(mask + bm)[None])
    np.testing.assert_allclose(out, ref.numpy(), atol=1e-12)


def test_tau_very_negative_gives_zero():
    rng = np.random.default_rng(2)
    q, k, v = (rng.standard_normal((1, 1, 10, 8)) for _ in range(3))
    out = lazy_forward(q, k, v, np.zeros((1, 4)), np.array([-100.0]), 4)
    assert np.abs(out).max() < 1e-12


def _torch_weights(q, k, bias, tau, W, varlen=None):
    B, H, L, D = q.shape
    s = q @ k.transpose(-1, -2) * D ** -0.5
    rel = torch.arange(L)[:, None] - torch.arange(L)[None, :]
    s = s + bias[:, rel.clamp(0, bias.shape[1] - 1)] * ((0 <= rel) & (rel < W))
    keep = torch.tril(torch.ones(L, L, dtype=torch.bool))[None, None].expand(B, H, L, L).clone()
    rowv = torch.ones(B, 1, L, 1, dtype=torch.bool)
    if varlen is not None:
        ar = torch.arange(L)
        keep &= (ar[None, :] < torch.as_tensor(varlen)[:, None])[:, None, None, :]
        rowv = (ar[None, :] < torch.as_tensor(varlen)[:, None])[:, None, :, None]
    w = torch.softmax(s.masked_fill(~keep, float("-inf")), -1)
    w = torch.relu(w + tau.view(1, H, 1, 1) / torch.arange(1, L + 1, dtype=q.dtype).view(1, 1, -1, 1))
    return w.masked_fill(~keep, 0).masked_fill(~rowv, 0)


@pytest.mark.parametrize("varlen", [None, [70, 130]])
def test_block_mask_properties(varlen):
    rng = np.random.default_rng(7)
    B, H, L, D, W = 2, 3, 130, 16, 20
    q, k, v = (rng.standard_normal((B, H, L, D)) for _ in range(3))
    bias = rng.standard_normal((H, W)) * 0.3
    tau = np.array([-1.0, -0.05, 0.4])
    e, margin = lazy_weights(q, k, bias, tau, W, varlen)
    ref_w = _torch_weights(*(torch.from_numpy(x) for x in (q, k, bias, tau)), W, varlen).numpy()
    assert np.abs(e - ref_w).max() < 1e-12
    m = lazy_block_mask(e)
    assert m.shape == (B, H, 3, 3)
    # output from the masked blocks alone equals the full output
    bm = np.repeat(np.repeat(m, 64, axis=2), 64, axis=3)[:, :, :L, :L]
    out = lazy_forward(q, k, v, bias, tau, W, varlen)
    assert np.abs(np.where(bm, e, 0.0) @ v - out).max() < 1e-12
    # tau > 0: every visible (row < len, key <= row, key < len) block is set
    n = [L, L] if varlen is None else varlen
    for b in range(B):
        vis = np.zeros((3, 3), dtype=bool)
        for r in range(3):
            for c in range(3):
                vis[r, c] = 64 * r < n[b] and 64 * c < n[b] and c <= r
        assert (m[b, 2] == vis).all()
    # tau = -100: nothing survives
    e0, _ = lazy_weights(q, k, bias, np.full(H, -100.0), W, varlen)
    assert not lazy_block_mask(e0).any()
    assert np.isfinite(margin[e > 0]).all()
