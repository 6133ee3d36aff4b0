"""Pins the entmax oracle against independent algorithms and known answers.

Nothing here retypes the oracle's formula: bisection is checked against sort-based
closed forms, brute-force support enumeration, the softmax limit and the known
answers of the reference's tests (tests/test_triton_entmax.py:66-85); the backward
is checked against finite differences and torch autograd through the closed forms.
"""
import numpy as np
import pytest
import torch

from oracle.entmax import (
    entmax15_sort,
    entmax_backward,
    entmax_bisect,
    entmax_support_brute,
    entmax_threshold,
    softmax,
    sparsemax_sort,
)


@pytest.mark.parametrize("shape", [(2,), (2, 4), (2, 4, 8), (2, 4, 8, 16), (7, 300)])
def test_bisect_matches_closed_forms(shape):
    rng = np.random.default_rng(0)
    x = rng.standard_normal(shape)
    np.testing.assert_allclose(entmax_bisect(x, 2.0), sparsemax_sort(x), atol=1e-12)
    np.testing.assert_allclose(entmax_bisect(x, 1.5), entmax15_sort(x), atol=1e-12)


@pytest.mark.parametrize("alpha", [1.1, 1.333, 1.5, 1.666, 2.0])
def test_bisect_matches_brute_force(alpha):
    rng = np.random.default_rng(1)
    for _ in range(20):
        x = rng.standard_normal(6) * 2
        np.testing.assert_allclose(entmax_bisect(x, alpha), entmax_support_brute(x, alpha), atol=1e-9)


def test_softmax_limit():
    x = np.random.default_rng(2).standard_normal((4, 9))
    np.testing.assert_allclose(entmax_bisect(x, 1.0 + 1e-4, n_iter=80), softmax(x), atol=2e-4)


@pytest.mark.parametrize("alpha", [1.333, 1.5, 1.666, 2.0])
def test_known_answers(alpha):
    # tests/test_triton_entmax.py:66-85
    y = entmax_bisect(np.zeros(64), alpha)
    np.testing.assert_allclose(y, np.full(64, 1 / 64), atol=1e-12)
    y = entmax_bisect(np.full(64, 1e3), alpha)
    np.testing.assert_allclose(y, np.full(64, 1 / 64), atol=1e-9)
    x = np.zeros(64)
    x[0] = 100
    np.testing.assert_allclose(entmax_bisect(x, alpha), np.eye(64)[0], atol=1e-12)


def test_invariants_and_masking():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 40)) * 3
    for a in (1.2, 1.5, 2.0):
        y = entmax_bisect(x, a)
        assert (y >= 0).all()
        np.testing.assert_allclose(y.sum(-1), 1, atol=1e-12)
        np.testing.assert_allclose(entmax_bisect(x + 7.5, a), y, atol=1e-10)
        perm = rng.permutation(40)
        np.testing.assert_allclose(entmax_bisect(x[:, perm], a), y[:, perm], atol=1e-10)
    # -inf entries get exactly zero probability and leave the rest as entmax of the finite part
    xm = x.copy()
    xm[:, 30:] = -np.inf
    ym = entmax_bisect(xm, 1.5, n_iter=60)
    assert (ym[:, 30:] == 0).all()
    np.testing.assert_allclose(ym[:, :30], entmax15_sort(x[:, :30]), atol=1e-12)


def test_threshold_is_root():
    x = np.random.default_rng(4).standard_normal((3, 50))
    for a in (1.25, 1.5, 2.0):
        tau = entmax_threshold(x, a)
        f = (np.maximum((a - 1) * x - tau, 0) ** (1 / (a - 1))).sum(-1)
        np.testing.assert_allclose(f, 1, atol=1e-12)


@pytest.mark.parametrize("alpha", [1.1, 1.333, 1.5, 1.666, 2.0])
def test_backward_finite_differences(alpha):
    rng = np.random.default_rng(5)
    x = rng.standard_normal(12)
    dy = rng.standard_normal(12)
    y = entmax_bisect(x, alpha, n_iter=80)
    g = entmax_backward(y, dy, alpha)
    eps = 1e-6
    fd = np.zeros(12)
    for i in range(12):
        e = np.zeros(12)
        e[i] = eps
        fd[i] = (entmax_bisect(x + e, alpha, n_iter=80) @ dy - entmax_bisect(x - e, alpha, n_iter=80) @ dy) / (2 * eps)
    np.testing.assert_allclose(g, fd, atol=1e-6)


def _torch_entmax15(x):
    z = x / 2
    zs, _ = torch.sort(z, dim=-1, descending=True)
    k = torch.arange(1, x.shape[-1] + 1, dtype=x.dtype)
    mean = zs.cumsum(-1) / k
    msq = (zs * zs).cumsum(-1) / k
    delta = torch.clamp((1 - k * (msq - mean * mean)) / k, min=0)
    tau = mean - torch.sqrt(delta)
    ks = (tau <= zs).sum(-1, keepdim=True)
    ts = tau.gather(-1, ks - 1)
    return torch.clamp(z - ts, min=0) ** 2


def _torch_sparsemax(x):
    zs, _ = torch.sort(x, dim=-1, descending=True)
    k = torch.arange(1, x.shape[-1] + 1, dtype=x.dtype)
    cs = zs.cumsum(-1)
    ks = (1 + k * zs > cs).sum(-1, keepdim=True)
    tau = (cs.gather(-1, ks - 1) - 1) / ks
    return torch.clamp(x - tau, min=0)


@pytest.mark.parametrize("alpha,fn", [(1.5, _torch_entmax15), (2.0, _torch_sparsemax)])
def test_backward_vs_autograd(alpha, fn):
    g = torch.Generator().manual_seed(6)
    x = torch.randn(6, 33, dtype=torch.float64, generator=g, requires_grad=True)
    dy = torch.randn(6, 33, dtype=torch.float64, generator=g)
    y = fn(x)
    y.backward(dy)
    ours = entmax_backward(y.detach().numpy(), dy.numpy(), alpha)
    np.testing.assert_allclose(ours, x.grad.numpy(), atol=1e-10)
