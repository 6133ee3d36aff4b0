"""triton_entmax on the GPU vs the oracle (mirrors tests/test_triton_entmax.py)."""
import numpy as np
import pytest
import torch

from _gpu_util import DEV, assert_close, banner, rand, to_np
from oracle.entmax import entmax_backward, entmax_bisect

pytestmark = pytest.mark.gpu


def _ent():
    from adasplash import triton_entmax

    return triton_entmax


@pytest.mark.parametrize("shape", [(2,), (2, 4), (2, 4, 8), (2, 4, 8, 16), (128, 256), (3, 1000), (5, 3000)])
@pytest.mark.parametrize("alpha", [1.1, 1.333, 1.5, 1.666, 2.0])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32, torch.bfloat16])
@pytest.mark.parametrize("fast_math", [False, True])
def test_forward(shape, alpha, dtype, fast_math):
    banner("entmax fwd", shape, alpha, dtype, fast_math)
    x = rand(shape, dtype, 42)
    ref = entmax_bisect(to_np(x), alpha, n_iter=60)
    y = _ent()(x.to(DEV), alpha=alpha, fast_math=fast_math)
    assert y.dtype == dtype and y.shape == x.shape
    atol = {torch.float32: 2e-6, torch.float16: 1e-3, torch.bfloat16: 8e-3}[dtype]
    assert_close(to_np(y), ref, atol, "entmax forward")


@pytest.mark.parametrize("shape", [(2,), (2, 4), (2, 4, 8), (6, 300)])
@pytest.mark.parametrize("alpha", [1.1, 1.333, 1.5, 1.666, 2.0])
def test_backward_vs_oracle(shape, alpha):
    banner("entmax bwd", shape, alpha)
    x = rand(shape, torch.float32, 1).to(DEV).requires_grad_(True)
    dy = rand(shape, torch.float32, 2)
    y = _ent()(x, alpha, 10, True)
    y.backward(dy.to(DEV))
    ref = entmax_backward(entmax_bisect(to_np(x), alpha, n_iter=60), to_np(dy), alpha)
    assert_close(to_np(x.grad), ref, 2e-5, "entmax backward")


@pytest.mark.parametrize("alpha", [1.1, 1.333, 1.5, 1.666, 2.0])
def test_gradcheck(alpha):
    # tests/test_triton_entmax.py:33-41
    x = rand((2, 4, 8), torch.float32, 42).to(DEV).requires_grad_(True)
    assert torch.autograd.gradcheck(lambda t: _ent()(t, alpha, 10, True), x, atol=1e-2, eps=1e-4, rtol=1e-2)


@pytest.mark.parametrize("alpha", [1.1, 1.333, 1.5, 1.666, 2.0])
def test_numerical_stability(alpha):
    for shape in [(2,), (2, 5), (2, 4, 8)]:
        x = (rand(shape, torch.float32, 3) * 100).to(DEV).requires_grad_(True)
        y = _ent()(x, alpha=alpha)
        assert torch.isfinite(y).all() and (y >= 0).all()
        assert torch.allclose(y.sum(-1), torch.ones(y.shape[:-1], device=DEV), atol=1e-2)
        y.sum().backward()
        assert not torch.isnan(x.grad).any()


@pytest.mark.parametrize("alpha", [1.333, 1.5, 1.666, 2.0])
def test_edge_cases(alpha):
    e = _ent()
    y = e(torch.zeros(64, device=DEV), alpha=alpha)
    assert torch.allclose(y, torch.full_like(y, 1 / 64), atol=1e-6)
    y = e(torch.full((64,), 1e3, device=DEV), alpha=alpha)
    assert torch.allclose(y, torch.full_like(y, 1 / 64), atol=1e-6)
    x = torch.zeros(64, device=DEV)
    x[0] = 100
    y = e(x, alpha=alpha)
    assert torch.allclose(y, torch.eye(64, device=DEV)[0], atol=1e-6)


@pytest.mark.parametrize("dim", [0, 1, 2])
def test_different_dimensions(dim):
    x = rand((32, 32, 32), torch.float32, 5)
    ref = entmax_bisect(to_np(x), 1.5, axis=dim, n_iter=60)
    xd = x.to(DEV)
    perm = {0: (1, 2, 0), 1: (0, 2, 1), 2: (0, 1, 2)}[dim]
    inv = np.argsort(perm)
    y = _ent()(xd.permute(perm).contiguous(), alpha=1.5).permute(*inv)
    assert_close(to_np(y), ref, 1e-5, "entmax dim")


def test_repeat_bit_identical():
    x = rand((64, 777), torch.float32, 6).to(DEV)
    y1 = _ent()(x, fast_math=True)
    y2 = _ent()(x, fast_math=True)
    assert torch.equal(y1, y2)


def test_masked_entries():
    x = rand((4, 100), torch.float32, 7)
    x[:, 60:] = float("-inf")
    y = _ent()(x.to(DEV), alpha=1.5)
    assert (y[:, 60:] == 0).all()
    assert_close(to_np(y), entmax_bisect(to_np(x), 1.5, n_iter=60), 2e-6, "masked")
