"""LazyAttention host-side pieces that need no GPU: the rotary embedding and input checks.

RoPE is pinned by properties that fix it independently of its formula: it is a rotation
(norms preserved), scores depend only on the position difference, position 0 is the
identity, and the pair (x_i, x_{i+D/2}) turns by pos * base^(-2i/D) (checked on a one-hot
vector against cos/sin of that angle).
"""
import math

import pytest
import torch

from adasplash.lazy_attention import LazyAttention, RotaryEmbedding


def test_rope_is_a_rotation_and_relative():
    torch.manual_seed(0)
    D, L = 16, 12
    rope = RotaryEmbedding(D, base=10000.0)
    q = torch.randn(1, L, 2, D, dtype=torch.float64)
    k = torch.randn(1, L, 2, D, dtype=torch.float64)
    rq, rk = rope(q.float(), k.float())
    assert torch.allclose(rq.norm(dim=-1), q.float().norm(dim=-1), atol=1e-5)
    assert torch.allclose(rq[:, 0], q[:, 0].float(), atol=1e-6)  # position 0: identity
    # the same q and k placed at positions (m, n) give scores depending on m - n only
    qq = q[:, :1].expand(1, L, 2, D).float()
    kk = k[:, :1].expand(1, L, 2, D).float()
    a, b = rope(qq, kk)
    s = torch.einsum("bmhd,bnhd->bhmn", a, b)
    for m in range(1, L):
        assert torch.allclose(s[..., m, 1:], s[..., m - 1, :-1], atol=1e-4)


def test_rope_angle_on_one_hot():
    D, base = 8, 500.0
    rope = RotaryEmbedding(D, base=base)
    x = torch.zeros(1, 5, 1, D)
    x[..., 1] = 1.0  # pair (x_1, x_5), frequency base^(-2/8)
    r, _ = rope(x, x)
    for pos in range(5):
        ang = pos * base ** (-2.0 / D)
        assert abs(r[0, pos, 0, 1].item() - math.cos(ang)) < 1e-6
        assert abs(r[0, pos, 0, 5].item() - math.sin(ang)) < 1e-6


def test_module_parameters_and_cpu_input_raises():
    m = LazyAttention(dim=32, num_heads=4, window_size=4)
    assert m.tau.shape == (4,) and m.tau.dtype == torch.float32 and torch.all(m.tau == -1.0)
    assert m.attention_biases.shape == (4, 4) and m.attention_biases.dtype == torch.float32
    with pytest.raises(ValueError, match="GPU"):
        m(torch.randn(2, 16, 32))
    with pytest.raises(ValueError):
        LazyAttention(dim=30, num_heads=4)
    with pytest.raises(ValueError):
        LazyAttention(dim=32, num_heads=4, num_kv_heads=3)
