"""LazyAttention layer on the GPU.

Mirrors the reference's tests/test_lazy_attention.py:5-71 (shapes, gradients reach tau and
attention_biases, tau = -100 gives a zero output, RoPE layer runs) on GPU tensors, and checks
the layer against the lazy oracle applied to the layer's own projections (float64).
"""
import numpy as np
import pytest
import torch

from _gpu_util import DEV, assert_close, banner, to_np
from oracle.lazy import lazy_backward, lazy_forward

pytestmark = pytest.mark.gpu


def _mod(**kw):
    from adasplash import LazyAttention

    return LazyAttention(**kw).to(DEV)


def test_forward_shape():
    torch.manual_seed(0)
    m = _mod(dim=32, num_heads=4, window_size=4)
    out = m(torch.randn(2, 16, 32, device=DEV))
    assert out.shape == (2, 16, 32)


def test_backward_reaches_parameters():
    torch.manual_seed(0)
    m = _mod(dim=32, num_heads=4, window_size=4)
    x = torch.randn(2, 16, 32, device=DEV, requires_grad=True)
    m(x).sum().backward()
    assert x.grad is not None and torch.isfinite(x.grad).all()
    assert m.tau.grad is not None and m.attention_biases.grad is not None
    assert m.q_proj.weight.grad is not None and m.k_proj.weight.grad is not None


def test_elastic_softmax_all_zero():
    torch.manual_seed(0)
    m = _mod(dim=16, num_heads=1)
    with torch.no_grad():
        m.tau.fill_(-100.0)
    out = m(torch.randn(1, 10, 16, device=DEV))
    assert torch.allclose(out, torch.zeros_like(out), atol=1e-5)


def test_rope_layer_runs():
    m = _mod(dim=4, num_heads=2)
    out = m(torch.ones(1, 4, 4, device=DEV))
    assert out.shape == (1, 4, 4)


def _layer_qkv(m, x):
    """q, k, v [B, H(kv), L, Dh] of the layer in float64 (projections + RoPE, no kernel)."""
    B, L, _ = x.shape
    with torch.no_grad():
        xd = x.double().cpu()
        q = (xd @ m.q_proj.weight.double().cpu().T).view(B, L, m.num_heads, m.head_dim)
        k = (xd @ m.k_proj.weight.double().cpu().T).view(B, L, m.num_kv_heads, m.head_dim)
        v = (xd @ m.v_proj.weight.double().cpu().T).view(B, L, m.num_kv_heads, m.head_dim)
        D = m.head_dim
        inv = m.rotary.base ** (-np.arange(0, D, 2) / D)
        ang = torch.from_numpy(np.arange(L)[:, None] * inv[None, :])
        cos, sin = ang.cos()[None, :, None, :], ang.sin()[None, :, None, :]

        def rot(t):
            a, b = t.chunk(2, dim=-1)
            return torch.cat((a * cos - b * sin, b * cos + a * sin), dim=-1)

        q, k = rot(q), rot(k)
    return [t.transpose(1, 2).numpy() for t in (q, k, v)]


@pytest.mark.parametrize("heads,kv_heads", [(4, 4), (4, 2)])
@pytest.mark.parametrize("varlen", [None, [90, 200]])
def test_layer_vs_oracle_fp32(heads, kv_heads, varlen):
    banner("lazy module", heads, kv_heads, varlen)
    torch.manual_seed(3)
    B, L, dim, W = 2, 200, 128, 40
    m = _mod(dim=dim, num_heads=heads, num_kv_heads=kv_heads, window_size=W)
    with torch.no_grad():
        m.attention_biases.normal_(0.0, 0.5)
        m.tau.copy_(torch.linspace(-1.0, 0.2, heads))
    x = torch.randn(B, L, dim, device=DEV)
    vl = None if varlen is None else torch.tensor(varlen, device=DEV, dtype=torch.int32)
    out = m(x, varlen=vl)
    out.sum().backward()

    q, k, v = _layer_qkv(m, x)
    G = heads // kv_heads
    k, v = np.repeat(k, G, axis=1), np.repeat(v, G, axis=1)
    bias, tau = to_np(m.attention_biases), to_np(m.tau)
    o = lazy_forward(q, k, v, bias, tau, W, varlen=varlen)  # [B, H, L, Dh]
    wo = m.o_proj.weight.double().detach().cpu().numpy()
    ref = o.transpose(0, 2, 1, 3).reshape(B, L, dim) @ wo.T
    assert_close(to_np(out), ref, 1e-4, "layer out")
    # loss = out.sum(): d(attention output) = column sums of W_o, the same for every token
    do = np.broadcast_to(wo.sum(axis=0).reshape(heads, m.head_dim)[None, :, None, :], q.shape).copy()
    _dq, _dk, _dv, dbias, dtau = lazy_backward(q, k, v, bias, tau, do, W, varlen=varlen)
    assert_close(to_np(m.attention_biases.grad), dbias, 1e-4 * max(1.0, np.abs(dbias).max()), "dbias")
    assert_close(to_np(m.tau.grad), dtau, 1e-4 * max(1.0, np.abs(dtau).max()), "dtau")


def test_layer_bf16_runs_and_keeps_fp32_params():
    torch.manual_seed(0)
    m = _mod(dim=256, num_heads=4, window_size=64)
    for lin in (m.q_proj, m.k_proj, m.v_proj, m.o_proj):
        lin.to(torch.bfloat16)
    x = torch.randn(2, 300, 256, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    out = m(x)
    out.float().sum().backward()
    assert out.dtype == torch.bfloat16 and torch.isfinite(out.float()).all()
    assert m.tau.grad.dtype == torch.float32 and m.attention_biases.grad.dtype == torch.float32
