"""Grouped-query attention (H query heads over H_kv key/value heads) on the GPU.

The reference reaches GQA by expanding K and V with ``repeat_interleave`` over the head dim
before calling the op (examples/sw_attention_lazy.py:154-157); the kernels here read K/V head
h // (H / H_kv) in place.  The oracle is therefore the ordinary oracle on the expanded K/V,
with dK / dV summed over each group of query heads (the adjoint of the expansion).
"""
import numpy as np
import pytest
import torch

from _gpu_util import DEV, assert_close, banner, rand, to_np
from oracle.adasplash import reference_attention, reference_attention_backward
from oracle.lazy import lazy_backward, lazy_forward

pytestmark = pytest.mark.gpu


def _expand(x, G):
    return np.repeat(x, G, axis=1)


def _fold(dx, G):
    B, H, L, D = dx.shape
    return dx.reshape(B, H // G, G, L, D).sum(axis=2)


@pytest.mark.parametrize("H,Hkv", [(4, 2), (6, 1), (4, 4)])
@pytest.mark.parametrize("is_causal", [True, False])
@pytest.mark.parametrize("alpha", [1.5, 2.0])
@pytest.mark.parametrize("varlen", [None, [200, 77]])
def test_adasplash_gqa_fp32(H, Hkv, is_causal, alpha, varlen):
    from adasplash import adasplash, adasplash_stats

    B, L, D = 2, 256, 64
    G = H // Hkv
    banner("ada gqa", H, Hkv, is_causal, alpha, varlen)
    q = rand((B, H, L, D), torch.float32, 1)
    k = rand((B, Hkv, L, D), torch.float32, 2)
    v = rand((B, Hkv, L, D), torch.float32, 3)
    do = rand((B, H, L, D), torch.float32, 4)
    qn, kn, vn = to_np(q), _expand(to_np(k), G), _expand(to_np(v), G)
    ref = reference_attention(qn, kn, vn, alpha, varlen=varlen, is_causal=is_causal)
    rq, rk, rv = reference_attention_backward(qn, kn, vn, to_np(do), alpha, varlen=varlen, is_causal=is_causal)
    vl = None if varlen is None else torch.tensor(varlen, device=DEV)
    ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v)]
    out = adasplash(*ts, alpha=alpha, is_causal=is_causal, varlen=vl)
    assert_close(to_np(out), ref, 1e-4, "out")
    out.backward(do.to(DEV))
    assert_close(to_np(ts[0].grad), rq, 1e-4 * max(1.0, np.abs(rq).max()), "dq")
    assert_close(to_np(ts[1].grad), _fold(rk, G), 1e-4 * max(1.0, np.abs(rk).max()), "dk")
    assert_close(to_np(ts[2].grad), _fold(rv, G), 1e-4 * max(1.0, np.abs(rv).max()), "dv")
    # Block mask of the grouped call equals the one of the expanded call (same kernels, same scores).
    _o, _t, m_gqa = adasplash_stats(q.to(DEV), k.to(DEV), v.to(DEV), alpha=alpha, is_causal=is_causal, varlen=vl)
    _o, _t, m_exp = adasplash_stats(q.to(DEV), torch.from_numpy(kn).float().to(DEV),
                                    torch.from_numpy(vn).float().to(DEV), alpha=alpha, is_causal=is_causal, varlen=vl)
    assert torch.equal(m_gqa, m_exp)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_adasplash_gqa_lowp(dtype):
    from adasplash import adasplash

    B, H, Hkv, L, D = 1, 8, 2, 384, 64
    G = H // Hkv
    banner("ada gqa lowp", dtype)
    q = rand((B, H, L, D), dtype, 11)
    k = rand((B, Hkv, L, D), dtype, 12)
    v = rand((B, Hkv, L, D), dtype, 13)
    do = rand((B, H, L, D), dtype, 14)
    qn, kn, vn = to_np(q), _expand(to_np(k), G), _expand(to_np(v), G)
    ref = reference_attention(qn, kn, vn, 1.5, is_causal=True)
    rq, rk, rv = reference_attention_backward(qn, kn, vn, to_np(do), 1.5, is_causal=True)
    ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v)]
    out = adasplash(*ts, alpha=1.5, is_causal=True)
    assert_close(to_np(out), ref, 2e-2, "out")
    out.backward(do.to(DEV))
    # Gradients are sums over L = 384 rows (and over G heads for dk / dv): relative bound.
    assert_close(to_np(ts[0].grad), rq, 2e-2 * max(1.0, np.abs(rq).max()), "dq")
    assert_close(to_np(ts[1].grad), _fold(rk, G), 2e-2 * max(1.0, np.abs(_fold(rk, G)).max()), "dk")
    assert_close(to_np(ts[2].grad), _fold(rv, G), 2e-2 * max(1.0, np.abs(_fold(rv, G)).max()), "dv")


@pytest.mark.parametrize("H,Hkv", [(4, 2), (6, 3), (3, 1)])
@pytest.mark.parametrize("varlen", [None, [150, 300]])
def test_lazy_gqa_fp32(H, Hkv, varlen):
    from adasplash import lazy_attention_triton

    B, L, D, W = 2, 300, 32, 48
    G = H // Hkv
    banner("lazy gqa", H, Hkv, varlen)
    q = rand((B, H, L, D), torch.float32, 21)
    k = rand((B, Hkv, L, D), torch.float32, 22)
    v = rand((B, Hkv, L, D), torch.float32, 23)
    bias = rand((H, W + 2), torch.float32, 24)
    tau = torch.linspace(-1.0, 0.3, H)
    do = rand((B, H, L, D), torch.float32, 25)
    qn, kn, vn = to_np(q), _expand(to_np(k), G), _expand(to_np(v), G)
    ref = lazy_forward(qn, kn, vn, to_np(bias), to_np(tau), W, varlen=varlen)
    rq, rk, rv, rb, rt = lazy_backward(qn, kn, vn, to_np(bias), to_np(tau), to_np(do), W, varlen=varlen)
    vl = None if varlen is None else torch.tensor(varlen, device=DEV, dtype=torch.int32)
    ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v, bias, tau)]
    out = lazy_attention_triton(*ts, window_size=W, varlen=vl)
    assert_close(to_np(out), ref, 1e-5, "out")
    out.backward(do.to(DEV))
    refs = [rq, _fold(rk, G), _fold(rv, G), rb, rt]
    for t, r, n in zip(ts, refs, ("dq", "dk", "dv", "dbias", "dtau")):
        assert_close(to_np(t.grad), r, 1e-4 * max(1.0, np.abs(r).max()), n)


def test_gqa_shape_errors():
    from adasplash import adasplash, lazy_attention_triton

    q = torch.zeros(1, 4, 64, 32, device=DEV)
    k = torch.zeros(1, 3, 64, 32, device=DEV)
    with pytest.raises(ValueError):
        adasplash(q, k, k)
    with pytest.raises(ValueError):
        lazy_attention_triton(q, k, k, torch.zeros(4, 8, device=DEV), torch.zeros(4, device=DEV))
