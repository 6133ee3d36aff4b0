"""Lazy attention over a KV cache (Lq < Lk) on the GPU.

The square oracle pins the decode path: query i of batch b sits at position
len_b - Lq + i, so running the oracle on a full-length query tensor that holds these rows at
those positions (anything elsewhere) must give the decode output in those rows.  The layer's
cached decoding is checked against the layer run on the whole sequence at once.
"""
import numpy as np
import pytest
import torch

from _gpu_util import DEV, assert_close, banner, rand, to_np
from oracle.lazy import lazy_forward

pytestmark = pytest.mark.gpu


def _decode_case(H, Hkv, Lq, varlen, D, dtype, tol):
    from adasplash import lazy_attention_triton

    banner("lazy decode", H, Hkv, Lq, varlen, D, dtype)
    B, Lk, W = 2, 777, 100
    G = H // Hkv
    qf = rand((B, H, Lk, D), dtype, 1)
    k = rand((B, Hkv, Lk, D), dtype, 2)
    v = rand((B, Hkv, Lk, D), dtype, 3)
    bias = rand((H, W), torch.float32, 4) * 0.5
    tau = torch.linspace(-1.0, 0.3, H)
    lens = [Lk] * B if varlen is None else varlen
    q = torch.zeros(B, H, Lq, D, dtype=dtype)
    for b in range(B):
        for i in range(Lq):
            p = lens[b] - Lq + i
            if p >= 0:
                q[b, :, i] = qf[b, :, p]
    full = lazy_forward(to_np(qf), np.repeat(to_np(k), G, 1), np.repeat(to_np(v), G, 1), to_np(bias), to_np(tau), W,
                        varlen=varlen)
    ref = np.zeros((B, H, Lq, D))
    for b in range(B):
        for i in range(Lq):
            p = lens[b] - Lq + i
            if p >= 0:
                ref[b, :, i] = full[b, :, p]
    vl = None if varlen is None else torch.tensor(varlen, dtype=torch.int32, device=DEV)
    with torch.no_grad():
        out = lazy_attention_triton(q.to(DEV), k.to(DEV), v.to(DEV), bias.to(DEV), tau.to(DEV), window_size=W, varlen=vl)
    assert out.shape == (B, H, Lq, D)
    assert_close(to_np(out), ref, tol, "decode out")


@pytest.mark.parametrize("H,Hkv", [(4, 4), (8, 2), (6, 1)])
@pytest.mark.parametrize("Lq", [1, 3, 17])
@pytest.mark.parametrize("varlen", [None, [700, 9]])
@pytest.mark.parametrize("D", [32, 64, 128])
def test_decode_vs_square_oracle(H, Hkv, Lq, varlen, D):
    _decode_case(H, Hkv, Lq, varlen, D, torch.float32, 1e-5)


# 16-bit inputs with two or more query rows per K/V head take the matrix-core kernels (rows in
# groups of 32: G * Lq = 102 rows spans four groups, the last one partial).
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("H,Hkv", [(4, 4), (8, 2), (6, 1)])
@pytest.mark.parametrize("Lq", [1, 3, 17])
@pytest.mark.parametrize("varlen", [None, [700, 9]])
@pytest.mark.parametrize("D", [32, 128])
def test_decode_lowp_vs_square_oracle(dtype, H, Hkv, Lq, varlen, D):
    _decode_case(H, Hkv, Lq, varlen, D, dtype, 2e-2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_decode_lowp(dtype):
    from adasplash import lazy_attention_triton

    B, H, Hkv, Lk, D, W = 2, 8, 2, 3000, 64, 512
    q = rand((B, H, 1, D), dtype, 5)
    k = rand((B, Hkv, Lk, D), dtype, 6)
    v = rand((B, Hkv, Lk, D), dtype, 7)
    bias = rand((H, W), torch.float32, 8) * 0.02
    tau = torch.full((H,), -1.0)
    qf = torch.zeros(B, H, Lk, D, dtype=dtype)
    qf[:, :, -1] = q[:, :, 0]
    full = lazy_forward(to_np(qf), np.repeat(to_np(k), 4, 1), np.repeat(to_np(v), 4, 1), to_np(bias), to_np(tau), W)
    out = lazy_attention_triton(q.to(DEV), k.to(DEV), v.to(DEV), bias.to(DEV), tau.to(DEV), window_size=W)
    assert_close(to_np(out), full[:, :, -1:], 1e-2, "decode lowp")


def test_decode_requires_no_grad():
    from adasplash import lazy_attention_triton

    q = torch.zeros(1, 2, 1, 32, device=DEV, requires_grad=True)
    k = torch.zeros(1, 2, 8, 32, device=DEV)
    with pytest.raises(NotImplementedError):
        lazy_attention_triton(q, k, k, torch.zeros(2, 4, device=DEV), torch.zeros(2, device=DEV))


@pytest.mark.parametrize("kv_heads", [4, 2])
def test_layer_cached_decoding_matches_full_sequence(kv_heads):
    from adasplash import LazyAttention

    torch.manual_seed(5)
    B, L, dim, L0 = 2, 150, 128, 100
    m = LazyAttention(dim=dim, num_heads=4, num_kv_heads=kv_heads, window_size=32).to(DEV)
    with torch.no_grad():
        m.attention_biases.normal_(0.0, 0.3)
        m.tau.copy_(torch.tensor([-1.0, -0.5, -0.1, 0.2]))
        x = torch.randn(B, L, dim, device=DEV)
        full = m(x)
        cache = m.new_cache(B, L)
        outs = [m(x[:, :L0], cache=cache)]
        t = L0
        for step in (1, 1, 5, 1, L - L0 - 8):
            outs.append(m(x[:, t:t + step], cache=cache))
            t += step
        got = torch.cat(outs, dim=1)
    assert t == L and cache.len == L
    assert_close(to_np(got), to_np(full), 2e-5, "cached decoding")
