"""Edge lengths on the GPU: sequences of length 0 and 1 next to a ragged one, in one batch.

The reference pads with zeros past each length (tests/test_adasplash.py:161-174,
tests/test_lazy_attention_varlen.py:13-134): rows at or past varlen[b] give zero output and
zero gradients, and a sequence of length 0 contributes nothing.  The oracle covers the valid
rows (float64); the zeros are checked exactly.
"""
import numpy as np
import pytest
import torch

from _gpu_util import DEV, assert_close, banner, rand, to_np
from oracle.adasplash import reference_attention, reference_attention_backward
from oracle.lazy import lazy_backward, lazy_forward

pytestmark = pytest.mark.gpu

LENS = [0, 1, 137]


def _zero_past(t, lens):
    for b, n in enumerate(lens):
        assert (t[b, :, n:] == 0).all(), f"nonzero past length {n} in batch {b}"


@pytest.mark.parametrize("is_causal", [True, False])
@pytest.mark.parametrize("alpha", [1.5, 2.0])
def test_adasplash_lengths_0_1(is_causal, alpha):
    from adasplash import adasplash

    banner("ada edge", is_causal, alpha)
    B, H, L, D = 3, 2, 200, 32
    q, k, v, do = (rand((B, H, L, D), torch.float32, 60 + i) for i in range(4))
    vl = torch.tensor(LENS, device=DEV)
    ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v)]
    out = adasplash(*ts, alpha=alpha, is_causal=is_causal, varlen=vl)
    out.backward(do.to(DEV))
    ref = reference_attention(to_np(q), to_np(k), to_np(v), alpha, varlen=LENS, is_causal=is_causal)
    rq, rk, rv = reference_attention_backward(to_np(q), to_np(k), to_np(v), to_np(do), alpha, varlen=LENS,
                                              is_causal=is_causal)
    _zero_past(out.detach(), LENS)
    assert_close(to_np(out), ref, 1e-4, "out")
    for t, r, n in zip(ts, (rq, rk, rv), ("dq", "dk", "dv")):
        _zero_past(t.grad, LENS)
        assert_close(to_np(t.grad), r, 1e-4 * max(1.0, np.abs(r).max()), n)


def test_lazy_lengths_0_1():
    from adasplash import lazy_attention_triton

    banner("lazy edge")
    B, H, L, D, W = 3, 2, 200, 32, 16
    q, k, v, do = (rand((B, H, L, D), torch.float32, 70 + i) for i in range(4))
    bias = rand((H, W), torch.float32, 74)
    tau = torch.tensor([-1.0, 0.2])
    vl = torch.tensor(LENS, dtype=torch.int32, device=DEV)
    ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v, bias, tau)]
    out = lazy_attention_triton(*ts, window_size=W, varlen=vl)
    out.backward(do.to(DEV))
    ref = lazy_forward(to_np(q), to_np(k), to_np(v), to_np(bias), to_np(tau), W, varlen=LENS)
    refs = lazy_backward(to_np(q), to_np(k), to_np(v), to_np(bias), to_np(tau), to_np(do), W, varlen=LENS)
    _zero_past(out.detach(), LENS)
    assert_close(to_np(out), ref, 1e-5, "out")
    for t, r, n in zip(ts, refs, ("dq", "dk", "dv", "dbias", "dtau")):
        if n in ("dq", "dk", "dv"):
            _zero_past(t.grad, LENS)
        assert_close(to_np(t.grad), r, 1e-4 * max(1.0, np.abs(r).max()), n)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decode_lengths_0_1(dtype):
    from adasplash import lazy_attention_triton

    banner("decode edge", dtype)
    B, H, Hkv, Lq, Lk, D, W = 3, 4, 2, 2, 300, 64, 40
    G = H // Hkv
    lens = [0, 1, 137]
    qf = rand((B, H, Lk, D), dtype, 80)
    k, v = rand((B, Hkv, Lk, D), dtype, 81), rand((B, Hkv, Lk, D), dtype, 82)
    bias = rand((H, W), torch.float32, 83) * 0.5
    tau = torch.linspace(-1.0, 0.3, H)
    q = torch.zeros(B, H, Lq, D, dtype=dtype)
    for b in range(B):
        for i in range(Lq):
            p = lens[b] - Lq + i
            if p >= 0:
                q[b, :, i] = qf[b, :, p]
    full = lazy_forward(to_np(qf), np.repeat(to_np(k), G, 1), np.repeat(to_np(v), G, 1), to_np(bias), to_np(tau), W,
                        varlen=lens)
    ref = np.zeros((B, H, Lq, D))
    for b in range(B):
        for i in range(Lq):
            p = lens[b] - Lq + i
            if p >= 0:
                ref[b, :, i] = full[b, :, p]
    vl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    with torch.no_grad():
        out = lazy_attention_triton(q.to(DEV), k.to(DEV), v.to(DEV), bias.to(DEV), tau.to(DEV), window_size=W,
                                    varlen=vl)
    # positions < 0 (length 0; the first query row of length 1) are zero rows
    assert (out[0] == 0).all() and (out[1, :, 0] == 0).all()
    assert_close(to_np(out), ref, 1e-5 if dtype == torch.float32 else 2e-2, "decode out")
