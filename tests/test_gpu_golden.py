"""HIP kernels vs the committed golden fixtures (fp32 inputs)."""
import os

import numpy as np
import pytest
import torch

from _gpu_util import DEV, assert_close

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _load(name):
    return dict(np.load(os.path.join(GOLD, name + ".npz"), allow_pickle=False))


def _t(x, grad=False):
    t = torch.from_numpy(np.ascontiguousarray(x)).to(DEV)
    return t.requires_grad_(True) if grad else t


@pytest.mark.parametrize("a", [1.25, 1.5, 2.0])
def test_entmax(a):
    from adasplash import triton_entmax

    d = _load(f"entmax_a{a}")
    x = _t(d["x"], True)
    y = triton_entmax(x, alpha=a)
    y.backward(_t(d["dy"]))
    assert_close(y.detach().cpu().numpy(), d["y"], 2e-6, "y")
    assert_close(x.grad.cpu().numpy(), d["dx"], 2e-5, "dx")


@pytest.mark.parametrize("a", [1.5, 2.0])
@pytest.mark.parametrize("c", [0, 1])
def test_adasplash(a, c):
    from adasplash import adasplash, adasplash_stats

    d = _load(f"ada_a{a}_c{c}")
    q, k, v = (_t(d[n], True) for n in "qkv")
    vl = _t(d["varlen"])
    out = adasplash(q, k, v, alpha=a, is_causal=bool(c), varlen=vl)
    out.backward(_t(d["do"]))
    assert_close(out.detach().cpu().numpy(), d["out"], 1e-4, "out")
    for t, n in zip((q, k, v), ("dq", "dk", "dv")):
        assert_close(t.grad.cpu().numpy(), d[n], 2e-4, n)
    _o, tau, mask = adasplash_stats(q.detach(), k.detach(), v.detach(), alpha=a, is_causal=bool(c), varlen=vl)
    assert (mask.cpu().numpy() == d["mask"]).all()
    tr = d["tau"]
    ok = np.isfinite(tau.cpu().numpy())
    assert_close(tau.cpu().numpy()[ok] / (1 + np.abs(tr[ok])), tr[ok] / (1 + np.abs(tr[ok])), 1e-6, "tau")


@pytest.mark.parametrize("name", ["lazy_full", "lazy_varlen"])
def test_lazy(name):
    from adasplash import lazy_attention_triton

    d = _load(name)
    ts = [_t(d[n], True) for n in ("q", "k", "v", "bias", "tau")]
    vl = _t(d["varlen"]) if "varlen" in d else None
    out = lazy_attention_triton(*ts, window_size=int(d["window"]), varlen=vl)
    out.backward(_t(d["do"]))
    assert_close(out.detach().cpu().numpy(), d["out"], 1e-5, "out")
    for t, n in zip(ts, ("dq", "dk", "dv", "dbias", "dtau")):
        assert_close(t.grad.cpu().numpy(), d[n], 2e-4 * max(1.0, np.abs(d[n]).max()), n)
