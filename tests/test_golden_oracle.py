"""The oracle reproduces the committed golden fixtures (guards against oracle drift)."""
import glob
import os

import numpy as np
import pytest

from oracle.adasplash import block_mask, pack_block_mask, reference_attention, reference_attention_backward
from oracle.entmax import entmax_backward, entmax_bisect
from oracle.lazy import lazy_backward, lazy_forward

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _load(name):
    return dict(np.load(os.path.join(GOLD, name + ".npz"), allow_pickle=False))


def test_fixture_set_present():
    names = sorted(os.path.basename(p)[:-4] for p in glob.glob(os.path.join(GOLD, "*.npz")))
    assert len(names) == 9, names


@pytest.mark.parametrize("a", [1.25, 1.5, 2.0])
def test_entmax(a):
    d = _load(f"entmax_a{a}")
    y = entmax_bisect(d["x"], a, n_iter=80)
    np.testing.assert_allclose(y, d["y"], atol=1e-6)
    np.testing.assert_allclose(entmax_backward(y, d["dy"], a), d["dx"], atol=1e-5)


@pytest.mark.parametrize("a", [1.5, 2.0])
@pytest.mark.parametrize("c", [0, 1])
def test_adasplash(a, c):
    d = _load(f"ada_a{a}_c{c}")
    o, aux = reference_attention(d["q"], d["k"], d["v"], a, d["varlen"], bool(c), return_aux=True)
    np.testing.assert_allclose(o, d["out"], atol=1e-6)
    m = pack_block_mask(block_mask(aux["p"], aux["row_valid"])).view(np.int32)
    assert (m == d["mask"]).all()
    g = reference_attention_backward(d["q"], d["k"], d["v"], d["do"], a, d["varlen"], bool(c))
    for got, key in zip(g, ("dq", "dk", "dv")):
        np.testing.assert_allclose(got, d[key], atol=1e-5)


@pytest.mark.parametrize("name", ["lazy_full", "lazy_varlen"])
def test_lazy(name):
    d = _load(name)
    vl = d.get("varlen")
    W = int(d["window"])
    o = lazy_forward(d["q"], d["k"], d["v"], d["bias"], d["tau"], W, vl)
    np.testing.assert_allclose(o, d["out"], atol=1e-6)
    g = lazy_backward(d["q"], d["k"], d["v"], d["bias"], d["tau"], d["do"], W, vl)
    for got, key in zip(g, ("dq", "dk", "dv", "dbias", "dtau")):
        np.testing.assert_allclose(got, d[key], atol=1e-5)
