"""Writes the small golden fixtures of this directory from the CPU oracle (float64).

    python tests/golden/make_golden.py

The reference ships no golden vectors and its Python package is absent, so the fixtures
are the oracle's outputs on seeded inputs (the oracle itself is pinned by
tests/test_oracle_*.py).  Each .npz holds inputs and expected outputs; tests compare
the oracle (regression) and the HIP kernels (GPU parity) against them.  Outputs are
stored as float32.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle.adasplash import (  # noqa: E402
    block_mask,
    pack_block_mask,
    reference_attention,
    reference_attention_backward,
)
from oracle.entmax import entmax_backward, entmax_bisect  # noqa: E402
from oracle.lazy import lazy_backward, lazy_forward  # noqa: E402


def f32(x):
    return np.asarray(x, dtype=np.float32)


def main():
    rng = np.random.default_rng(20241201)
    out = {}
    # entmax rows
    x = f32(rng.standard_normal((6, 37)) * 2)
    dy = f32(rng.standard_normal((6, 37)))
    for a in (1.25, 1.5, 2.0):
        y = entmax_bisect(x, a, n_iter=80)
        out[f"entmax_a{a}"] = dict(x=x, dy=dy, alpha=np.float64(a), y=y, dx=entmax_backward(y, dy, a))
    # adasplash
    B, H, L, D = 1, 1, 128, 32
    q, k, v, do = (f32(rng.standard_normal((B, H, L, D))) for _ in range(4))
    for a in (1.5, 2.0):
        for causal in (False, True):
            vl = np.array([117], dtype=np.int32)
            o, aux = reference_attention(q, k, v, a, vl, causal, return_aux=True)
            dq, dk, dv = reference_attention_backward(q, k, v, do, a, vl, causal)
            m = pack_block_mask(block_mask(aux["p"], aux["row_valid"])).view(np.int32)
            out[f"ada_a{a}_c{int(causal)}"] = dict(
                q=q, k=k, v=v, do=do, varlen=vl, alpha=np.float64(a), causal=np.int64(causal),
                out=o, tau=aux["tau"], mask=m, dq=dq, dk=dk, dv=dv)
    # lazy
    B, H, L, D, W = 1, 2, 96, 32, 24
    q, k, v, do = (f32(rng.standard_normal((B, H, L, D))) for _ in range(4))
    bias = f32(rng.standard_normal((H, W + 1)) * 0.5)
    tau = f32([-1.0, -0.4])
    for vl in (None, np.array([77], dtype=np.int32)):
        o, lse = lazy_forward(q, k, v, bias, tau, W, vl, return_aux=True)
        g = lazy_backward(q, k, v, bias, tau, do, W, vl)
        key = "lazy_full" if vl is None else "lazy_varlen"
        d = dict(q=q, k=k, v=v, do=do, bias=bias, tau=tau, window=np.int64(W), out=o, lse=lse,
                 dq=g[0], dk=g[1], dv=g[2], dbias=g[3], dtau=g[4])
        if vl is not None:
            d["varlen"] = vl
        out[key] = d
    for name, d in out.items():
        d = {k_: (v_.astype(np.float32) if isinstance(v_, np.ndarray) and v_.dtype == np.float64 else v_)
             for k_, v_ in d.items()}
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **d)
    print("wrote", len(out), "fixtures")


if __name__ == "__main__":
    main()
