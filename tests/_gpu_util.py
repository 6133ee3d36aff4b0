"""Helpers shared by the GPU parity tests (seeded inputs made on the CPU, compared on the CPU)."""
import sys

import numpy as np
import torch

DEV = "cuda"


def rand(shape, dtype, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def to_np(x):
    return x.detach().float().cpu().double().numpy()


def banner(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def assert_close(got, ref, atol, what=""):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    err = np.abs(got - ref)
    bad = ~(err <= atol)
    if bad.any():
        idx = np.unravel_index(np.argmax(np.where(np.isnan(err), np.inf, err)), err.shape)
        raise AssertionError(
            f"{what}: max abs err {np.nanmax(err):.3e} > {atol:g} at {idx} (got {got[idx]}, ref {ref[idx]}); "
            f"{bad.sum()} / {bad.size} entries out of tolerance"
        )
