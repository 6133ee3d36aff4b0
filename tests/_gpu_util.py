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
    got = np.atleast_1d(np.asarray(got, dtype=np.float64))
    ref = np.atleast_1d(np.asarray(ref, dtype=np.float64))
    err = np.abs(got - ref)
    bad = ~(err <= atol)
    if bad.any():
        tols = np.broadcast_to(np.asarray(atol, dtype=np.float64), err.shape)
        ratio = np.where(np.isnan(err), np.inf, err / np.maximum(tols, 1e-300))
        idx = np.unravel_index(np.argmax(ratio), err.shape)  # the worst violation
        tol = float(tols[idx])
        raise AssertionError(
            f"{what}: abs err {err[idx]:.3e} > {tol:g} at {idx} (got {got[idx]}, ref {ref[idx]}; max abs err "
            f"{np.nanmax(err):.3e}); "
            f"{bad.sum()} / {bad.size} entries out of tolerance"
        )


def rope(x, base=10000.0):
    """Rotary position embedding (rotate-half, examples/lazy_attention_layer.py:81-89) of a
    [B, H, L, D] tensor, computed in float32 and returned in x's dtype."""
    B, H, L, D = x.shape
    inv = 1.0 / (base ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    ang = torch.arange(L, dtype=torch.float32)[:, None] * inv[None, :]
    cos, sin = torch.cos(ang).repeat(1, 2), torch.sin(ang).repeat(1, 2)
    xf = x.float()
    rot = torch.cat((-xf[..., D // 2:], xf[..., : D // 2]), dim=-1)
    return (xf * cos + rot * sin).to(x.dtype)


def ulp32(x):
    """Spacing of float32 numbers at |x| (float64 array)."""
    x = np.abs(np.asarray(x, dtype=np.float64)).astype(np.float32)
    with np.errstate(invalid="ignore"):
        return (np.nextafter(x, np.float32(np.inf)) - x).astype(np.float64)
