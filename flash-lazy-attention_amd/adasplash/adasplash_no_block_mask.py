"""AdaSplash without the block mask: same kernels, every visible tile is computed.

Drop-in for ``adasplash.adasplash_no_block_mask(q, k, v, alpha=1.5, niter=10,
is_causal=False, varlen=None)`` (reference README.md:50-58,
tests/test_adasplash_no_block_mask.py).
"""
import torch

from .adasplash_block_mask import AdaSplashFunction, _forward


def adasplash_no_block_mask(q, k, v, alpha=1.5, niter=10, is_causal=False, varlen=None):
    if torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v)):
        return AdaSplashFunction.apply(q, k, v, alpha, niter, is_causal, varlen, False)
    out, *_rest = _forward(q, k, v, alpha, niter, is_causal, varlen, False, False)
    D = q.shape[-1]
    return out[..., :D] if out.shape[-1] != D else out
