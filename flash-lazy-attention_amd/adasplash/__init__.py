"""AdaSplash / Lazy attention for AMD Instinct MI355X (gfx950), hand-written HIP kernels.

Drop-in names of the reference package (README.md:25-137):
``triton_entmax``, ``adasplash``, ``adasplash_no_block_mask``, ``lazy_attention_triton``,
and the ``LazyAttention`` layer (``adasplash.lazy_attention``, tests/test_lazy_attention.py).
"""
from .adasplash_block_mask import adasplash, adasplash_stats
from .adasplash_no_block_mask import adasplash_no_block_mask
from .lazy_attention import LazyAttention, LazyKVCache, RotaryEmbedding
from .lazy_attention_triton import LazyAttentionTritonFunc, get_sparsity_stats, lazy_attention_triton
from .triton_entmax import triton_entmax

__all__ = [
    "triton_entmax",
    "adasplash",
    "adasplash_no_block_mask",
    "adasplash_stats",
    "lazy_attention_triton",
    "LazyAttentionTritonFunc",
    "get_sparsity_stats",
    "LazyAttention",
    "RotaryEmbedding",
    "LazyKVCache",
]
