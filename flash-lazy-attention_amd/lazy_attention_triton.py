"""Top-level module of the same name as the reference's only shipped module
(setup.py:12 ``py_modules=["lazy_attention_triton"]``), re-exporting the HIP-backed op."""
from adasplash.lazy_attention_triton import LazyAttentionTritonFunc, lazy_attention_triton  # noqa: F401
