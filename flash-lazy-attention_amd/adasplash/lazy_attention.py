"""LazyAttention: the attention layer around ``lazy_attention_triton``.

Drop-in for ``adasplash.lazy_attention.LazyAttention(dim, num_heads, window_size, rope_base)``
(the module is absent from the reference tree; its contract is README.md:88-108 and
tests/test_lazy_attention.py:5-71: ``forward(x)`` maps [B, L, dim] to [B, L, dim], learnable
``tau`` [H] and ``attention_biases`` [H, window_size], RoPE on q and k).  Layout and
parameter conventions follow the reference's layer example (examples/lazy_attention_layer.py:
34-90): q/k/v/o projections without output bias, fp32 ``tau`` initialised to -1, fp32 biases
initialised to 0, rotate-half RoPE with base ``rope_base``, grouped K/V heads.

With a ``LazyKVCache`` the layer also decodes: the cached (rotated) keys and values are
attended by the new positions through the KV-cache kernels (the layer example's
past_key_values path, examples/lazy_attention_layer.py:133-144).

The attention itself is the HIP kernel pair behind ``lazy_attention_triton``: inputs must be
GPU tensors (a CPU input raises, there is no PyTorch fallback).  K/V heads are read in place
for grouped-query attention (no repeat_interleave, unlike examples/sw_attention_lazy.py:154).
"""
import torch
import torch.nn as nn

from .lazy_attention_triton import lazy_attention_triton


class RotaryEmbedding(nn.Module):
    """Rotate-half rotary position embedding (pairs (x_i, x_{i+D/2}) rotated by angle
    pos * base^(-2i/D)), the convention of the layer example's RotaryEmbedding
    (examples/lazy_attention_layer.py:81,131)."""

    def __init__(self, dim, base=10000.0):
        super().__init__()
        if dim % 2:
            raise ValueError("rotary dim must be even")
        self.dim = dim
        self.base = float(base)
        self._cache = {}

    def _cos_sin(self, L, offset, device, dtype):
        key = (L, offset, device, dtype)
        if key not in self._cache:
            inv = self.base ** (-torch.arange(0, self.dim, 2, dtype=torch.float64, device=device) / self.dim)
            pos = torch.arange(offset, offset + L, dtype=torch.float64, device=device)
            ang = pos[:, None] * inv[None, :]
            self._cache = {key: (ang.cos().to(dtype), ang.sin().to(dtype))}
        return self._cache[key]

    def forward(self, q, k, offset=0):
        """q, k: [B, L, H, D] -> rotated copies (positions offset .. offset+L-1)."""
        L = q.shape[1]
        cos, sin = self._cos_sin(L, offset, q.device, torch.float32)
        cos, sin = cos[None, :, None, :], sin[None, :, None, :]

        def rot(x):
            x1, x2 = x.float().chunk(2, dim=-1)
            return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1).to(x.dtype)

        return rot(q), rot(k)


class LazyKVCache:
    """Preallocated K/V cache [B, H_kv, max_len, D] for LazyAttention decoding (rotated keys)."""

    def __init__(self, batch, num_kv_heads, max_len, head_dim, device=None, dtype=torch.float32):
        self.k = torch.zeros(batch, num_kv_heads, max_len, head_dim, device=device, dtype=dtype)
        self.v = torch.zeros_like(self.k)
        self.len = 0

    def append(self, k, v):
        """k, v [B, H_kv, L, D] -> views of the whole cache so far."""
        L = k.shape[2]
        if self.len + L > self.k.shape[2]:
            raise ValueError("KV cache is full")
        self.k[:, :, self.len:self.len + L] = k
        self.v[:, :, self.len:self.len + L] = v
        self.len += L
        return self.k[:, :, :self.len], self.v[:, :, :self.len]


class LazyAttention(nn.Module):
    def __init__(self, dim, num_heads, window_size=512, rope_base=10000.0, num_kv_heads=None, qkv_bias=False):
        super().__init__()
        if dim % num_heads:
            raise ValueError(f"dim={dim} is not a multiple of num_heads={num_heads}")
        self.dim = dim
        self.num_heads = num_heads
        self.num_kv_heads = num_heads if num_kv_heads is None else num_kv_heads
        if num_heads % self.num_kv_heads:
            raise ValueError("num_heads must be a multiple of num_kv_heads")
        self.head_dim = dim // num_heads
        self.window_size = window_size
        kv_dim = self.num_kv_heads * self.head_dim
        self.q_proj = nn.Linear(dim, dim, bias=qkv_bias)
        self.k_proj = nn.Linear(dim, kv_dim, bias=qkv_bias)
        self.v_proj = nn.Linear(dim, kv_dim, bias=qkv_bias)
        self.o_proj = nn.Linear(dim, dim, bias=False)
        self.rotary = RotaryEmbedding(self.head_dim, rope_base)
        # fp32 so that bf16 training does not underflow their gradients (lazy_attention_layer.py:84-89)
        self.attention_biases = nn.Parameter(torch.zeros(num_heads, window_size, dtype=torch.float32))
        self.tau = nn.Parameter(torch.full((num_heads,), -1.0, dtype=torch.float32))

    def new_cache(self, batch, max_len, device=None, dtype=None):
        w = self.q_proj.weight
        return LazyKVCache(batch, self.num_kv_heads, max_len, self.head_dim, device or w.device, dtype or w.dtype)

    def forward(self, x, varlen=None, cache=None):
        """x: [B, L, dim] -> [B, L, dim].  varlen: optional [B] true lengths (right padding);
        output rows at positions >= varlen[b] are zero before the output projection.
        cache: optional LazyKVCache; x then holds the next L positions after the cached ones
        (prefill when the cache is empty, decode steps after that; inference only)."""
        B, L, _ = x.shape
        q = self.q_proj(x).view(B, L, self.num_heads, self.head_dim)
        k = self.k_proj(x).view(B, L, self.num_kv_heads, self.head_dim)
        v = self.v_proj(x).view(B, L, self.num_kv_heads, self.head_dim)
        offset = 0 if cache is None else cache.len
        q, k = self.rotary(q, k, offset)
        # [B, L, H, D] -> [B, H, L, D] as strided views; the op reads them in place
        q, k, v = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
        if cache is not None:
            if varlen is not None:
                raise ValueError("varlen is not supported together with a KV cache")
            k, v = cache.append(k, v)
        o = lazy_attention_triton(q, k, v, self.attention_biases, self.tau, window_size=self.window_size, varlen=varlen)
        return self.o_proj(o.transpose(1, 2).reshape(B, L, self.dim))
