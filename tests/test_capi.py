"""The C ABI library loads without a GPU, exports every symbol include/flashlazy.h declares,
and rejects bad arguments before touching the device."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "flashlazy.h")


def _lib():
    from adasplash import _lib as L

    if not os.path.exists(L.LIB_PATH):
        pytest.skip("libflashlazy.so not built")
    return L, L.lib()


def _declared():
    txt = open(HEADER).read()
    return sorted(set(re.findall(r"^\w[\w\s\*]*?\b(fla_\w+)\s*\(", txt, flags=re.M)))


def test_header_declares_the_abi():
    names = _declared()
    for n in ("fla_entmax_fwd", "fla_entmax_bwd", "fla_adasplash_fwd", "fla_adasplash_bwd", "fla_lazy_fwd",
              "fla_lazy_bwd", "fla_lazy_bwd_workspace_size", "fla_adasplash_mask_words", "fla_version",
              "fla_lazy_decode_fwd", "fla_lazy_decode_workspace_size"):
        assert n in names


def test_every_declared_symbol_is_exported():
    L, lib = _lib()
    for n in _declared():
        assert hasattr(lib, n), n
        assert n in L.SIGNATURES, f"{n} has no ctypes signature"


def test_decode_workspace_plan():
    L, lib = _lib()
    assert lib.fla_lazy_decode_workspace_size(2, 8, 2, 1, 4096, 64) > 0
    assert lib.fla_lazy_decode_workspace_size(2, 8, 3, 1, 4096, 64) == 0  # H % Hkv != 0
    assert lib.fla_lazy_decode_workspace_size(2, 8, 2, 1, 4096, 48) == 0  # not a kernel head dim
    # 8 rows per K/V head at D = 64: the 16-bit path keeps the scores (8 rows x 1024 keys,
    # fp32) besides the per-chunk partials; 32 rows at D = 64 read K again instead
    ws = lib.fla_lazy_decode_workspace_size(1, 8, 1, 1, 1000, 64)
    assert ws % 256 == 0 and ws >= 8 * 1024 * 4
    assert lib.fla_lazy_decode_workspace_size(1, 8, 1, 4, 1000, 64) % 256 == 0


def test_pure_helpers():
    _L, lib = _lib()
    assert lib.fla_version().startswith(b"flashlazy")
    assert lib.fla_adasplash_mask_words(8192) == 4
    assert lib.fla_adasplash_mask_words(64) == 1
    assert lib.fla_adasplash_mask_words(2049) == 2
    assert lib.fla_adasplash_mask_words(0) == 0
    ws = lib.fla_lazy_bwd_workspace_size(2, 8, 4096, 512)
    assert ws >= 2 * 8 * 32 * 512 * 4 + 2 * 8 * 4096 * 4 and ws % 256 == 0
    assert lib.fla_lazy_bwd_workspace_size(0, 8, 4096, 512) == 0


def test_argument_validation_without_gpu():
    L, lib = _lib()
    buf = ctypes.create_string_buffer(4096 + 16)
    base = (ctypes.addressof(buf) + 15) // 16 * 16
    t = L.Tensor4(base, 64 * 64, 64 * 64, 64)
    tp = ctypes.byref(t)
    # head dim 48 is not a kernel head dim
    assert lib.fla_adasplash_fwd(tp, tp, tp, tp, base, None, None, None, 1, 1, 1, 64, 48, L.FLA_BF16, 1.5, 10, 0, 1,
                                 0.125, None) == -1
    # alpha outside (1, 2]
    assert lib.fla_adasplash_fwd(tp, tp, tp, tp, base, None, None, None, 1, 1, 1, 64, 64, L.FLA_BF16, 2.5, 10, 0, 1,
                                 0.125, None) == -1
    # misaligned row stride
    bad = L.Tensor4(base, 64 * 64, 64 * 64, 63)
    assert lib.fla_adasplash_fwd(ctypes.byref(bad), tp, tp, tp, base, None, None, None, 1, 1, 1, 64, 64, L.FLA_BF16,
                                 1.5, 10, 0, 1, 0.125, None) == -1
    # unknown dtype
    assert lib.fla_entmax_fwd(base, base, 4, 8, 8, 8, 7, 1.5, 10, 1, None) == -1
    # lazy backward without workspace
    assert lib.fla_lazy_bwd(tp, tp, tp, tp, tp, tp, tp, base, 64, base, 16, base, base, None, None, None, None, 0, 1,
                            1, 1, 64, 64, L.FLA_BF16, 0.125, None) == -3
    # dbias without dtau
    assert lib.fla_lazy_bwd(tp, tp, tp, tp, tp, tp, tp, base, 64, base, 16, base, base, None, base, None, None, 0, 1,
                            1, 1, 64, 64, L.FLA_BF16, 0.125, None) == -1
    # H not a multiple of H_kv
    assert lib.fla_adasplash_fwd(tp, tp, tp, tp, base, None, None, None, 1, 3, 2, 64, 64, L.FLA_BF16, 1.5, 10, 0, 1,
                                 0.125, None) == -1


def test_host_layout_helpers():
    import torch

    from adasplash._lib import kernel_head_dim, prep_bhld

    assert [kernel_head_dim(d) for d in (8, 16, 32, 33, 64, 100, 128)] == [32, 32, 32, 64, 64, 128, 128]
    with pytest.raises(ValueError):
        kernel_head_dim(129)
    x = torch.randn(2, 3, 5, 16)
    y = prep_bhld(x, 32)
    assert y.shape == (2, 3, 5, 32) and torch.equal(y[..., :16], x) and (y[..., 16:] == 0).all()
    z = torch.randn(2, 5, 3, 64).transpose(1, 2)  # [B, H, L, D] view of a [B, L, H, D] tensor
    assert prep_bhld(z, 64).data_ptr() == z.data_ptr()
