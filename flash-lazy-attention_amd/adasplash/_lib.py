"""ctypes binding of libflashlazy.so (the C ABI declared in include/flashlazy.h).

The library is the only compute path: there is no CPU or PyTorch fallback.  If it is
missing, importing an operator raises immediately.
"""
import ctypes
import math
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libflashlazy.so")

FLA_F32, FLA_F16, FLA_BF16 = 0, 1, 2
DTYPE_CODE = {torch.float32: FLA_F32, torch.float16: FLA_F16, torch.bfloat16: FLA_BF16}

_ERRORS = {-1: "invalid argument", -2: "unsupported dtype / head dim", -3: "workspace too small or misaligned"}


class Tensor4(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("stride_b", ctypes.c_int64),
        ("stride_h", ctypes.c_int64),
        ("stride_l", ctypes.c_int64),
    ]


_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float
_T4 = ctypes.POINTER(Tensor4)

SIGNATURES = {
    "fla_version": ([], ctypes.c_char_p),
    "fla_entmax_fwd": ([_P, _P, _I64, _I64, _I64, _I64, _I, _F, _I, _I, _P], _I),
    "fla_entmax_bwd": ([_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I, _F, _P], _I),
    "fla_adasplash_mask_words": ([_I], _I),
    "fla_unpack_block_mask": ([_P, _P, _I64, _I, _I, _P], _I),
    "fla_adasplash_fwd": (
        [_T4, _T4, _T4, _T4, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _I, _I, _I, _F, _P],
        _I,
    ),
    "fla_adasplash_bwd": (
        [_T4, _T4, _T4, _T4, _T4, _T4, _T4, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _I, _F, _P],
        _I,
    ),
    "fla_lazy_fwd": ([_T4, _T4, _T4, _T4, _P, _I64, _P, _I, _P, _P, _P, _P, _I, _P, _I, _I, _I, _I, _I, _I, _F, _P], _I),
    "fla_lazy_bwd_workspace_size": ([_I, _I, _I, _I], ctypes.c_size_t),
    "fla_lazy_decode_workspace_size": ([_I, _I, _I, _I, _I, _I], ctypes.c_size_t),
    "fla_lazy_decode_fwd": (
        [_T4, _T4, _T4, _T4, _P, _I64, _P, _I, _P, _P, ctypes.c_size_t, _I, _I, _I, _I, _I, _I, _I, _F, _P],
        _I,
    ),
    "fla_lazy_decode_fwd_static": (
        [_T4, _T4, _T4, _T4, _P, _I64, _P, _I, _P, _I, _I, _I, _I, _I, _I, _I, _F, _P],
        _I,
    ),
    "fla_lazy_bwd": (
        [_T4, _T4, _T4, _T4, _T4, _T4, _T4, _P, _I64, _P, _I, _P, _P, _P, _P, _P, _P, ctypes.c_size_t,
         _I, _I, _I, _I, _I, _I, _F, _P],
        _I,
    ),
}

_lib = None


def lib():
    """Load libflashlazy.so once; raise loudly if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} not found: build the HIP library first "
                "(python flash-lazy-attention_amd/build.py)"
            )
        l = ctypes.CDLL(LIB_PATH)
        for name, (argt, rest) in SIGNATURES.items():
            fn = getattr(l, name)
            fn.argtypes = argt
            fn.restype = rest
        _lib = l
    return _lib


def check(rc, what):
    if rc != 0:
        msg = _ERRORS.get(rc, f"HIP error {rc}")
        raise RuntimeError(f"{what} failed: {msg}")


def t4(x):
    return Tensor4(x.data_ptr(), x.stride(0), x.stride(1), x.stride(2))


def ptr(x):
    # A plain int: ctypes converts it for c_void_p parameters without building a wrapper.
    return None if x is None else x.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(x):
    """Handle of the current HIP stream of x's device (an int; cheaper than a Stream object)."""
    if _raw_stream is not None:
        return _raw_stream(x.get_device())
    return torch.cuda.current_stream(x.device).cuda_stream


def kernel_head_dim(D):
    for k in (32, 64, 128):
        if D <= k:
            return k
    raise ValueError(f"head dim {D} > 128 is not supported")


def _aligned(x):
    es = x.element_size()
    return (
        x.stride(-1) == 1
        and x.data_ptr() % 16 == 0
        and all((s * es) % 16 == 0 for s in x.stride()[:-1])
        and 0 < x.stride(-2) * es <= (1 << 24)
    )


def prep_bhld(x, Dk):
    """[B, H, L, D] -> kernel layout: D padded with zeros to Dk, last dim contiguous, 16-byte rows."""
    if x.dim() != 4:
        raise ValueError(f"expected a [B, H, L, D] tensor, got shape {tuple(x.shape)}")
    if x.shape[-1] != Dk:
        x = torch.nn.functional.pad(x, (0, Dk - x.shape[-1]))
    if not _aligned(x):
        x = x.contiguous()
    return x


def check_inputs(q, k, v, kv_longer=False):
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise ValueError("q, k, v must be GPU tensors")
    if q.dtype not in DTYPE_CODE:
        raise TypeError(f"unsupported dtype {q.dtype}; expected float32, float16 or bfloat16")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise TypeError("q, k, v must share one dtype")
    if q.dim() != 4 or k.shape != v.shape or k.dim() != 4:
        raise ValueError(f"expected [B, H, L, D] q and matching k, v; got {tuple(q.shape)}, {tuple(k.shape)}, "
                         f"{tuple(v.shape)}")
    B, H, L, D = q.shape
    okL = k.shape[2] >= L if kv_longer else k.shape[2] == L
    if k.shape[0] != B or not okL or k.shape[3] != D or k.shape[1] <= 0 or H % k.shape[1]:
        raise ValueError(f"k, v must be [B, H_kv, L, D] with H_kv dividing H={H}; got {tuple(k.shape)}")
    return D, 1.0 / math.sqrt(D)


def prep_varlen(varlen, B, device):
    if varlen is None:
        return None
    vl = torch.as_tensor(varlen, device=device).reshape(-1)
    if vl.numel() != B:
        raise ValueError(f"varlen must have B={B} entries, got {vl.numel()}")
    return vl.to(torch.int32).contiguous()


def unpack_block_mask(words, ncols):
    """int32 [..., R, MW] bit rows (bit c%32 of word c/32 = column c) -> bool [..., R, ncols],
    expanded by one kernel (fla_unpack_block_mask) on the current stream."""
    words = words.contiguous()
    out = torch.empty((*words.shape[:-1], ncols), device=words.device, dtype=torch.bool)
    rows = words.numel() // words.shape[-1] if words.numel() else 0
    rc = lib().fla_unpack_block_mask(ptr(words), ptr(out), rows, words.shape[-1], ncols, stream_of(words))
    check(rc, "fla_unpack_block_mask")
    return out
