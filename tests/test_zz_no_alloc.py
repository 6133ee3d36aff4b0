"""fla_lazy_decode_fwd_static (static per-GPU scratch, no allocation) against fla_lazy_decode_fwd
(caller workspace) through the C ABI: identical results on consecutive calls, the second one
smaller than the first, and a clear rejection of plans larger than the static scratch."""
import ctypes

import pytest
import torch

from _gpu_util import DEV, banner, rand

pytestmark = pytest.mark.gpu


def _call_both(B, H, Hkv, Lq, Lk, D, dtype, seed, varlen=None):
    from adasplash import _lib as L

    lib = L.lib()
    q = rand((B, H, Lq, D), dtype, seed).to(DEV)
    k = rand((B, Hkv, Lk, D), dtype, seed + 1).to(DEV)
    v = rand((B, Hkv, Lk, D), dtype, seed + 2).to(DEV)
    W = 256
    bias = (rand((H, W), torch.float32, seed + 3) * 0.3).to(DEV)
    tau = torch.full((H,), -0.5, device=DEV)
    vl = None if varlen is None else torch.tensor(varlen, dtype=torch.int32, device=DEV)
    o_ws = torch.empty_like(q)
    o_st = torch.full_like(q, float("nan"))
    code = L.DTYPE_CODE[dtype]
    scale = D ** -0.5
    nbytes = int(lib.fla_lazy_decode_workspace_size(B, H, Hkv, Lq, Lk, D))
    assert 0 < nbytes <= lib_static_bytes()
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    st = L.stream_of(q)
    rc = lib.fla_lazy_decode_fwd(L.t4(q), L.t4(k), L.t4(v), L.t4(o_ws), L.ptr(bias), W, L.ptr(tau), W, L.ptr(vl),
                                 L.ptr(ws), nbytes, B, H, Hkv, Lq, Lk, D, code, scale, st)
    L.check(rc, "fla_lazy_decode_fwd")
    rc = lib.fla_lazy_decode_fwd_static(L.t4(q), L.t4(k), L.t4(v), L.t4(o_st), L.ptr(bias), W, L.ptr(tau), W,
                                        L.ptr(vl), B, H, Hkv, Lq, Lk, D, code, scale, st)
    L.check(rc, "fla_lazy_decode_fwd_static")
    torch.cuda.synchronize()
    return o_ws, o_st


def lib_static_bytes():
    return 64 << 20


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_static_scratch_matches_workspace_entry_point(dtype):
    banner("decode static scratch", dtype)
    # first call: GQA-4, 4096 cached keys, D = 128 (score cache in use on the 16-bit path)
    a_ws, a_st = _call_both(4, 16, 4, 1, 4096, 128, dtype, 10, varlen=[4096, 3000, 17, 2500])
    assert torch.equal(a_ws, a_st)
    # second call, smaller: the scratch keeps the first call's contents, which must not leak in
    b_ws, b_st = _call_both(2, 8, 2, 3, 1000, 64, dtype, 20)
    assert torch.equal(b_ws, b_st)
    assert torch.isfinite(b_st).all()


def test_static_scratch_rejects_oversized_plans():
    from adasplash import _lib as L

    lib = L.lib()
    B, H, Hkv, Lq, Lk, D = 64, 64, 64, 1, 65536, 128
    assert lib.fla_lazy_decode_workspace_size(B, H, Hkv, Lq, Lk, D) > lib_static_bytes()
    dummy = torch.empty(16, device=DEV)
    t = L.Tensor4(dummy.data_ptr(), 0, 0, D)
    rc = lib.fla_lazy_decode_fwd_static(ctypes.byref(t), ctypes.byref(t), ctypes.byref(t), ctypes.byref(t),
                                        dummy.data_ptr(), 1, dummy.data_ptr(), 1, None, B, H, Hkv, Lq, Lk, D,
                                        L.FLA_BF16, 0.1, None)
    assert rc == -3  # FLA_EWORKSPACE: use fla_lazy_decode_fwd with a caller workspace
