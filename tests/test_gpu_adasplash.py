"""adasplash / adasplash_no_block_mask on the GPU vs the oracle.

Mirrors tests/test_adasplash.py and tests/test_adasplash_no_block_mask.py of the reference,
with the oracle restating its reference_attention (:22-60).  Tolerances: fp32 1e-4 (the
reference's, :73), bf16 2e-2 and fp16 1e-2 max-abs (tighter than the reference's 1e-1).
Support sets and block-mask bits are compared bit-exactly on fp32 inputs, excluding only
near-ties: entries whose distance to the oracle's threshold is within TIE_ULPS float32 ulps of
max(|z|, |tau|) (z = (alpha-1) * score); their number is printed and bounded.
"""
import math

import numpy as np
import pytest
import torch

from _gpu_util import DEV, assert_close, banner, rand, to_np, ulp32
from oracle.adasplash import block_mask, pack_block_mask, reference_attention, reference_attention_backward

pytestmark = pytest.mark.gpu
TOL = {torch.float32: 1e-4, torch.float16: 1e-2, torch.bfloat16: 2e-2}
TIE_ULPS = 8


def _ops():
    from adasplash import adasplash, adasplash_no_block_mask, adasplash_stats

    return adasplash, adasplash_no_block_mask, adasplash_stats


def _inputs(B, H, L, D, dtype, seed=42, scale=1.0):
    return [rand((B, H, L, D), dtype, seed + i, scale) for i in range(3)]


@pytest.mark.parametrize("B,H", [(1, 1), (2, 2)])
@pytest.mark.parametrize("L", [128, 256])
@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("alpha", [1.333, 1.5, 2.0])
@pytest.mark.parametrize("is_causal", [False, True])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32, torch.bfloat16])
@pytest.mark.parametrize("masked", [True, False])
def test_forward(B, H, L, D, alpha, is_causal, dtype, masked):
    banner("ada fwd", B, H, L, D, alpha, is_causal, dtype, masked)
    q, k, v = _inputs(B, H, L, D, dtype)
    g = torch.Generator().manual_seed(7)
    varlen = torch.randint(L // 2, L, (B,), generator=g)
    ref = reference_attention(to_np(q), to_np(k), to_np(v), alpha, varlen.numpy(), is_causal)
    op = _ops()[0] if masked else _ops()[1]
    out = op(q.to(DEV), k.to(DEV), v.to(DEV), alpha=alpha, varlen=varlen.to(DEV), is_causal=is_causal)
    assert out.dtype == dtype and out.shape == q.shape
    assert_close(to_np(out), ref, TOL[dtype], "adasplash forward")
    for b in range(B):
        assert (out[b, :, int(varlen[b]):] == 0).all()


@pytest.mark.parametrize("alpha", [1.5, 2.0, 1.25])
@pytest.mark.parametrize("is_causal", [False, True])
def test_threshold_support_and_block_mask(alpha, is_causal):
    B, H, L, D = 2, 2, 384, 64
    banner("ada support", alpha, is_causal)
    q, k, v = _inputs(B, H, L, D, torch.float32, seed=3, scale=1.5)
    varlen = np.array([384, 301])
    ref, aux = reference_attention(to_np(q), to_np(k), to_np(v), alpha, varlen, is_causal, return_aux=True)
    out, tau, mask = _ops()[2](q.to(DEV), k.to(DEV), v.to(DEV), alpha=alpha, is_causal=is_causal,
                              varlen=torch.tensor(varlen, device=DEV))
    assert_close(to_np(out), ref, 1e-4, "forward")
    tau = tau.cpu().double().numpy()
    rowv = aux["row_valid"]
    assert np.isinf(tau[~np.broadcast_to(rowv[:, None, :], tau.shape)]).all()
    tref = aux["tau"]
    valid = np.broadcast_to(rowv[:, None, :], tau.shape)
    assert_close(tau[valid] / (1 + np.abs(tref[valid])), tref[valid] / (1 + np.abs(tref[valid])), 1e-6, "threshold (relative)")
    # support: z - tau > 0 with the kernel's tau, compared to the oracle's support away from ties
    s = np.einsum("bhid,bhjd->bhij", to_np(q), to_np(k)) / math.sqrt(D)
    z = (alpha - 1) * s
    gap = z - tref[..., None]
    keyok = np.arange(L)[None, None, None, :] < varlen[:, None, None, None]
    if is_causal:
        keyok = keyok & np.tril(np.ones((L, L), dtype=bool))[None, None]
    ours = (z - np.where(np.isfinite(tau), tau, np.inf)[..., None] > 0) & keyok
    theirs = aux["p"] > 0
    tref_b = np.where(np.isfinite(tref), tref, 0.0)[..., None]
    win = TIE_ULPS * ulp32(np.maximum(np.abs(z), np.abs(tref_b)))
    cmp_ = valid[..., None] & keyok
    sure = (np.abs(gap) > win) & cmp_
    n_near = int((cmp_ & ~sure).sum())
    print(f"[case] support entries compared {int(cmp_.sum())}, near-ties (<= {TIE_ULPS} ulp) {n_near}, "
          f"differing {int((ours != theirs)[cmp_].sum())}", flush=True)
    assert (ours[sure] == theirs[sure]).all()
    assert n_near <= 1e-4 * cmp_.sum() + 4
    # block mask bits, exactly (ties excluded from the oracle mask only if they change a bit)
    mref = pack_block_mask(block_mask(aux["p"], rowv)).view(np.int32)
    got = mask.cpu().numpy()
    near = block_mask(cmp_ & ~sure, rowv)
    diff = (got != mref)
    if diff.any():
        # any differing word must come from a tile that holds a near-tie
        assert pack_block_mask(near)[diff].any(), "block mask differs away from near-ties"


@pytest.mark.parametrize("L", [256, 512])
@pytest.mark.parametrize("alpha", [1.5, 2.0])
@pytest.mark.parametrize("masked", [True, False])
def test_backward_fp32(L, alpha, masked):
    # tests/test_adasplash.py:94-122 (atol 1e-2 there; 2e-4 here)
    banner("ada bwd fp32", L, alpha, masked)
    B, H, D = 2, 2, 64
    q, k, v = _inputs(B, H, L, D, torch.float32)
    do = rand((B, H, L, D), torch.float32, 99)
    ref = reference_attention_backward(to_np(q), to_np(k), to_np(v), to_np(do), alpha)
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    op = _ops()[0] if masked else _ops()[1]
    out = op(qd, kd, vd, alpha=alpha)
    out.backward(do.to(DEV))
    for got, r, n in zip((qd.grad, kd.grad, vd.grad), ref, "qkv"):
        assert_close(to_np(got), r, 2e-4, f"d{n}")


@pytest.mark.parametrize("alpha", [1.5, 2.0, 1.333])
@pytest.mark.parametrize("is_causal", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [32, 64, 128])
def test_backward_lowp_varlen(alpha, is_causal, dtype, D):
    # 16-bit tiles use a head-dim-specific LDS layout (rows shifted per head dim), so every
    # supported D is compared with the oracle
    banner("ada bwd lowp", alpha, is_causal, dtype, D)
    B, H, L = 2, 2, 320
    q, k, v = _inputs(B, H, L, D, dtype, seed=11)
    do = rand((B, H, L, D), dtype, 12)
    varlen = np.array([320, 199])
    ref = reference_attention_backward(to_np(q), to_np(k), to_np(v), to_np(do), alpha, varlen, is_causal)
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    out = _ops()[0](qd, kd, vd, alpha=alpha, is_causal=is_causal, varlen=torch.tensor(varlen, device=DEV))
    out.backward(do.to(DEV))
    # P and dS enter the gradient products rounded to 16 bits (bf16: 2^-8 relative).  A row of
    # dQ = sum_j dS_ij k_j can cancel, so its absolute error follows sum_j |dS_ij k_j| rather than
    # |dQ_i|: typically up to ~0.4% of max|ref| at D = 32, 64, 128 alike, 1% on a cancelling row
    # (D = 32, alpha = 1.333).  The bound is 2% of max|ref| (at least 2e-2); a wrong operand or
    # layout gives errors of the order of max|ref| itself.
    for got, r, n in zip((qd.grad, kd.grad, vd.grad), ref, "qkv"):
        assert_close(to_np(got), r, 2e-2 * max(1.0, np.abs(r).max()), f"d{n}")
    for b in range(B):
        n = varlen[b]
        for gt in (qd.grad, kd.grad, vd.grad):
            assert (gt[b, :, n:] == 0).all()


def test_head_dim_padding_and_strides():
    banner("ada D=16/48 strided")
    for D in (16, 48):
        q, k, v = _inputs(1, 3, 200, D, torch.float32, seed=21)
        ref = reference_attention(to_np(q), to_np(k), to_np(v), 1.5, None, True)
        # non-contiguous [B, L, H, D] views
        qt, kt, vt = (t.transpose(1, 2).contiguous().to(DEV).transpose(1, 2) for t in (q, k, v))
        out = _ops()[0](qt, kt, vt, alpha=1.5, is_causal=True)
        assert_close(to_np(out), ref, 1e-4, f"D={D}")


@pytest.mark.parametrize("alpha,L", [(1.1, 512), (1.25, 768)])
def test_support_overflow_fallback(alpha, L):
    # supports larger than the per-row candidate list take the full-sweep Newton path
    banner("ada fallback", alpha, L)
    q, k, v = _inputs(1, 2, L, 32, torch.float32, seed=31, scale=0.5)
    ref = reference_attention(to_np(q), to_np(k), to_np(v), alpha, None, False)
    out = _ops()[0](q.to(DEV), k.to(DEV), v.to(DEV), alpha=alpha)
    assert_close(to_np(out), ref, 1e-4, "fallback forward")


@pytest.mark.parametrize("seq_len", [64, 128, 512])
def test_simple_case(seq_len):
    # tests/test_adasplash.py:148-158: zero q, k with v = 1 gives out = 1 (support = whole row)
    q = torch.zeros(1, 1, seq_len, 64, device=DEV)
    v = torch.ones_like(q)
    out = _ops()[0](q, q, v, alpha=1.5)
    assert torch.allclose(out, torch.ones_like(out), atol=1e-5)


def test_variable_length_handling():
    varlen = torch.tensor([128, 64], device=DEV)
    q, k, v = (t.to(DEV) for t in _inputs(2, 1, 256, 64, torch.float32, seed=5))
    out = _ops()[0](q, k, v, varlen=varlen)
    for i in range(2):
        assert (out[i, :, varlen[i]:] == 0).all()


@pytest.mark.parametrize("seq_len", [512, 1024])
def test_numerical_stability(seq_len):
    q, k, v = (t.to(DEV) for t in _inputs(2, 2, seq_len, 64, torch.float16, seed=6, scale=100.0))
    out = _ops()[0](q, k, v, alpha=1.5)
    assert torch.isfinite(out).all()
    assert out.abs().max() < 1e3


def test_repeat_bit_identical():
    q, k, v = (t.to(DEV) for t in _inputs(2, 4, 1024, 64, torch.bfloat16, seed=8))
    a = _ops()[0](q, k, v, alpha=1.5, is_causal=True)
    b = _ops()[0](q, k, v, alpha=1.5, is_causal=True)
    assert torch.equal(a, b)
