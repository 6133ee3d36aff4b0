"""lazy_attention_triton on the GPU vs the oracle.

Mirrors tests/test_lazy_attention_triton.py, tests/test_lazy_attention_triton_backward.py and
tests/test_lazy_attention_varlen.py; the bias window follows the kernel (0 <= i-j < W,
lazy_attention_triton.py:62).
"""
import numpy as np
import pytest
import torch

from _gpu_util import DEV, assert_close, banner, rand, to_np
from oracle.lazy import lazy_backward, lazy_block_mask, lazy_forward, lazy_weights

pytestmark = pytest.mark.gpu


def _op():
    from adasplash import lazy_attention_triton

    return lazy_attention_triton


def _case(B, H, L, D, Wb, dtype, seed=42, tau=-1.0):
    q, k, v = (rand((B, H, L, D), dtype, seed + i) for i in range(3))
    bias = rand((H, Wb), torch.float32, seed + 3)
    t = torch.full((H,), tau, dtype=torch.float32)
    return q, k, v, bias, t


def test_forward_vs_reference_fp32():
    # tests/test_lazy_attention_triton.py:16-90 (B2 H4 L128 D64, W=32, bias [H, W+1])
    q, k, v, bias, tau = _case(2, 4, 128, 64, 33, torch.float32)
    ref = lazy_forward(to_np(q), to_np(k), to_np(v), to_np(bias), to_np(tau), 32)
    out = _op()(q.to(DEV), k.to(DEV), v.to(DEV), bias.to(DEV), tau.to(DEV), window_size=32)
    assert_close(to_np(out), ref, 1e-5, "lazy forward")


@pytest.mark.parametrize("tauval", [-1.0, -0.2, 0.3])
@pytest.mark.parametrize("shape", [(1, 1, 32, 16, 8), (2, 2, 200, 64, 48), (1, 2, 300, 32, 500)])
def test_backward_vs_reference_fp32(tauval, shape):
    # tests/test_lazy_attention_triton_backward.py:40-111 (B1 H1 L32 D16 W8)
    B, H, L, D, W = shape
    banner("lazy bwd fp32", shape, tauval)
    q, k, v, bias, tau = _case(B, H, L, D, W + 1, torch.float32, seed=5, tau=tauval)
    do = rand((B, H, L, D), torch.float32, 77)
    ref_out = lazy_forward(to_np(q), to_np(k), to_np(v), to_np(bias), to_np(tau), W)
    ref = lazy_backward(to_np(q), to_np(k), to_np(v), to_np(bias), to_np(tau), to_np(do), W)
    ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v, bias, tau)]
    out = _op()(*ts, window_size=W)
    assert_close(to_np(out), ref_out, 1e-5, "forward")
    out.backward(do.to(DEV))
    for got, r, n in zip([t.grad for t in ts], ref, ["dq", "dk", "dv", "dbias", "dtau"]):
        assert_close(to_np(got), r, 1e-4 * max(1.0, np.abs(r).max()), n)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [32, 64, 128])
def test_lowp_forward_backward(dtype, D):
    banner("lazy lowp", dtype, D)
    B, H, L, W = 2, 2, 384, 96
    q, k, v, bias, tau = _case(B, H, L, D, W, dtype, seed=9)
    bias = bias * 0.5
    do = rand((B, H, L, D), dtype, 10)
    ref_out = lazy_forward(to_np(q), to_np(k), to_np(v), to_np(bias), to_np(tau), W)
    ref = lazy_backward(to_np(q), to_np(k), to_np(v), to_np(bias), to_np(tau), to_np(do), W)
    ts = [q.to(DEV).requires_grad_(True), k.to(DEV).requires_grad_(True), v.to(DEV).requires_grad_(True),
          bias.to(DEV).requires_grad_(True), tau.to(DEV).requires_grad_(True)]
    out = _op()(*ts)
    assert_close(to_np(out), ref_out, 2e-2, "forward")
    out.backward(do.to(DEV))
    for got, r, n in zip([t.grad for t in ts], ref, ["dq", "dk", "dv", "dbias", "dtau"]):
        assert_close(to_np(got), r, 2e-2 * max(1.0, np.abs(r).max() / 2), n)


def test_varlen_forward_and_padding():
    # tests/test_lazy_attention_varlen.py:13-134
    q, k, v, bias, tau = _case(2, 4, 128, 64, 33, torch.float32, seed=1)
    varlen = torch.tensor([64, 100], dtype=torch.int32)
    ref = lazy_forward(to_np(q), to_np(k), to_np(v), to_np(bias), to_np(tau), 32, varlen.numpy())
    out = _op()(q.to(DEV), k.to(DEV), v.to(DEV), bias.to(DEV), tau.to(DEV), window_size=32, varlen=varlen.to(DEV))
    assert (out[0, :, 64:] == 0).all() and (out[1, :, 100:] == 0).all()
    assert_close(to_np(out), ref, 1e-5, "varlen forward")


@pytest.mark.parametrize("tauval", [-1.0, 0.4])
def test_varlen_backward(tauval):
    # tests/test_lazy_attention_varlen.py:136-169 (+ values vs the oracle)
    B, H, L, D, W = 2, 4, 64, 32, 16
    q, k, v, bias, tau = _case(B, H, L, D, W, torch.float32, seed=2, tau=tauval)
    varlen = np.array([32, 48])
    do = rand((B, H, L, D), torch.float32, 3)
    ref = lazy_backward(to_np(q), to_np(k), to_np(v), to_np(bias), to_np(tau), to_np(do), W, varlen)
    ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v, bias, tau)]
    out = _op()(*ts, window_size=W, varlen=torch.tensor(varlen, dtype=torch.int32, device=DEV))
    out.backward(do.to(DEV))
    for got, r, n in zip([t.grad for t in ts], ref, ["dq", "dk", "dv", "dbias", "dtau"]):
        assert_close(to_np(got), r, 1e-4 * max(1.0, np.abs(r).max()), n)
    for t in ts[:3]:
        assert (t.grad[0, :, 32:] == 0).all() and (t.grad[1, :, 48:] == 0).all()


@pytest.mark.parametrize("varlen", [[90, 200], [64, 130]])
def test_varlen_whole_row_tiles_past_length(varlen):
    # Row tiles of 128 queries that start at or past varlen[b] while the window-free key range
    # before them is non-empty: they must do no work and write exact zeros (regression: they
    # once swept key tiles that were never loaded).
    banner("lazy varlen empty row tiles", varlen)
    B, H, L, D, W = 2, 2, 260, 32, 40
    q, k, v, bias, tau = _case(B, H, L, D, W, torch.float32, seed=8, tau=0.2)
    do = rand((B, H, L, D), torch.float32, 9)
    ref = lazy_forward(to_np(q), to_np(k), to_np(v), to_np(bias), to_np(tau), W, np.array(varlen))
    rg = lazy_backward(to_np(q), to_np(k), to_np(v), to_np(bias), to_np(tau), to_np(do), W, np.array(varlen))
    ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v, bias, tau)]
    for _rep in range(3):
        for t in ts:
            t.grad = None
        out = _op()(*ts, window_size=W, varlen=torch.tensor(varlen, dtype=torch.int32, device=DEV))
        assert_close(to_np(out), ref, 1e-5, "forward")
        out.backward(do.to(DEV))
        for got, r, n in zip([t.grad for t in ts], rg, ["dq", "dk", "dv", "dbias", "dtau"]):
            assert_close(to_np(got), r, 1e-4 * max(1.0, np.abs(r).max()), n)


def test_frozen_parameters_fast_path():
    q, k, v, bias, tau = _case(1, 2, 96, 64, 16, torch.float32, seed=4)
    do = rand((1, 2, 96, 64), torch.float32, 5)
    ref = lazy_backward(to_np(q), to_np(k), to_np(v), to_np(bias), to_np(tau), to_np(do), 16)
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    b, t = bias.to(DEV), tau.to(DEV)
    out = _op()(qd, kd, vd, b, t)
    out.backward(do.to(DEV))
    assert b.grad is None and t.grad is None
    for got, r, n in zip((qd.grad, kd.grad, vd.grad), ref[:3], "qkv"):
        assert_close(to_np(got), r, 1e-4, "d" + n)


def test_very_negative_tau_gives_zero():
    q, k, v, bias, tau = _case(1, 2, 64, 32, 8, torch.float32, seed=6, tau=-100.0)
    out = _op()(q.to(DEV), k.to(DEV), v.to(DEV), bias.to(DEV), tau.to(DEV))
    assert out.abs().max().item() < 1e-6


def test_bf16_bias_and_tau_dtypes():
    # examples pass bias / tau in the model dtype (lazy_attention_layer.py:164-170)
    q, k, v, bias, tau = _case(1, 2, 128, 64, 32, torch.bfloat16, seed=8)
    bb, tb = bias.to(torch.bfloat16), tau.to(torch.bfloat16)
    ref = lazy_forward(to_np(q), to_np(k), to_np(v), to_np(bb), to_np(tb), 32)
    ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v, bb, tb)]
    out = _op()(*ts)
    assert_close(to_np(out), ref, 2e-2, "bf16 params forward")
    out.sum().backward()
    assert ts[3].grad.dtype == torch.bfloat16 and ts[4].grad.dtype == torch.bfloat16


@pytest.mark.parametrize("tauval", [-1.0, -0.3, 0.3, -10.0])
@pytest.mark.parametrize("varlen", [None, [150, 260]])
def test_block_mask_vs_oracle(tauval, varlen):
    # Block sparsity planned at CURSOR_TASKS.md:214-312: 64x64 blocks with some relu(p + tau/i) > 0.
    banner("lazy block mask", tauval, varlen)
    B, H, L, D, W = 2, 2, 260, 32, 40
    q, k, v, bias, tau = _case(B, H, L, D, W, torch.float32, seed=31, tau=tauval)
    e, margin = lazy_weights(to_np(q), to_np(k), to_np(bias), to_np(tau), W, varlen)
    sure = lazy_block_mask(np.where(margin > 1e-6, e, 0.0))  # blocks with a weight clearly > 0
    maybe = lazy_block_mask(np.where(margin <= 1e-6, 1.0, e))  # ... or a near-tie
    vl = None if varlen is None else torch.tensor(varlen, dtype=torch.int32, device=DEV)
    args = [t.to(DEV) for t in (q, k, v, bias, tau)]
    out_m, bm = _op()(*args, window_size=W, varlen=vl, return_mask=True)
    out = _op()(*args, window_size=W, varlen=vl)
    got = bm.cpu().numpy()
    assert got.shape == sure.shape and got.dtype == np.bool_
    assert (got >= sure).all() and (got <= maybe).all(), "block mask differs from the oracle"
    assert torch.equal(out_m, out)  # skipped tiles contribute exactly zero
    if tauval == -10.0:
        from adasplash import get_sparsity_stats

        st = get_sparsity_stats(bm)
        assert st["block_density"] < 0.5 and st["theoretical_speedup"] > 2.0


def test_block_mask_with_autograd():
    q, k, v, bias, tau = _case(1, 2, 200, 64, 32, torch.float32, seed=12, tau=-0.5)
    do = rand((1, 2, 200, 64), torch.float32, 13)
    grads = []
    for want in (False, True):
        ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v, bias, tau)]
        res = _op()(*ts, window_size=32, return_mask=want)
        out = res[0] if want else res
        if want:
            assert res[1].dtype == torch.bool and not res[1].requires_grad
        out.backward(do.to(DEV))
        grads.append([t.grad.clone() for t in ts])
    for a, b, n in zip(*grads, ("dq", "dk", "dv", "dbias", "dtau")):
        assert torch.equal(a, b), n  # every reduction runs in a fixed order


@pytest.mark.parametrize("W", [300, 1500])
def test_parameter_gradients_bit_reproducible(W):
    """dbias / dtau are sums over every row of a head; the kernels build them in a fixed order
    (per-wave partial rows, then the waves and the tiles in index order), so repeated runs are
    bit-identical -- also for distances >= 1024, whose partials live in global memory."""
    banner("lazy dbias/dtau repeat", W)
    B, H, L, D = 2, 4, 1600, 64
    q, k, v, bias, tau = _case(B, H, L, D, W, torch.bfloat16, seed=40, tau=-0.7)
    do = rand((B, H, L, D), torch.bfloat16, 41)
    runs = []
    for _ in range(4):
        ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v, bias, tau)]
        _op()(*ts).backward(do.to(DEV))
        runs.append([t.grad.clone() for t in ts])
    for r in runs[1:]:
        for a, b, n in zip(runs[0], r, ("dq", "dk", "dv", "dbias", "dtau")):
            assert torch.equal(a, b), n
    ref = lazy_backward(to_np(q), to_np(k), to_np(v), to_np(bias), to_np(tau), to_np(do), W)
    for got, r, n in zip(runs[0][3:], ref[3:], ("dbias", "dtau")):
        assert_close(to_np(got), r, 2e-2 * max(1.0, np.abs(r).max() / 4), n)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_tie_at_row_zero_consistent(dtype):
    """tau = -1 puts row 0 exactly on the threshold (p = 1, p + tau/1 = 0).  Whichever side the
    float32 rounding picks, the forward (wdelta, hence delta) and the backward must pick the same
    one, and then dS of row 0 vanishes: dq row 0 = 0 on every head (regression: the backward
    re-derived p from a natural-log LSE and could disagree with the forward)."""
    banner("lazy row-0 tie", dtype)
    B, H, L, D, W = 2, 8, 200, 64, 64
    q, k, v, bias, tau = _case(B, H, L, D, W, dtype, seed=21, tau=-1.0)
    bias = bias * 0.5
    do = rand((B, H, L, D), dtype, 22)
    ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v, bias, tau)]
    out = _op()(*ts)
    out.backward(do.to(DEV))
    # the row's one key gets p = 1 exactly, so e = relu(1 - 1) = 0 exactly, as in exact arithmetic
    assert (out[:, :, 0] == 0).all()
    assert ts[0].grad[:, :, 0].abs().max().item() < 1e-4
    ref = lazy_backward(to_np(q), to_np(k), to_np(v), to_np(bias), to_np(tau), to_np(do), W)
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    for got, r, n in zip([t.grad for t in ts], ref, ["dq", "dk", "dv", "dbias", "dtau"]):
        assert_close(to_np(got), r, tol * max(1.0, np.abs(r).max() / 4), n)


@pytest.mark.parametrize("ncols", [1, 31, 32, 37, 64])
def test_unpack_block_mask_bits(ncols):
    # Bit c%32 of word c/32 -> column c, checked against numpy's little-endian bit unpacking
    # (sign bit 31 and a partial last word included).
    from adasplash._lib import unpack_block_mask

    banner("unpack_block_mask", ncols)
    mw = (ncols + 31) // 32
    w = np.random.default_rng(ncols).integers(-(2**31), 2**31, size=(2, 3, 5, mw), dtype=np.int64).astype(np.int32)
    w[0, 0, 0, -1] = np.int32(-(2**31))  # only bit 31 of the last word
    want = np.unpackbits(w.view(np.uint8), axis=-1, bitorder="little").reshape(2, 3, 5, 32 * mw)[..., :ncols]
    got = unpack_block_mask(torch.from_numpy(w).to(DEV), ncols)
    assert got.dtype == torch.bool and tuple(got.shape) == (2, 3, 5, ncols)
    assert np.array_equal(got.cpu().numpy(), want.astype(bool))


@pytest.mark.parametrize("H,G", [(9, 1), (12, 4)])
def test_launch_larger_than_one_round_matches_per_head(H, G):
    """Workgroups are ordered in a serpentine over dispatch rounds of one workgroup per compute
    unit; with more workgroups than compute units and a partial last round (B = 1, H = 9, L =
    4096: 288 row tiles on 256 units) the ranks must still cover each (head, row tile) once.
    Every head is independent, so the full launch equals the heads run one at a time
    (grids below one round), bit for bit: out, dq, dk, dv, dbias and dtau."""
    banner("lazy large launch vs per head", H, G)
    B, L, D, W = 1, 4096, 64, 512
    Hk = H // G
    q = rand((B, H, L, D), torch.bfloat16, 50)
    k, v = (rand((B, Hk, L, D), torch.bfloat16, 51 + i) for i in range(2))
    do = rand((B, H, L, D), torch.bfloat16, 53)
    bias = rand((H, W), torch.float32, 54) * 0.02
    tau = torch.linspace(-1.5, -0.2, H)
    ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v, bias, tau)]
    out = _op()(*ts, window_size=W)
    out.backward(do.to(DEV))
    for hk in range(Hk):
        hs = slice(hk * G, (hk + 1) * G)
        part = [t[:, hs] if i == 0 else (t[:, hk:hk + 1] if i < 3 else t[hs])
                for i, t in enumerate((q, k, v, bias, tau))]
        ps = [t.to(DEV).requires_grad_(True) for t in part]
        o1 = _op()(*ps, window_size=W)
        o1.backward(do[:, hs].to(DEV))
        assert torch.equal(out[:, hs], o1), ("out", hk)
        assert torch.equal(ts[0].grad[:, hs], ps[0].grad), ("dq", hk)
        assert torch.equal(ts[1].grad[:, hk:hk + 1], ps[1].grad), ("dk", hk)
        assert torch.equal(ts[2].grad[:, hk:hk + 1], ps[2].grad), ("dv", hk)
        assert torch.equal(ts[3].grad[hs], ps[3].grad), ("dbias", hk)
        assert torch.equal(ts[4].grad[hs], ps[4].grad), ("dtau", hk)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("L,varlen", [(260, None), (300, [300, 130]), (640, [577, 64])])
def test_mask_bytes_equal_mask_words(dtype, L, varlen):
    """The forward writes the block mask in two forms, bit words and one byte per block (the
    boolean mask of return_mask=True), from the same per-workgroup bits: every byte must equal
    the corresponding bit, for each dtype's kernel, ragged lengths and an odd number of 64-row
    blocks (the last workgroup's second block lies past the end)."""
    banner("lazy mask bytes vs words", dtype, L, varlen)
    from adasplash._lib import DTYPE_CODE, check, lib, ptr, stream_of, t4, unpack_block_mask

    B, H, D, W = 2, 3, 64, 48
    q, k, v, bias, tau = _case(B, H, L, D, W, dtype, seed=61, tau=-0.4)
    q, k, v = (t.to(DEV).contiguous() for t in (q, k, v))
    b32, t32 = bias.to(DEV), tau.to(DEV)
    vl = None if varlen is None else torch.tensor(varlen, dtype=torch.int32, device=DEV)
    nrb, mw = (L + 63) // 64, int(lib().fla_adasplash_mask_words(L))
    out = torch.empty_like(q)
    lse = torch.empty((B, H, L), device=DEV, dtype=torch.float32)
    words = torch.empty((B, H, nrb, mw), device=DEV, dtype=torch.int32)
    u8 = torch.full((B, H, nrb, nrb), 7, device=DEV, dtype=torch.uint8)
    rc = lib().fla_lazy_fwd(t4(q), t4(k), t4(v), t4(out), ptr(b32), W, ptr(t32), W, ptr(lse), None,
                            ptr(words), ptr(u8), 1, ptr(vl), B, H, H, L, D, DTYPE_CODE[dtype], D ** -0.5,
                            stream_of(q))
    check(rc, "fla_lazy_fwd")
    ref = unpack_block_mask(words, nrb)
    assert torch.equal(u8.bool(), ref) and int(u8.max()) <= 1
    assert bool(ref.any())
