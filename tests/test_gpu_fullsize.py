"""Parity at the BASELINE configurations' own sizes (GPU against the float64 oracle).

Each test runs the HIP path on the whole configuration and checks it against the oracle on the
same bf16 inputs:
  * whole (b, h) slices -- output, threshold, dq, dk, dv -- through the row-chunked oracle
    (oracle.rows.ada_slice; oracle.lazy for Lazy attention);
  * sampled query rows in every (b, h) slice (oracle.rows.ada_rows);
  * the support set of sampled rows, read from the kernels themselves: with an upstream gradient
    that is one-hot in column c for query row i_c, dv[j, c] = p[i_c, j], so the keys where dv is
    non-zero are exactly the keys the kernels gave p > 0;
  * block-mask words of sampled query tiles, which the forward builds from its own support.
Support entries and mask bits must agree exactly except at near-ties: entries whose exact
distance |z - tau| to the oracle's threshold is within TIE_ULPS float32 ulps of
max(|z|, |tau|) (z = (alpha-1) * score).  The number of such entries is printed and bounded.

Tolerances: the north star's bf16 max-abs 2e-2, plus what the bf16 format itself imposes on any
bf16 implementation (the reference's Triton kernels cast p and dS to the input dtype before
tl.dot in the same way): one bf16 rounding of the output value (2^-8 relative) and the bound
of rounding the matrix-product operands p and dS to bf16 (oracle.rows, ``unit_round``
= 2^-8: u |p| |v| for out, u |dS| |k| scale for dq ...).  At alpha = 2 and L = 8192, |dS| reaches
~20, where that bound alone is ~0.03.  Lazy dbias / dtau (float32 sums over a whole head):
2e-2 * max(1, max|ref| / 4) plus the jump a near-tie can cause.

Configs: 2 = [4,12,1024,64] no-mask bidirectional forward; 3 = [2,16,8192,64]
causal fwd+bwd at alpha 1.5 and 2.0 (plus the sparse-support input of the bench, k = q);
4 = 8 sequences of seeded lengths in [512, 8192], H 12, causal and bidirectional;
5 = Lazy [2,8,4096,64] RoPE'd, bias [8,512] ~ N(0, 0.02), tau -1, W 512, and its 4-sequence
varlen variant; and a Lazy window beyond 1024 (bias read from global memory).
Reference test grid: tests/test_adasplash.py:63-122, tests/test_lazy_attention_triton_backward.py.
"""
import math

import numpy as np
import pytest
import torch

from _gpu_util import DEV, assert_close, banner, rope, ulp32
from oracle.lazy import lazy_backward, lazy_block_mask, lazy_forward, lazy_weights
from oracle.rows import ada_rows, ada_slice, mask_row_words

pytestmark = pytest.mark.gpu
TIE_ULPS = 8
ATOL = 2e-2


def _gen(shape, seed, n, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return [(torch.randn(*shape, generator=g) * scale).to(torch.bfloat16) for _ in range(n)]


def _np(t):
    return t.float().numpy().astype(np.float64)


def _gtol(ref):
    """Tolerance of a bf16 output tensor: 2e-2 plus one bf16 ulp (2^-8 relative) of each value --
    the output dtype cannot resolve gradients of magnitude 8 and up below 2e-2."""
    return ATOL + np.abs(ref) * 2.0 ** -8


def _stol(ref):
    """Tolerance of the float32 Lazy parameter gradients (sums over every row of a head)."""
    return ATOL * max(1.0, float(np.abs(ref).max()) / 4)


def _run_ada(q, k, v, do, alpha, causal, varlen=None, masked=True):
    """Forward + backward on the GPU; returns CPU tensors (out, tau, mask, dq, dk, dv)."""
    from adasplash import adasplash, adasplash_no_block_mask, adasplash_stats

    vl = None if varlen is None else torch.as_tensor(varlen, dtype=torch.int32).to(DEV)
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    op = adasplash if masked else adasplash_no_block_mask
    out = op(qd, kd, vd, alpha=alpha, niter=10, is_causal=causal, varlen=vl)
    out.backward(do.to(DEV))
    with torch.no_grad():
        out2, tau, mask = adasplash_stats(qd.detach(), kd.detach(), vd.detach(), alpha=alpha, is_causal=causal,
                                          varlen=vl, use_mask=masked)
    assert torch.equal(out.detach(), out2), "forward not bit-identical between calls"
    torch.cuda.synchronize()
    cpu = lambda t: None if t is None else t.detach().cpu()
    return {"out": cpu(out), "tau": cpu(tau), "mask": cpu(mask), "dq": cpu(qd.grad), "dk": cpu(kd.grad),
            "dv": cpu(vd.grad)}


class TieStats:
    """Support comparison: entries that differ must be near-ties; counts are printed."""

    def __init__(self, tag):
        self.tag, self.total, self.near, self.diff, self.maxdist = tag, 0, 0, 0, 0.0
        self.tiny = 0  # support entries whose p is below the input dtype's smallest value

    def window(self, z, tau):
        return _tie_window(z, tau)

    def compare(self, ours, z, tau, ok, tiny=None):
        dist = np.abs(z - tau[:, None])
        near = (dist <= self.window(z, tau)) & ok
        if tiny is not None:
            # fp16: p below 2^-24 rounds to zero when the kernels cast p to the input dtype for
            # the P V product (as the reference's Triton kernels do), so such an entry may read
            # as outside the support
            self.tiny += int((tiny & ok & ~near).sum())
            near = near | (tiny & ok)
        theirs = (z - tau[:, None] > 0) & ok
        bad = (ours != theirs) & ok
        self.total += int(ok.sum())
        self.near += int(near.sum())
        self.diff += int(bad.sum())
        if bad.any():
            self.maxdist = max(self.maxdist, float(dist[bad].max()))
        assert not (bad & ~near).any(), (
            f"{self.tag}: {int((bad & ~near).sum())} support entries differ away from near-ties "
            f"(max distance {float(dist[bad & ~near].max()):.3e})")

    def report(self, max_frac=1e-4):
        banner(f"{self.tag}: support entries compared {self.total}, near-ties (<= {TIE_ULPS} ulp) {self.near}, "
               f"differing {self.diff}, max distance of a differing entry {self.maxdist:.3e}"
               + (f", p below the dtype's range {self.tiny}" if self.tiny else ""))
        assert self.near <= max(4, max_frac * self.total), f"{self.tag}: too many near-ties excluded"


U_BF16 = 2.0 ** -8


def _tie_window(z, tau):
    return TIE_ULPS * ulp32(np.maximum(np.abs(z), np.abs(tau)[:, None]))


def _check_rows(tag, x, res, b, h, rows, alpha, causal, n, gq=None):
    """Sampled rows of slice (b, h): output, threshold, dq (dq within the tolerance plus the
    jump a near-tie entry can cause, oracle.rows.ada_rows)."""
    hk = h if gq is None else h // gq
    q, k, v, do = (_np(t[b, hh]) for t, hh in zip(x, (h, hk, hk, h)))
    r = ada_rows(q, k, v, do, rows, alpha, causal, n, tie_window=_tie_window, unit_round=U_BF16)
    assert_close(_np(res["out"][b, h][rows]), r["out"], ATOL, f"{tag} out rows (b={b}, h={h})")
    assert_close(_np(res["dq"][b, h][rows]), r["dq"], _gtol(r["dq"]) + r["dq_round"] + r["dq_slack"],
                 f"{tag} dq rows (b={b}, h={h})")
    t = res["tau"][b, h][rows].double().numpy()
    valid = r["row_valid"]
    assert np.isinf(t[~valid]).all()
    tv, rv = t[valid], r["tau"][valid]
    err = np.abs(tv - rv)
    lim = TIE_ULPS * ulp32(np.maximum(np.abs(rv), 1.0))
    assert (err <= lim).all(), f"{tag}: threshold error {err.max():.3e} > {TIE_ULPS} ulp (b={b}, h={h})"
    return r


def _check_slice(tag, x, res, b, h, alpha, causal, n):
    q, k, v, do = (_np(t[b, h]) for t in x)
    sl = ada_slice(q, k, v, do, alpha, causal, n, tie_window=_tie_window, unit_round=U_BF16)
    assert_close(_np(res["out"][b, h]), sl["out"], ATOL, f"{tag} slice out (b={b}, h={h})")
    slack = {"dq": sl["dq_slack"], "dk": sl["dk_slack"], "dv": 0.0}
    for nm in ("dq", "dk", "dv"):
        assert_close(_np(res[nm][b, h]), sl[nm], _gtol(sl[nm]) + sl[nm + "_round"] + slack[nm],
                     f"{tag} slice {nm} (b={b}, h={h})")
    # how much of the budget the kernels use
    worst = {nm: float(np.max(np.abs(_np(res[nm][b, h]) - sl[nm]) / (_gtol(sl[nm]) + sl[nm + "_round"] + slack[nm])))
             for nm in ("dq", "dk", "dv")}
    nties = int((sl["dq_slack"].max(-1) > 0).sum())
    t = res["tau"][b, h].double().numpy()
    fin = np.isfinite(sl["tau"])
    assert (np.isfinite(t) == fin).all()
    err = np.abs(t[fin] - sl["tau"][fin])
    assert (err <= TIE_ULPS * ulp32(np.maximum(np.abs(sl["tau"][fin]), 1.0))).all(), f"{tag} slice tau {err.max():.3e}"
    banner(f"{tag} slice (b={b},h={h}) ok: max|dk| {np.abs(sl['dk']).max():.2f}, max|dv| {np.abs(sl['dv']).max():.2f}, "
           f"rows with a near-tie gradient jump {nties}; max err / tol {worst}")


def _probe_rows(L, n, seed):
    g = np.random.default_rng(seed)
    fixed = [0, 1, 2, 63, 64, 127, 128, 129, 255, 256, n // 2, n - 2, n - 1]
    fixed = [r for r in fixed if 0 <= r < n]
    rest = g.choice(n, size=64 - len(set(fixed)), replace=False)
    return np.array(sorted(set(fixed) | set(rest.tolist())))[:64]


def _check_support_probe(tag, x, b, h, alpha, causal, varlen, rows, stats):
    """Kernel support of 64 rows of slice (b, h) read from dv under a one-hot dO."""
    from adasplash import adasplash

    q, k, v, _do = x
    B, H, L, D = q.shape
    assert len(rows) <= D
    dop = torch.zeros(B, H, L, D, dtype=q.dtype)
    dop[b, h, torch.as_tensor(rows), torch.arange(len(rows))] = 1.0
    vl = None if varlen is None else torch.as_tensor(varlen, dtype=torch.int32).to(DEV)
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    adasplash(qd, kd, vd, alpha=alpha, is_causal=causal, varlen=vl).backward(dop.to(DEV))
    dv = vd.grad[b, h].float().cpu().numpy().astype(np.float64)  # [L, D]
    n = L if varlen is None else int(varlen[b])
    r = ada_rows(_np(q[b, h]), _np(k[b, h]), _np(v[b, h]), None, rows, alpha, causal, n)
    pk = dv[:, : len(rows)].T  # [R, L] kernel p of each probed row
    ok = np.isfinite(r["z"])
    tiny = (r["p"] > 0) & (r["p"] < 2.0 ** -24) if q.dtype == torch.float16 else None
    stats.compare(pk != 0, r["z"], r["tau"], ok, tiny)
    # the probed p values themselves (bf16-rounded by dv's dtype)
    assert_close(pk, r["p"], 4e-3 * max(1.0, float(r["p"].max())), f"{tag} probed p rows")


def _check_mask_tiles(tag, x, res, b, h, tiles, alpha, causal, n, stats):
    q, k, v, _ = (_np(t[b, h]) for t in x)
    L = q.shape[0]
    got = res["mask"][b, h].numpy().view(np.uint32)
    for tr in tiles:
        rows = np.arange(tr * 128, min(L, tr * 128 + 128))
        r = ada_rows(q, k, v, None, rows, alpha, causal, n)
        want = mask_row_words(r["p"])
        if np.array_equal(got[tr], want):
            continue
        # a differing bit must come from a key tile holding a near-tie of the support
        diff = np.unpackbits((got[tr] ^ want).view(np.uint8), bitorder="little")
        ok = np.isfinite(r["z"])
        near = (np.abs(r["z"] - r["tau"][:, None]) <= stats.window(r["z"], r["tau"])) & ok
        tc = -(-L // 64)
        pad = np.zeros((len(rows), tc * 64), dtype=bool)
        pad[:, :L] = near
        near_t = pad.reshape(len(rows), tc, 64).any(axis=(0, 2))
        for c in np.nonzero(diff[:tc])[0]:
            assert near_t[c], f"{tag}: mask bit (b={b}, h={h}, r={tr}, c={c}) differs away from near-ties"
            stats.near_mask = getattr(stats, "near_mask", 0) + 1


# ---------------------------------------------------------------------------------------------
# config 3: [2, 16, 8192, 64] causal, block-masked, alpha 1.5 / 2.0 -- the bench's own inputs


def _cfg3_inputs():
    g = torch.Generator(device="cpu").manual_seed(0)  # bench.py's generator and order
    return [torch.randn(2, 16, 8192, 64, generator=g).to(torch.bfloat16) for _ in range(4)]


@pytest.mark.parametrize("alpha", [1.5, 2.0])
def test_config3_causal_L8192(alpha):
    banner("config 3 full size", alpha)
    x = _cfg3_inputs()
    res = _run_ada(*x, alpha=alpha, causal=True)
    B, H, L, D = x[0].shape
    stats = TieStats(f"cfg3 a={alpha}")
    _check_slice("cfg3", x, res, 0, 0, alpha, True, L)
    _check_slice("cfg3", x, res, 1, 15, alpha, True, L)
    g = np.random.default_rng(5)
    for b in range(B):
        for h in range(H):
            rows = np.unique(np.concatenate([[L - 1], g.choice(L, 15, replace=False)]))
            _check_rows("cfg3", x, res, b, h, rows, alpha, True, L)
    _check_mask_tiles("cfg3", x, res, 0, 0, [0, 1, 31, 63], alpha, True, L, stats)
    _check_mask_tiles("cfg3", x, res, 1, 7, [62, 63], alpha, True, L, stats)
    _check_support_probe("cfg3", x, 0, 3, alpha, True, None, _probe_rows(L, L, 1), stats)
    stats.report()


def test_config3_sparse_support_mask():
    """The bench's block-skipping input (k = q ~ N(0, 1.5^2), alpha 2): most tiles are empty,
    so the mask bits carry real structure; checked on whole query tiles."""
    banner("config 3 sparse-support input")
    g = torch.Generator(device="cpu").manual_seed(1)
    q = (torch.randn(2, 16, 8192, 64, generator=g) * 1.5).to(torch.bfloat16)
    v, do = (torch.randn(2, 16, 8192, 64, generator=g).to(torch.bfloat16) for _ in range(2))
    x = [q, q, v, do]
    res = _run_ada(*x, alpha=2.0, causal=True)
    L = 8192
    stats = TieStats("cfg3 sparse")
    m = res["mask"].numpy().view(np.uint32)
    density = np.unpackbits(m.view(np.uint8)).sum() / (2 * 16 * sum(min(128, 2 * (r + 1)) for r in range(64)))
    banner(f"sparse input block density {density:.4f}")
    assert density < 0.2
    _check_mask_tiles("cfg3 sparse", x, res, 0, 0, list(range(0, 64, 7)) + [63], 2.0, True, L, stats)
    _check_mask_tiles("cfg3 sparse", x, res, 1, 11, [5, 40, 63], 2.0, True, L, stats)
    _check_slice("cfg3 sparse", x, res, 0, 0, 2.0, True, L)
    g2 = np.random.default_rng(6)
    for b in range(2):
        for h in range(0, 16, 3):
            _check_rows("cfg3 sparse", x, res, b, h, np.sort(g2.choice(L, 8, replace=False)), 2.0, True, L)
    _check_support_probe("cfg3 sparse", x, 1, 2, 2.0, True, None, _probe_rows(L, L, 2), stats)
    stats.report()


@pytest.mark.parametrize("alpha", [1.5, 2.0])
def test_long_sequence_L32768(alpha):
    """Beyond the BASELINE sizes: 32768 keys per row (16-word mask rows, 256 row tiles, lists
    tightened many times per row), causal, on sampled rows, late mask tiles and a support probe."""
    banner("long sequence L=32768", alpha)
    B, H, L, D = 1, 2, 32768, 64
    x = _gen((B, H, L, D), 77, 4)
    res = _run_ada(*x, alpha=alpha, causal=True)
    stats = TieStats(f"L32768 a={alpha}")
    g = np.random.default_rng(8)
    for h in range(H):
        rows = np.unique(np.concatenate([[0, 1, 8191, 8192, L - 129, L - 1], g.choice(L, 10, replace=False)]))
        _check_rows("L32768", x, res, 0, h, rows, alpha, True, L)
    _check_mask_tiles("L32768", x, res, 0, 1, [100, 255], alpha, True, L, stats)
    _check_support_probe("L32768", x, 0, 0, alpha, True, None, _probe_rows(L, L, 4), stats)
    stats.report()


@pytest.mark.parametrize("alpha", [1.5, 2.0])
def test_fp16_L8192(alpha):
    """fp16 inputs at the headline length (the fp16 MFMA path), on sampled rows, mask tiles and a
    support probe; tolerances as for bf16 (fp16 rounds finer)."""
    banner("fp16 L=8192", alpha)
    g = torch.Generator().manual_seed(91)
    x = [torch.randn(1, 4, 8192, 64, generator=g).to(torch.float16) for _ in range(4)]
    res = _run_ada(*x, alpha=alpha, causal=True)
    L = 8192
    stats = TieStats(f"fp16 a={alpha}")
    rg = np.random.default_rng(9)
    for h in range(4):
        rows = np.unique(np.concatenate([[0, L - 1], rg.choice(L, 10, replace=False)]))
        _check_rows("fp16", x, res, 0, h, rows, alpha, True, L)
    _check_mask_tiles("fp16", x, res, 0, 2, [0, 40, 63], alpha, True, L, stats)
    _check_support_probe("fp16", x, 0, 1, alpha, True, None, _probe_rows(L, L, 5), stats)
    stats.report()


# ---------------------------------------------------------------------------------------------
# config 4: varlen, 8 sequences of seeded lengths in [512, 8192], H 12


@pytest.mark.parametrize("causal", [True, False])
def test_config4_varlen(causal):
    banner("config 4 varlen", causal)
    lens = torch.randint(512, 8193, (8,), generator=torch.Generator().manual_seed(0)).numpy()
    B, H, L, D = 8, 12, 8192, 64
    x = _gen((B, H, L, D), 40, 4)
    res = _run_ada(*x, alpha=1.5, causal=causal, varlen=lens)
    stats = TieStats(f"cfg4 causal={causal}")
    for nm in ("out", "dq", "dk", "dv"):
        for b in range(B):
            assert (res[nm][b, :, int(lens[b]):] == 0).all(), f"{nm} padded rows not zero (b={b})"
    bs, bl = int(np.argmin(lens)), int(np.argmax(lens))
    _check_slice("cfg4", x, res, bs, 2, 1.5, causal, int(lens[bs]))
    _check_slice("cfg4", x, res, bl, 9, 1.5, causal, int(lens[bl]))
    g = np.random.default_rng(7)
    for b in range(B):
        n = int(lens[b])
        for h in (b % H, (b + 5) % H):
            rows = np.unique(np.concatenate([[0, n - 1, min(n, L - 1)], g.choice(n, 12, replace=False)]))
            _check_rows("cfg4", x, res, b, h, rows, 1.5, causal, n)
        _check_mask_tiles("cfg4", x, res, b, b % H, [(n - 1) // 128], 1.5, causal, n, stats)
    _check_support_probe("cfg4", x, bl, 4, 1.5, causal, lens, _probe_rows(L, int(lens[bl]), 3), stats)
    stats.report()


# ---------------------------------------------------------------------------------------------
# config 2: adasplash_no_block_mask forward, [4, 12, 1024, 64], bidirectional


def test_config2_nomask_forward():
    from adasplash import adasplash_no_block_mask, adasplash_stats

    banner("config 2")
    B, H, L, D = 4, 12, 1024, 64
    q, k, v = _gen((B, H, L, D), 50, 3)
    with torch.no_grad():
        out = adasplash_no_block_mask(q.to(DEV), k.to(DEV), v.to(DEV), alpha=1.5, niter=10, is_causal=False).cpu()
        _o, tau, _m = adasplash_stats(q.to(DEV), k.to(DEV), v.to(DEV), alpha=1.5, use_mask=False)
    tau = tau.cpu()
    for b in range(B):
        for h in range(H):
            rows = np.arange(L) if (b * H + h) % 8 == 0 else np.arange(0, L, 37)
            r = ada_rows(_np(q[b, h]), _np(k[b, h]), _np(v[b, h]), None, rows, 1.5, False, L)
            assert_close(_np(out[b, h][rows]), r["out"], ATOL, f"cfg2 out (b={b}, h={h})")
            err = np.abs(tau[b, h][rows].double().numpy() - r["tau"])
            assert (err <= TIE_ULPS * ulp32(np.maximum(np.abs(r["tau"]), 1.0))).all()


# ---------------------------------------------------------------------------------------------
# config 5: Lazy attention [2, 8, 4096, 64], RoPE'd, bias [8, 512] ~ N(0, 0.02), tau -1, W 512


def _lazy_inputs(B, seed):
    H, L, D, W = 8, 4096, 64, 512
    q, k, v, do = _gen((B, H, L, D), seed, 4)
    q, k = rope(q), rope(k)
    g = torch.Generator().manual_seed(seed + 100)
    bias = torch.randn(H, W, generator=g) * 0.02
    tau = torch.full((H,), -1.0)
    return q, k, v, do, bias, tau, W


def _run_lazy(q, k, v, do, bias, tau, W, varlen=None):
    from adasplash import lazy_attention_triton

    vl = None if varlen is None else torch.as_tensor(varlen, dtype=torch.int32).to(DEV)
    ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v, bias, tau)]
    out = lazy_attention_triton(*ts, window_size=W, varlen=vl)
    out.backward(do.to(DEV))
    with torch.no_grad():
        outm, bm = lazy_attention_triton(*[t.detach() for t in ts], window_size=W, varlen=vl, return_mask=True)
    assert torch.equal(outm, out.detach()), "block-sparse forward differs from the dense forward"
    return [out.detach().cpu()] + [t.grad.cpu() for t in ts] + [bm.cpu()]


def _check_lazy_heads(tag, inp, got, heads, varlen=None):
    q, k, v, do, bias, tau, W = inp
    out, dq, dk, dv, dbias, dtau, bm = got
    B, H, L, _ = q.shape
    ties = 0
    for h in heads:
        sl = lambda t: _np(t[:, h:h + 1])
        bh, th = _np(bias[h:h + 1]), _np(tau[h:h + 1])
        ref_out = lazy_forward(sl(q), sl(k), sl(v), bh, th, W, varlen)
        assert_close(_np(out[:, h:h + 1]), ref_out, ATOL, f"{tag} out (h={h})")
        rdq, rdk, rdv, rdb, rdt = lazy_backward(sl(q), sl(k), sl(v), bh, th, sl(do), W, varlen)
        for nm, g_, r in (("dq", dq, rdq), ("dk", dk, rdk), ("dv", dv, rdv)):
            assert_close(_np(g_[:, h:h + 1]), r, _gtol(r), f"{tag} {nm} (h={h})")
        # near-ties: p + tau/(i+1) within a relative 1e-5 of tau/(i+1).  m = 1[p + tau/(i+1) > 0]
        # may land on either side there; a flip moves dtau by dP/(i+1) and dbias by at most
        # 2 |p dP|.  Exact ties (margin 0: tau = -1 on row 0, p = 1) are not excused: the kernels
        # compute p = 1 exactly there and must decide as exact arithmetic does.
        e, margin = lazy_weights(sl(q), sl(k), bh, th, W, varlen)
        thr = np.abs(th[0]) / np.arange(1, L + 1)[None, None, :, None]
        tie = (margin <= 1e-5 * thr) & (margin > 0)
        tb, _th, ti, tj = np.nonzero(tie)
        dPt = np.einsum("nd,nd->n", _np(do[tb, h, ti]), _np(v[tb, h, tj]))
        pt = np.abs(th[0]) / (ti + 1)  # p at a tie
        dtau_slack = float(np.sum(np.abs(dPt) / (ti + 1)))
        dbias_slack = float(np.sum(2 * pt * np.abs(dPt)))
        assert_close(dbias[h].double().numpy(), rdb[0], _stol(rdb) + dbias_slack, f"{tag} dbias (h={h})")
        assert_close(np.atleast_1d(dtau[h].double().numpy()), rdt, _stol(rdt) + dtau_slack, f"{tag} dtau (h={h})")
        # 64x64 block mask: exact away from the near-ties
        sure = lazy_block_mask(np.where(tie, 0.0, e))
        maybe = lazy_block_mask(np.where(tie, 1.0, e))
        gm = bm[:, h:h + 1].numpy()
        assert (gm >= sure).all() and (gm <= maybe).all(), f"{tag}: lazy block mask differs (h={h})"
        ties += int((sure != maybe).sum())
        banner(f"{tag} h={h}: max|dbias| {np.abs(rdb).max():.3f}, dtau {rdt[0]:.3f} (kernel {float(dtau[h]):.3f}, "
               f"tie slack {dtau_slack:.3f}), "
               f"mask blocks decided by a near-tie {int((sure != maybe).sum())}, near-tie entries {int(tie.sum())}")
    return ties


def test_config5_lazy():
    banner("config 5 lazy")
    inp = _lazy_inputs(2, 60)
    got = _run_lazy(*inp)
    _check_lazy_heads("cfg5", inp, got, [0, 5])


def test_config5_lazy_varlen():
    banner("config 5 lazy varlen")
    inp = _lazy_inputs(4, 70)
    lens = torch.randint(512, 4097, (4,), generator=torch.Generator().manual_seed(1)).numpy()
    got = _run_lazy(*inp, varlen=lens)
    for nm, t in zip(("out", "dq", "dk", "dv"), got[:4]):
        for b in range(4):
            assert (t[b, :, int(lens[b]):] == 0).all(), f"{nm} padded rows (b={b})"
    _check_lazy_heads("cfg5 varlen", inp, got, [3], lens)


@pytest.mark.parametrize("tauval", [-1.0, 0.3])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_lazy_window_beyond_lds(tauval, dtype):
    """Bias window W = 1500 > 1024: bias read from global memory in every sweep, dbias
    accumulated in global memory (entries d >= 1024 included)."""
    from adasplash import lazy_attention_triton

    banner("lazy W=1500", tauval, dtype)
    B, H, L, D, W = 1, 1, 2048, 64, 1500
    g = torch.Generator().manual_seed(80)
    q, k, v, do = ((torch.randn(B, H, L, D, generator=g)).to(dtype) for _ in range(4))
    bias = torch.randn(H, W, generator=g) * 0.5
    tau = torch.full((H,), tauval)
    ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v, bias, tau)]
    out = lazy_attention_triton(*ts, window_size=W)
    out.backward(do.to(DEV))
    a = [_np(t) for t in (q, k, v)]
    ref_out = lazy_forward(*a, _np(bias), _np(tau), W)
    ref = lazy_backward(*a, _np(bias), _np(tau), _np(do), W)
    lowp = dtype != torch.float32
    assert_close(_np(out.detach().cpu()), ref_out, ATOL if lowp else 1e-5, "out")
    for t, r, nm in zip(ts, ref, ("dq", "dk", "dv", "dbias", "dtau")):
        if lowp:
            tol = _stol(r) if nm in ("dbias", "dtau") else _gtol(r)
        else:
            tol = 1e-4 * max(1.0, float(np.abs(r).max()))
        assert_close(_np(t.grad.cpu()), r, tol, nm)
    # the far end of the window (d >= 1024) must carry gradient
    assert np.abs(ref[3][0, 1024:]).max() > 0
