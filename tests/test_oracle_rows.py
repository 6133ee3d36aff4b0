"""The row-sampled / row-chunked oracle (oracle.rows) against the whole-matrix oracle
(oracle.adasplash, pinned by closed forms, brute force and autograd) and against the sort-based
closed forms of alpha-entmax.  CPU only."""
import numpy as np
import pytest

from oracle.adasplash import block_mask, pack_block_mask, reference_attention, reference_attention_backward
from oracle.entmax import entmax15_sort, sparsemax_sort
from oracle.rows import ada_rows, ada_slice, entmax_tau_topk, mask_row_words


@pytest.mark.parametrize("alpha,closed", [(1.5, entmax15_sort), (2.0, sparsemax_sort)])
def test_topk_threshold_matches_closed_form(alpha, closed):
    rng = np.random.default_rng(0)
    # kmax below the row length exercises the partition path; scale 3 gives small supports,
    # scale 0.05 supports larger than kmax (the whole-row fallback)
    for scale in (3.0, 0.05):
        x = rng.standard_normal((40, 3000)) * scale
        tau = entmax_tau_topk((alpha - 1) * x, alpha, kmax=200)
        p = np.maximum((alpha - 1) * x - tau[:, None], 0) ** (1 / (alpha - 1))
        np.testing.assert_allclose(p, closed(x), atol=1e-12)


@pytest.mark.parametrize("alpha", [1.5, 2.0, 1.333])
@pytest.mark.parametrize("is_causal", [True, False])
def test_rows_and_slice_match_full_oracle(alpha, is_causal):
    rng = np.random.default_rng(1)
    B, H, L, D = 2, 1, 300, 32
    q, k, v, do = (rng.standard_normal((B, H, L, D)) for _ in range(4))
    varlen = np.array([300, 211])
    out, aux = reference_attention(q, k, v, alpha, varlen, is_causal, return_aux=True)
    dq, dk, dv = reference_attention_backward(q, k, v, do, alpha, varlen, is_causal)
    for b in range(B):
        n = int(varlen[b])
        sl = ada_slice(q[b, 0], k[b, 0], v[b, 0], do[b, 0], alpha, is_causal, n, chunk=64)
        np.testing.assert_allclose(sl["out"], out[b, 0], atol=1e-10)
        np.testing.assert_allclose(sl["dq"], dq[b, 0], atol=1e-9)
        np.testing.assert_allclose(sl["dk"], dk[b, 0], atol=1e-9)
        np.testing.assert_allclose(sl["dv"], dv[b, 0], atol=1e-9)
        t = aux["tau"][b, 0][:n]
        np.testing.assert_allclose(sl["tau"][:n], t, atol=1e-12)
        assert np.isinf(sl["tau"][n:]).all()
        rows = np.array([0, 1, 127, 128, 250, 299])
        r = ada_rows(q[b, 0], k[b, 0], v[b, 0], do[b, 0], rows, alpha, is_causal, n)
        np.testing.assert_array_equal(r["p"] > 0, aux["p"][b, 0][rows] > 0)
        # mask words of the first query tile
        rt = ada_rows(q[b, 0], k[b, 0], v[b, 0], None, np.arange(128), alpha, is_causal, n)
        want = pack_block_mask(block_mask(aux["p"][b:b + 1], aux["row_valid"][b:b + 1]))[0, 0, 0]
        np.testing.assert_array_equal(mask_row_words(rt["p"]), want)


@pytest.mark.parametrize("alpha", [2.0, 1.5])
def test_tie_flip_matches_perturbed_inputs(alpha):
    """ds_flip / dq_slack of a near-tie equal the whole-matrix oracle's gradient with that entry
    pushed just across the threshold (at alpha = 2 U jumps there from 0 to 1, below 2 it does not)."""
    rng = np.random.default_rng(3)
    L, D, i = 64, 16, 5
    q, k, v, do = (rng.standard_normal((1, 1, L, D)) for _ in range(4))
    sc = 1 / np.sqrt(D)
    r0 = ada_rows(q[0, 0], k[0, 0], v[0, 0], do[0, 0], [i], alpha, False, L)
    z, tau = r0["z"][0], r0["tau"][0]
    j = int(np.argmax(np.where(z < tau, z, -np.inf)))  # the largest entry outside the support
    qi = q[0, 0, i]

    def moved(eps):
        kk = k.copy()
        target = (tau + eps) / (alpha - 1)  # score that puts z_ij at tau + eps
        kk[0, 0, j] += (target - kk[0, 0, j] @ qi * sc) / (qi @ qi * sc) * qi
        return kk

    kp, km = moved(1e-10), moved(-1e-10)
    r = ada_rows(q[0, 0], kp[0, 0], v[0, 0], do[0, 0], [i], alpha, False, L,
                 tie_window=lambda zz, tt: np.full(zz.shape, 1e-8))
    assert r["near"][0, j] and r["near"].sum() == 1 and r["p"][0, j] > 0
    dq_plus = reference_attention_backward(q, kp, v, do, alpha)[0][0, 0, i]
    dq_minus = reference_attention_backward(q, km, v, do, alpha)[0][0, 0, i]
    np.testing.assert_allclose(r["dq"][0], dq_plus, atol=1e-6)
    np.testing.assert_allclose(r["ds_flip"][0] @ kp[0, 0] * sc, dq_minus, atol=1e-6)
    np.testing.assert_allclose(r["dq_slack"][0], np.abs(dq_plus - dq_minus), atol=1e-6)
    if alpha == 2.0:
        assert np.abs(dq_plus - dq_minus).max() > 1e-2  # the jump is real


def test_unit_round_bounds_bf16_operand_rounding():
    """out_round / dq_round bound the error of rounding p and dS to bf16 before the products."""
    import torch

    rng = np.random.default_rng(4)
    L, D = 512, 64
    q, k, v, do = (rng.standard_normal((L, D)) for _ in range(4))
    rows = np.arange(0, L, 7)
    r = ada_rows(q, k, v, do, rows, 2.0, True, L, unit_round=2.0 ** -8)
    bf = lambda a: torch.tensor(a).to(torch.bfloat16).double().numpy()
    assert (np.abs(bf(r["p"]) @ v - r["out"]) <= r["out_round"] + 1e-12).all()
    assert (np.abs(bf(r["ds"]) @ k / 8 - r["dq"]) <= r["dq_round"] + 1e-12).all()
    assert r["dq_round"].max() > 0


@pytest.mark.parametrize("alpha", [1.5, 2.0])
def test_torch_cpu_path_matches_oracle(alpha):
    """oracle.torch_cpu (the float32 torch path bench.py times as the CPU baseline) against the
    float64 oracle: rows 0..L-1 in two blocks, causal."""
    import torch

    from oracle.torch_cpu import attention_rows

    rng = np.random.default_rng(9)
    L, D = 200, 32
    q, k, v, do = (rng.standard_normal((1, 1, L, D)) for _ in range(4))
    out = reference_attention(q, k, v, alpha, None, True)
    dq, dk, dv = reference_attention_backward(q, k, v, do, alpha, None, True)
    t = [torch.tensor(a[0, 0], dtype=torch.float32) for a in (q, k, v, do)]
    acc = [np.zeros((L, D)) for _ in range(4)]
    for rows in (np.arange(0, 120), np.arange(120, L)):
        o, gq, gk, gv = attention_rows(*t, rows, alpha)
        acc[0][rows] = o.numpy()
        acc[1][rows] = gq.numpy()
        acc[2] += gk.numpy()
        acc[3] += gv.numpy()
    for got, ref in zip(acc, (out[0, 0], dq[0, 0], dk[0, 0], dv[0, 0])):
        np.testing.assert_allclose(got, ref, atol=2e-4)
