"""Pins of the indexer-KL oracle restatement (CPU).

The indexer KL has no upstream kernel (docs/msa_training_flow.md:92-138 defines
it; docs/implementation_plan.md:66-69 leaves it unimplemented), so the oracle is
pinned by what the mathematics fixes: a zero loss when the student equals the
teacher, a two-key closed form, finite differences of its own loss, and torch
float64 autograd of an independently written dense formulation (masked
log-softmax, head-mean teacher, xlogy).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import msa_oracle as O
from tests.helpers import cu_list, random_selection


def _inputs(lengths, groups, ratio, dim, dim_i, block, topk, seed):
    rng = np.random.default_rng(seed)
    total = sum(lengths)
    iq = rng.standard_normal((total, groups, dim_i))
    ik = rng.standard_normal((total, 1, dim_i))
    q = rng.standard_normal((total, groups * ratio, dim))
    k = rng.standard_normal((total, groups, dim))
    ids = random_selection(total, groups, topk, lengths, block, 1, torch.Generator().manual_seed(seed)).numpy()
    return iq, ik, q, k, ids, np.array(cu_list(lengths), dtype=np.int32)


def _torch_dense(iq, ik, q, k, ids, cu, block, index_scale, scale):
    """Independent dense formulation: loss and (d_iq, d_ik) by float64 autograd."""
    iq_t = torch.tensor(iq, requires_grad=True)
    ik_t = torch.tensor(ik, requires_grad=True)
    q_t, k_t = torch.tensor(q), torch.tensor(k)
    total, groups, _ = iq.shape
    ratio = q.shape[1] // groups
    loss = torch.zeros((), dtype=torch.float64)
    for a, b in zip(cu[:-1], cu[1:]):
        n = int(b - a)
        if n == 0:
            continue
        pos = torch.arange(n)
        for g in range(groups):
            sel = torch.zeros(n, n, dtype=torch.bool)
            for t in range(n):
                for blk in ids[a + t, g]:
                    if 0 <= blk <= t // block:
                        sel[t, blk * block: min((blk + 1) * block, n)] = True
            mask = sel & (pos[None, :] <= pos[:, None])
            has = mask.any(-1)
            z = index_scale * iq_t[a:b, g] @ ik_t[a:b, 0].T
            log_s = torch.log_softmax(z.masked_fill(~mask, -math.inf), -1)
            att = scale * torch.einsum("trd,kd->trk", q_t[a:b, g * ratio:(g + 1) * ratio], k_t[a:b, g])
            teacher = torch.softmax(att.masked_fill(~mask[:, None, :], -math.inf), -1).mean(1)
            terms = torch.xlogy(teacher, teacher) - teacher * log_s.masked_fill(~mask, 0.0)
            loss = loss + terms[has].sum()
    loss = loss / (total * groups)
    loss.backward()
    return loss.item(), iq_t.grad.numpy(), ik_t.grad.numpy()


@pytest.mark.parametrize("lengths,groups,ratio,dim,dim_i,block,topk,index_scale,scale", [
    ([9], 1, 1, 4, 3, 4, 2, 1.0, 0.5),
    ([13, 6], 2, 3, 5, 4, 4, 2, 0.7, None),
    ([0, 11, 3], 2, 2, 6, 5, 3, 3, 1.3, 0.4),
])
def test_matches_torch_autograd_of_dense_formulation(lengths, groups, ratio, dim, dim_i, block, topk, index_scale,
                                                    scale):
    iq, ik, q, k, ids, cu = _inputs(lengths, groups, ratio, dim, dim_i, block, topk, 7)
    res = O.indexer_kl(iq, ik, q, k, ids, cu, block_size=block, index_scale=index_scale, scale=scale)
    sc = dim ** -0.5 if scale is None else scale
    loss, d_iq, d_ik = _torch_dense(iq, ik, q, k, ids, cu, block, index_scale, sc)
    assert res["loss"] == pytest.approx(loss, rel=1e-12, abs=1e-14)
    np.testing.assert_allclose(res["d_iq"], d_iq, rtol=1e-10, atol=1e-14)
    np.testing.assert_allclose(res["d_ik"], d_ik, rtol=1e-10, atol=1e-14)
    assert (res["row_kl"] >= -1e-15).all()


def test_zero_when_student_equals_teacher():
    """One head per group, q = iq and k = ik, equal scales: teacher == student."""
    lengths, groups, block, topk = [10, 7], 2, 3, 2
    rng = np.random.default_rng(3)
    total = sum(lengths)
    iq = rng.standard_normal((total, groups, 6))
    ik = rng.standard_normal((total, 1, 6))
    k = np.repeat(ik, groups, axis=1)
    ids = random_selection(total, groups, topk, lengths, block, 1, torch.Generator().manual_seed(3)).numpy()
    cu = np.array(cu_list(lengths), dtype=np.int32)
    res = O.indexer_kl(iq, ik, iq.copy(), k, ids, cu, block_size=block, index_scale=0.8, scale=0.8)
    assert abs(res["loss"]) < 1e-15
    assert np.abs(res["d_iq"]).max() < 1e-15 and np.abs(res["d_ik"]).max() < 1e-15


def test_two_key_closed_form():
    """Token 1 sees keys 0 and 1: KL = t log(t/s) + (1-t) log((1-t)/(1-s)); token 0 sees one key (KL 0)."""
    iq = np.array([[[0.3]], [[1.2]]])
    ik = np.array([[[0.5]], [[-0.25]]])
    q = np.array([[[1.0]], [[-0.8]]])
    k = np.array([[[0.4]], [[1.1]]])
    ids = np.zeros((2, 1, 1), dtype=np.int64)
    res = O.indexer_kl(iq, ik, q, k, ids, [0, 2], block_size=2, index_scale=1.5, scale=0.9)
    z = 1.5 * 1.2 * np.array([0.5, -0.25])
    a = 0.9 * -0.8 * np.array([0.4, 1.1])
    s = np.exp(z[0]) / np.exp(z).sum()
    t = np.exp(a[0]) / np.exp(a).sum()
    kl = t * np.log(t / s) + (1 - t) * np.log((1 - t) / (1 - s))
    assert res["row_kl"][0, 0] == 0.0
    assert res["row_kl"][1, 0] == pytest.approx(kl, rel=1e-13)
    assert res["loss"] == pytest.approx(kl / 2, rel=1e-13)
    # dLoss/dz = (S - T) / 2, dz/d iq[1] = 1.5 * ik
    dz = (np.array([s, 1 - s]) - np.array([t, 1 - t])) / 2
    assert res["d_iq"][1, 0, 0] == pytest.approx(1.5 * (dz @ ik[:, 0, 0]), rel=1e-12)


def test_finite_differences():
    iq, ik, q, k, ids, cu = _inputs([8, 5], 2, 2, 3, 3, 3, 2, 11)
    res = O.indexer_kl(iq, ik, q, k, ids, cu, block_size=3, index_scale=1.1, scale=0.6)
    h = 1e-6
    for arr, grad, idx in ((iq, res["d_iq"], (6, 1, 2)), (ik, res["d_ik"], (4, 0, 1)), (iq, res["d_iq"], (12, 0, 0))):
        plus, minus = arr.copy(), arr.copy()
        plus[idx] += h
        minus[idx] -= h
        args = lambda x: (x, ik, q, k) if arr is iq else (iq, x, q, k)  # noqa: E731
        lp = O.indexer_kl(*args(plus), ids, cu, block_size=3, index_scale=1.1, scale=0.6)["loss"]
        lm = O.indexer_kl(*args(minus), ids, cu, block_size=3, index_scale=1.1, scale=0.6)["loss"]
        assert grad[idx] == pytest.approx((lp - lm) / (2 * h), rel=1e-6, abs=1e-10)


def test_row_and_key_subsets_match_full():
    iq, ik, q, k, ids, cu = _inputs([12, 9], 2, 2, 4, 4, 4, 2, 5)
    full = O.indexer_kl(iq, ik, q, k, ids, cu, block_size=4, index_scale=0.9, scale=0.7)
    tokens = [0, 3, 11, 12, 20]
    rows = O.indexer_kl_rows(iq, ik, q, k, ids, cu, tokens, block_size=4, index_scale=0.9, scale=0.7)
    np.testing.assert_allclose(rows["row_kl"], full["row_kl"][tokens], rtol=1e-13, atol=1e-16)
    np.testing.assert_allclose(rows["d_iq"], full["d_iq"][tokens], rtol=1e-13, atol=1e-16)
    keys = [0, 5, 11, 13, 20]
    d_ik = O.indexer_kl_key_rows(iq, ik, q, k, ids, cu, keys, block_size=4, index_scale=0.9, scale=0.7)
    np.testing.assert_allclose(d_ik, full["d_ik"][keys, 0], rtol=1e-12, atol=1e-16)
