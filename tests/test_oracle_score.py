"""Pin the stage-1 oracle (oracle.msa_oracle.index_score / index_score_backward).

Checks: the reference's known answers (tests/test_eager.py:143-152,
tests/test_triton_score.py:111-182, docs/code_review_response.md:33-41), exact
rational brute force for the public fp32 rounding, and torch float64 autograd
of an independently written amax formulation for the subgradient.
"""

from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import msa_oracle as O
from tests.helpers import cu_list


def _grads(q, k, cu, max_seqlen, block_size, scale, upstream):
    dq, dk = O.index_score_backward(q, k, cu, max_seqlen, upstream, block_size=block_size, scale=scale)
    return dq, dk


def test_ties_split_gradient_and_future_mask_is_zero():
    # tests/test_eager.py:143-152
    q = np.ones((3, 1, 1))
    k = np.ones((3, 1, 1))
    cu = [0, 3]
    s64, s32, tie = O.index_score(q, k, cu, 4, block_size=4)
    assert s32.shape == (3, 1, 1)
    ds = np.zeros((3, 1, 1))
    ds[-1] = 1.0
    dq, dk = _grads(q, k, cu, 4, 4, 1.0, ds)
    np.testing.assert_array_equal(dq[:, 0, 0], [0.0, 0.0, 1.0])
    np.testing.assert_allclose(dk[:, 0, 0], [1 / 3] * 3, rtol=0, atol=1e-15)
    assert tie[-1, 0, 0] == -3 and tie[0, 0, 0] == 1
    ds = np.zeros((3, 1, 1))
    ds[0] = 1.0
    _, dk = _grads(q, k, cu, 4, 4, 1.0, ds)
    np.testing.assert_array_equal(dk[:, 0, 0], [1.0, 0.0, 0.0])


@pytest.mark.parametrize("exact_tie", [False, True])
def test_cancellation_known_answers(exact_tie):
    # docs/code_review_response.md:26-41: score[1] = 2^-24 with a unique winner,
    # dQ[1] = [1, 2^-12, -1], dK[0] = [1, 2^-12, 1]; with k1 = [0, 2^-12, 0] an exact tie.
    small = 2.0**-12
    q = np.array([[[1.0, small, 1.0]], [[1.0, small, 1.0]]])
    k1 = [0.0, small, 0.0] if exact_tie else [0.0, 0.0, 0.0]
    k = np.array([[[1.0, small, -1.0]], [k1]])
    s64, s32, tie = O.index_score(q, k, [0, 2], 2, block_size=2)
    if exact_tie:
        assert s32[1, 0, 0] == np.float32(2.0**-24) and tie[1, 0, 0] == -2
    else:
        assert s32[1, 0, 0] == np.float32(5.960464477539063e-08) and tie[1, 0, 0] == 1
    ds = np.zeros((2, 1, 1))
    ds[1] = 1.0
    dq, dk = _grads(q, k, [0, 2], 2, 2, 1.0, ds)
    if exact_tie:
        np.testing.assert_array_equal(dq[1, 0], [0.5, 0.5 * small + 0.5 * small, -0.5])
        np.testing.assert_array_equal(dk[:, 0], [[0.5, 0.5 * small, 0.5], [0.5, 0.5 * small, 0.5]])
    else:
        np.testing.assert_array_equal(dq[1, 0], [1.0, small, -1.0])
        np.testing.assert_array_equal(dk[:, 0], [[1.0, small, 1.0], [0.0, 0.0, 0.0]])


def test_rounded_score_tie_has_unique_exact_winner():
    # tests/test_triton_score.py:145-146: both public scores round to 1.0 in fp32,
    # the exact winner is unique (key0).
    q = np.array([[[1.0, 1.0]], [[1.0, 1.0]]])
    k = np.array([[[1.0, 2.0**-24]], [[1.0, 0.0]]])
    _, s32, tie = O.index_score(q, k, [0, 2], 2, block_size=2)
    assert s32[1, 0, 0] == np.float32(1.0) and tie[1, 0, 0] == 1


def test_groups_remain_independent():
    # tests/test_triton_score.py:111-120
    q = np.array([[[1.0, 0.0], [0.0, 1.0]]] * 4)
    k = np.array([[[9.0, 1.0]], [[1.0, 8.0]], [[0.0, 0.0]], [[0.0, 0.0]]])
    _, s32, _ = O.index_score(q, k, [0, 4], 4, block_size=1)
    assert s32.shape == (4, 2, 4)
    assert s32[-1, 0].argmax() == 0 and s32[-1, 1].argmax() == 1


@pytest.mark.parametrize("scale", [1.0, -1.0, 0.0, 0.3, -1.7, 2.0**-3])
def test_public_score_is_the_reference_fp32_form_of_the_exact_max(scale):
    """Brute force with exact rationals: with x the exact directed block maximum
    (sign(scale) * dot) and s = fl32(|scale|), the reference's public score
    (triton/index_score.py:121-127, fp32 arithmetic without fusion) is
    fl32(fl32(hi * s) + fl32(lo * s)) for hi = fl32(x), lo = fl32(x - hi); for |scale| in
    {0, 1} and powers of two that is fl32(scale * max dot)."""
    gen = torch.Generator().manual_seed(7)
    lengths, groups, dim, block = [5, 7], 2, 9, 3
    q = torch.randn(sum(lengths), groups, dim, generator=gen).bfloat16().double().numpy()
    k = torch.randn(sum(lengths), 1, dim, generator=gen).bfloat16().double().numpy()
    cu = cu_list(lengths)
    _, s32, tie = O.index_score(q, k, cu, 8, block_size=block, scale=scale)
    sc = Fraction(scale)
    for a, b in zip(cu[:-1], cu[1:]):
        for t in range(a, b):
            for g in range(groups):
                for blk in range(s32.shape[2]):
                    keys = [j for j in range(a + blk * block, min(a + (blk + 1) * block, b)) if j <= t]
                    if not keys:
                        assert s32[t, g, blk] == -np.inf and tie[t, g, blk] == 0
                        continue
                    exact = [sc * sum(Fraction(x) * Fraction(y) for x, y in zip(q[t, g], k[j, 0])) for j in keys]
                    best = max(exact)
                    sign = 1 if scale > 0 else (-1 if scale < 0 else 0)
                    directed = max(sign * sum(Fraction(x) * Fraction(y) for x, y in zip(q[t, g], k[j, 0]))
                                   for j in keys)
                    s32f = Fraction(float(np.float32(abs(scale))))
                    hi = Fraction(float(_round_f32(directed)))
                    lo = Fraction(float(_round_f32(directed - hi)))
                    expected = _round_f32(Fraction(float(_round_f32(hi * s32f))) + Fraction(float(_round_f32(lo * s32f))))
                    assert s32[t, g, blk] == expected
                    if abs(scale) in (0.0, 1.0, 2.0**-3):
                        assert expected == _round_f32(best)  # one rounding of the scaled maximum
                    winners = [i for i, e in enumerate(exact) if e == best]
                    code = winners[0] + 1 if len(winners) == 1 else -len(winners)
                    assert tie[t, g, blk] == code


def _round_f32(x: Fraction) -> np.float32:
    """Correctly rounded fp32 of an exact rational (ties to even)."""
    guess = np.float32(float(x))
    candidates = [np.nextafter(guess, np.float32(-np.inf)), guess, np.nextafter(guess, np.float32(np.inf))]
    best = min(candidates, key=lambda c: (abs(Fraction(float(c)) - x), int(np.float32(c).view(np.int32)) & 1))
    return np.float32(best)


def _torch_amax_reference(q, k, cu, max_seqlen, block_size, scale):
    """Independent dense formulation differentiated by torch float64 autograd."""
    total, groups, dim = q.shape
    nb = (max_seqlen + block_size - 1) // block_size
    cols = []
    for a, b in zip(cu[:-1], cu[1:]):
        n = b - a
        logits = torch.einsum("tgd,kd->tgk", q[a:b], k[a:b, 0]) * scale  # [n, G, n]
        pos = torch.arange(n)
        causal = pos[None, :] <= pos[:, None]
        masked = logits.masked_fill(~causal[:, None, :], float("-inf"))
        pad = nb * block_size - n
        masked = torch.nn.functional.pad(masked, (0, pad), value=float("-inf"))
        cols.append(masked.reshape(n, groups, nb, block_size).amax(-1))
    return torch.cat(cols)


@pytest.mark.parametrize("lengths,groups,dim,block_size,scale", [
    ([3, 7], 2, 7, 4, 1.0), ([7, 11], 4, 16, 8, 0.5), ([9], 2, 64, 4, 1.0), ([0, 3, 0, 2, 0], 2, 7, 4, 1.0),
    ([6, 5], 2, 5, 4, -1.0),
])
def test_backward_matches_torch_amax_autograd(lengths, groups, dim, block_size, scale):
    gen = torch.Generator().manual_seed(731)
    total = sum(lengths)
    q = torch.randn(total, groups, dim, generator=gen).bfloat16().double().requires_grad_()
    k = torch.randn(total, 1, dim, generator=gen).bfloat16().double().requires_grad_()
    cu = cu_list(lengths)
    max_seqlen = max(lengths) + block_size
    ref = _torch_amax_reference(q, k, cu, max_seqlen, block_size, scale)
    s64, _, _ = O.index_score(q.detach().numpy(), k.detach().numpy(), cu, max_seqlen, block_size=block_size, scale=scale)
    finite = torch.isfinite(ref)
    np.testing.assert_array_equal(np.isfinite(s64), finite.numpy())
    np.testing.assert_allclose(s64[np.isfinite(s64)], ref[finite].detach().numpy(), rtol=1e-13, atol=1e-13)
    upstream = torch.randn(ref.shape, generator=gen).double()
    ref.backward(upstream.masked_fill(~finite, 0))
    dq, dk = O.index_score_backward(q.detach().numpy(), k.detach().numpy(), cu, max_seqlen,
                                    upstream.numpy(), block_size=block_size, scale=scale)
    np.testing.assert_allclose(dq, q.grad.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(dk, k.grad.numpy(), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("scale", [1.0, -0.5])
def test_index_score_rows_matches_full(scale):
    """The row-subset score restatement used at large sizes agrees with ``index_score`` bit for bit."""
    rng = np.random.default_rng(5)
    cu = np.array([0, 19, 19, 60], dtype=np.int32)
    iq = torch.from_numpy(rng.standard_normal((60, 2, 16))).bfloat16().float().numpy()
    ik = torch.from_numpy(rng.standard_normal((60, 1, 16))).bfloat16().float().numpy()
    f64, f32, _ = O.index_score(iq, ik, cu, 41, block_size=8, scale=scale)
    rows = np.array([0, 7, 8, 18, 19, 30, 59])
    r64, r32 = O.index_score_rows(iq, ik, cu, rows, f64.shape[2], block_size=8, scale=scale)
    np.testing.assert_array_equal(r64, f64[rows])
    np.testing.assert_array_equal(r32, f32[rows])


@pytest.mark.parametrize("scale", [1.0, -0.5, 0.0])
def test_backward_row_and_key_subsets_match_dense(scale):
    """index_score_backward_rows / _keys (the sampled-row restatements the large-config GPU
    tests use) equal the dense index_score_backward on a ragged pack with several groups,
    including exact ties (small-integer inputs) and an empty sequence."""
    rng = np.random.default_rng(5)
    lengths = [37, 0, 70, 9]
    cu = cu_list(lengths)
    total, groups, dim, block = cu[-1], 3, 6, 8
    q = rng.integers(-2, 3, size=(total, groups, dim)).astype(np.float64)  # many exact ties
    k = rng.integers(-2, 3, size=(total, 1, dim)).astype(np.float64)
    max_seqlen = max(lengths)
    nb = (max_seqlen + block - 1) // block
    ds = rng.standard_normal((total, groups, nb))
    dq, dk = O.index_score_backward(q, k, cu, max_seqlen, ds, block_size=block, scale=scale)
    tokens = np.array([0, 7, 8, 36, 37, 38, 60, 106, 107, 115])
    got_q = O.index_score_backward_rows(q, k, cu, ds, tokens, block_size=block, scale=scale)
    np.testing.assert_allclose(got_q, dq[tokens], rtol=1e-13, atol=1e-13)
    keys = np.array([0, 5, 8, 36, 37, 44, 45, 100, 106, 107, 115])
    got_k = O.index_score_backward_keys(q, k, cu, ds, keys, block_size=block, scale=scale)
    np.testing.assert_allclose(got_k, dk[keys], rtol=1e-13, atol=1e-13)
    # every key: the subsets add up to the dense result (block grouping, slab edges)
    got_all = O.index_score_backward_keys(q, k, cu, ds, np.arange(total), block_size=block, scale=scale)
    np.testing.assert_allclose(got_all, dk, rtol=1e-13, atol=1e-13)


def test_backward_key_subset_spans_query_slabs():
    """A sequence longer than the key restatement's 4096-token query slab."""
    rng = np.random.default_rng(11)
    lengths = [4300]
    cu = cu_list(lengths)
    q = rng.standard_normal((4300, 2, 4))
    k = rng.standard_normal((4300, 1, 4))
    block = 512
    nb = (4300 + block - 1) // block
    ds = rng.standard_normal((4300, 2, nb))
    _, dk = O.index_score_backward(q, k, cu, 4300, ds, block_size=block)
    keys = np.array([0, 1, 511, 4095, 4096, 4299])
    got = O.index_score_backward_keys(q, k, cu, ds, keys, block_size=block)
    np.testing.assert_allclose(got, dk[keys], rtol=1e-12, atol=1e-12)
