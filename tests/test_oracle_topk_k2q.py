"""Pin the stage-2 (top-k) and k2q CSR oracles.

Top-k: independent Python ranking (tests/test_topk.py:20-50), the hand example
(tests/test_eager.py:155-170), all-equal scores with forced locals
(tests/test_topk.py:53-66) and the fixed slot count (tests/test_eager.py:173-180).
CSR: pure-Python inversion (tests/test_k2q.py:21-51) and the known answers of
tests/test_k2q.py:101-135.
"""

from __future__ import annotations

from collections import Counter

import numpy as np
import pytest
import torch

from oracle import msa_oracle as O
from tests.helpers import cu_list


@pytest.mark.parametrize("lengths,block,k,local", [
    ([1, 7, 3], 2, 3, 1), ([127, 128, 129], 128, 16, 1), ([17, 0, 9], 4, 2, 0), ([8, 5], 2, 3, 3), ([2], 1, 0, 0),
])
def test_topk_matches_independent_ranking(lengths, block, k, local):
    cu = cu_list(lengths)
    groups, blocks = 3, (max(lengths) + block - 1) // block
    scores = torch.randn(sum(lengths), groups, blocks, generator=torch.Generator().manual_seed(82)).numpy()
    selected = O.topk(scores, cu, block_size=block, topk_blocks=k, local_blocks=local)
    assert selected.dtype == np.int32 and selected.shape == (sum(lengths), groups, k)
    start = 0
    for length in lengths:
        for position in range(length):
            current = position // block
            forced = list(range(max(0, current - local + 1), current + 1)) if local else []
            for group in range(groups):
                candidates = [b for b in range(current + 1) if b not in forced]
                candidates.sort(key=lambda b: -float(scores[start + position, group, b]))
                expected_set = set(forced) | set(candidates[: k - len(forced)])
                actual = selected[start + position, group].tolist()
                kept = [b for b in actual if b != -1]
                assert len(kept) == len(set(kept)) and set(kept) == expected_set
                assert actual == kept + [-1] * (k - len(kept))
                # canonical order: forced (ascending) first, then descending score
                expected_order = (sorted(forced) + candidates)[: min(k, len(forced) + len(candidates))]
                assert kept == expected_order[: len(kept)]
        start += length


def test_topk_hand_example_and_no_mutation():
    scores = np.broadcast_to(np.array([[[10.0, 2.0, 0.0], [1.0, 9.0, 0.0]]], dtype=np.float32), (5, 2, 3)).copy()
    original = scores.copy()
    ids = O.topk(scores, [0, 5], block_size=2, topk_blocks=2, local_blocks=1)
    assert set(ids[-1, 0].tolist()) == {0, 2} and set(ids[-1, 1].tolist()) == {1, 2}
    assert ids[0, 0].tolist() == [0, -1]
    np.testing.assert_array_equal(scores, original)


def test_topk_equal_scores_keep_local():
    ids = O.topk(np.zeros((7, 2, 4), dtype=np.float32), [0, 7], block_size=2, topk_blocks=2, local_blocks=1)
    for token in range(7):
        for group in range(2):
            valid = [b for b in ids[token, group].tolist() if b >= 0]
            assert token // 2 in valid and len(valid) == min(2, token // 2 + 1)
            assert len(set(valid)) == len(valid) and all(0 <= b <= token // 2 for b in valid)


@pytest.mark.parametrize("k,local", [(0, 0), (1, 0), (8, 1), (8, 8)])
def test_topk_short_sequence_fixed_slot_count(k, local):
    ids = O.topk(np.zeros((2, 2, 1), dtype=np.float32), [0, 1, 2], block_size=4, topk_blocks=k, local_blocks=local)
    assert ids.shape == (2, 2, k)
    if k:
        assert (ids[..., 0] == 0).all() and (ids[..., 1:] == -1).all()


def test_topk_minus_inf_scores_become_padding():
    scores = np.full((4, 1, 2), -np.inf, dtype=np.float32)
    ids = O.topk(scores, [0, 4], block_size=2, topk_blocks=2, local_blocks=0)
    assert (ids == -1).all()


def _invert_python(indices, lengths, block_size):
    """Pure-Python edge inversion, independent of the oracle (tests/test_k2q.py:21-51)."""
    tokens, groups, slots = indices.shape
    values = indices.tolist()
    block_prefix = [0]
    for length in lengths:
        block_prefix.append(block_prefix[-1] + (length + block_size - 1) // block_size)
    rows = [[] for _ in range(block_prefix[-1] * groups)]
    valid_edges = []
    start = 0
    for sequence, length in enumerate(lengths):
        nblocks = (length + block_size - 1) // block_size
        for local_query in range(length):
            query = start + local_query
            for group in range(groups):
                for slot in range(slots):
                    block = values[query][group][slot]
                    if block < 0 or block >= nblocks or block * block_size > local_query:
                        continue
                    row = (block_prefix[sequence] + block) * groups + group
                    rows[row].append((query, slot))
                    valid_edges.append((row, query, slot))
        start += length
    row_ptr, queries, sel = [0], [], []
    for row in rows:
        for query, slot in sorted(row):
            queries.append(query)
            sel.append(slot)
        row_ptr.append(len(queries))
    padding = tokens * groups * slots - len(queries)
    return row_ptr, queries + [-1] * padding, sel + [-1] * padding, block_prefix, valid_edges


def check_csr(result, indices, lengths, block_size):
    ptr, queries, slots, prefix, edges = _invert_python(indices, lengths, block_size)
    for actual, expected in zip(result, (ptr, queries, slots, prefix)):
        np.testing.assert_array_equal(np.asarray(actual), np.asarray(expected, dtype=np.int32))
    actual_ptr = np.asarray(result[0]).tolist()
    reconstructed = []
    for row, (lo, hi) in enumerate(zip(actual_ptr[:-1], actual_ptr[1:])):
        for e in range(lo, hi):
            reconstructed.append((row, int(result[1][e]), int(result[2][e])))
    assert Counter(reconstructed) == Counter(edges)


@pytest.mark.parametrize("lengths,groups,slots,block_size", [
    ([1], 1, 4, 128), ([3, 5], 3, 5, 2), ([0, 3, 0, 2, 0], 2, 4, 2),
    ([127, 128, 129], 4, 5, 128), ([0, 0], 3, 5, 128), ([4, 2], 3, 0, 2),
])
def test_k2q_oracle_matches_python_inversion(lengths, groups, slots, block_size):
    generator = torch.Generator().manual_seed(951)
    max_blocks = (max(lengths) + block_size - 1) // block_size
    ids = torch.randint(-2, max_blocks + 4, (sum(lengths), groups, slots), generator=generator, dtype=torch.int32).numpy()
    check_csr(O.k2q_csr(ids, cu_list(lengths), block_size=block_size), ids, lengths, block_size)


def test_k2q_duplicates_and_per_sequence_block_reset():
    ids = np.array(
        [[[0, 0, 1], [1, 0, -1]], [[0, -1, 8], [0, 0, 1]], [[1, 0, 1], [0, 1, -2]], [[0, 0, 1], [0, -1, 9]],
         [[0, 0, -1], [0, 0, -1]]], dtype=np.int32)
    result = O.k2q_csr(ids, [0, 3, 5], block_size=2)
    check_csr(result, ids, [3, 2], 2)
    assert result[3].tolist() == [0, 2, 3]
    ptr = result[0].tolist()
    assert set(result[1][ptr[4]:ptr[5]].tolist()) == {3, 4}


def test_k2q_all_invalid():
    ids = np.full((7, 2, 4), 99, dtype=np.int32)
    ids[:, :, 0] = -1
    result = O.k2q_csr(ids, [0, 3, 7], block_size=2)
    assert np.count_nonzero(result[0]) == 0 and (result[1] == -1).all()


@pytest.mark.parametrize("local_blocks", [0, 1, 2])
def test_topk_rows_matches_full_topk(local_blocks):
    """The row-subset restatement used at large sizes agrees with ``topk`` row by row."""
    rng = np.random.default_rng(11)
    lengths, groups, block = [37, 0, 70], 3, 8
    cu = np.array([0, 37, 37, 107], dtype=np.int32)
    nb = (70 + block - 1) // block
    scores = rng.standard_normal((107, groups, nb)).astype(np.float32)
    scores[5, 1, 2] = scores[5, 1, 0]  # an exact tie
    full = O.topk(scores, cu, block_size=block, topk_blocks=5, local_blocks=local_blocks)
    rows = np.array([0, 5, 36, 37, 40, 99, 106])
    starts = np.where(rows < 37, 0, 37)
    part = O.topk_rows(scores[rows], rows - starts, block_size=block, topk_blocks=5, local_blocks=local_blocks)
    np.testing.assert_array_equal(part, full[rows])


def test_eager_baseline_score_and_topk_match_oracle():
    """The CPU baseline's eager score / top-k restatements (oracle/eager_baseline.py) agree
    with the oracle: scores to fp32 rounding of the dot, the selection as a set per row."""
    from oracle.eager_baseline import eager_score_rows, eager_topk

    gen = torch.Generator().manual_seed(3)
    n, groups, dim, block = 300, 2, 16, 32
    iq = torch.randn(n, groups, dim, generator=gen).bfloat16()
    ik = torch.randn(n, 1, dim, generator=gen).bfloat16()
    _, ref32, _ = O.index_score(iq.double().numpy(), ik.double().numpy(), [0, n], n, block_size=block)
    got = eager_score_rows(iq, ik, (100, 300), block_size=block).numpy()
    np.testing.assert_allclose(got, ref32[100:300], rtol=1e-5, atol=1e-5)
    ids = eager_topk(torch.from_numpy(ref32), torch.arange(n), block_size=block, topk_blocks=4, local_blocks=1)
    ref_ids = O.topk(ref32, [0, n], block_size=block, topk_blocks=4, local_blocks=1)
    assert np.array_equal(np.sort(ids.numpy(), -1), np.sort(ref_ids, -1))


@pytest.mark.parametrize("local", [0, 1])
def test_topk_nan_ranks_like_torch_topk(local):
    """Scores with NaN (either sign) and -inf, at most one NaN per row and distinct values
    otherwise (so that torch.topk's order is fully determined): the oracle equals the
    reference's own steps (triton/topk.py:31-46: causal -inf mask, +inf local boost,
    torch.topk sorted, -inf picks -> -1, -1 padding), in which NaN ranks above +inf."""
    gen = torch.Generator().manual_seed(11 + local)
    lengths, block, groups, k = [37, 20], 2, 2, 6
    cu = cu_list(lengths)
    nb = (max(lengths) + block - 1) // block
    total = sum(lengths)
    scores = torch.randn(total, groups, nb, generator=gen)
    scores[::5, 0, ::4] = float("-inf")
    rows = torch.randint(0, nb, (total, groups), generator=gen)
    sign = torch.where(torch.rand(total, groups, generator=gen) < 0.5, -1.0, 1.0)
    has_nan = torch.rand(total, groups, generator=gen) < 0.6
    scores.scatter_(2, rows[..., None], torch.where(has_nan, sign * float("nan"), scores.gather(2, rows[..., None])[..., 0])[..., None])
    got = O.topk(scores.numpy(), cu, block_size=block, topk_blocks=k, local_blocks=local)
    start = 0
    for length in lengths:
        for pos in range(length):
            t, qb = start + pos, pos // block
            for g in range(groups):
                row = scores[t, g].clone()
                row[qb + 1:] = float("-inf")
                if local:
                    row[max(0, qb - local + 1): qb + 1] = float("inf")
                count = min(k, nb)
                val, idx = torch.topk(row, count, sorted=True)
                want = torch.where(val == float("-inf"), -1, idx).tolist() + [-1] * (k - count)
                assert got[t, g].tolist() == want, (t, g, row.tolist())
        start += length
