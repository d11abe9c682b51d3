"""GPU parity of stage 2 (m3_topk) and the k2q CSR against the CPU oracle: bit-exact.

Cases mirror tests/test_topk.py and tests/test_k2q.py of the reference, plus
adversarial ties/-inf rows and BASELINE-sized rows (T=8192..65536 rows).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import msa_triton_amd as msa
from msa_triton_amd.k2q import build_k2q_csr
from oracle import msa_oracle as O
from tests.helpers import cu_list, cu_tensor

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("lengths,block,k,local", [
    ([1, 7, 3], 2, 3, 1), ([127, 128, 129], 128, 16, 1), ([17, 0, 9], 4, 2, 0), ([8, 5], 2, 3, 3), ([2], 1, 0, 0),
])
def test_topk_matches_oracle(lengths, block, k, local, device):
    groups, blocks = 3, (max(lengths) + block - 1) // block
    scores_cpu = torch.randn(sum(lengths), groups, blocks, generator=torch.Generator().manual_seed(82))
    scores = scores_cpu.to(device)
    saved = scores.clone()
    cu = cu_tensor(lengths, device)
    selected = msa.m3_topk(scores, cu, block_size=block, topk_blocks=k, local_blocks=local)
    assert selected.dtype == torch.int32 and selected.shape == (sum(lengths), groups, k)
    assert not selected.requires_grad
    torch.testing.assert_close(scores, saved, atol=0, rtol=0)
    expected = O.topk(scores_cpu.numpy(), cu_list(lengths), block_size=block, topk_blocks=k, local_blocks=local)
    np.testing.assert_array_equal(selected.cpu().numpy(), expected)


def test_topk_equal_scores_local_and_no_gradient(device):
    scores = torch.zeros(7, 2, 4, requires_grad=True, device=device)
    cu = cu_tensor([7], device)
    out = msa.m3_topk(scores, cu, block_size=2, topk_blocks=2, local_blocks=1)
    assert not out.requires_grad
    expected = O.topk(np.zeros((7, 2, 4), np.float32), [0, 7], block_size=2, topk_blocks=2, local_blocks=1)
    np.testing.assert_array_equal(out.cpu().numpy(), expected)


def test_topk_adversarial_ties_infinities_and_wide_rows(device):
    gen = torch.Generator().manual_seed(5)
    lengths, block, groups, k = [700, 300], 4, 2, 9
    nb = (max(lengths) + block - 1) // block
    scores = torch.randint(-3, 3, (sum(lengths), groups, nb), generator=gen).float()
    scores[::7] = float("-inf")
    scores[::11, :, ::3] = float("inf")
    scores[5::13] = -0.0
    cu = cu_tensor(lengths, device)
    for local in (0, 2, 9):
        got = msa.m3_topk(scores.to(device), cu, block_size=block, topk_blocks=k, local_blocks=local)
        ref = O.topk(scores.numpy(), cu_list(lengths), block_size=block, topk_blocks=k, local_blocks=local)
        np.testing.assert_array_equal(got.cpu().numpy(), ref)


@pytest.mark.parametrize("tokens,block", [(200, 4), (4000, 2), (9000, 1)])
def test_topk_nan_scores_rank_above_inf(tokens, block, device):
    """NaN scores of either sign rank above +inf, as in torch.topk (the oracle's order is
    pinned against torch.topk on the CPU), on all three selection paths: 16 lanes per row
    (50 blocks), a wavefront per row (2000) and the streamed rows (9000); several NaNs per
    row are emitted in ascending block order, like other equal values."""
    gen = torch.Generator().manual_seed(tokens)
    nb = (tokens + block - 1) // block
    scores = torch.randint(-3, 4, (tokens, 2, nb), generator=gen).float()
    pick = torch.rand(tokens, 2, nb, generator=gen)
    scores[pick < 0.02] = float("nan")
    scores[(pick > 0.02) & (pick < 0.03)] = -float("nan")
    scores[(pick > 0.5) & (pick < 0.52)] = float("inf")
    scores[(pick > 0.6) & (pick < 0.7)] = float("-inf")
    cu = cu_tensor([tokens], device)
    for k, local in ((8, 0), (24, 2)):
        got = msa.m3_topk(scores.to(device), cu, block_size=block, topk_blocks=k, local_blocks=local)
        ref = O.topk(scores.numpy(), [0, tokens], block_size=block, topk_blocks=k, local_blocks=local)
        np.testing.assert_array_equal(got.cpu().numpy(), ref)


@pytest.mark.parametrize("total,groups,nb,k,local", [(8192, 4, 64, 16, 1), (32768, 4, 256, 16, 1), (4096, 8, 512, 32, 2)])
def test_topk_baseline_sized_rows(total, groups, nb, k, local, device):
    gen = torch.Generator().manual_seed(total)
    block = 128 if nb * 128 >= total else 64
    lengths = [total]
    scores = torch.randn(total, groups, nb, generator=gen)
    got = msa.m3_topk(scores.to(device), cu_tensor(lengths, device), block_size=block, topk_blocks=k, local_blocks=local)
    ref = O.topk(scores.numpy(), cu_list(lengths), block_size=block, topk_blocks=k, local_blocks=local)
    np.testing.assert_array_equal(got.cpu().numpy(), ref)


@pytest.mark.parametrize("tokens,block,k,local", [(2048, 2, 16, 1), (3000, 2, 32, 2), (4400, 2, 8, 0)])
def test_topk_long_rows(tokens, block, k, local, device):
    """Rows of 1024 blocks (sixteen lanes per row) and of 1500 / 2200 blocks (one
    wavefront per row), with integer scores for ties."""
    gen = torch.Generator().manual_seed(tokens)
    nb = (tokens + block - 1) // block
    scores = torch.randint(-4, 5, (tokens, 2, nb), generator=gen).float()
    got = msa.m3_topk(scores.to(device), cu_tensor([tokens], device), block_size=block, topk_blocks=k,
                      local_blocks=local)
    ref = O.topk(scores.numpy(), [0, tokens], block_size=block, topk_blocks=k, local_blocks=local)
    np.testing.assert_array_equal(got.cpu().numpy(), ref)


def _check_csr(ids_cpu, lengths, block_size, device):
    ids = ids_cpu.to(device)
    original = ids.clone()
    result = build_k2q_csr(ids, cu_tensor(lengths, device), block_size=block_size)
    expected = O.k2q_csr(ids_cpu.contiguous().numpy(), cu_list(lengths), block_size=block_size)
    for actual, exp in zip((result.row_ptr, result.query_indices, result.slot_indices, result.cu_block_lens), expected):
        assert actual.dtype == torch.int32 and actual.device == ids.device and not actual.requires_grad
        np.testing.assert_array_equal(actual.cpu().numpy(), exp)
    torch.testing.assert_close(ids, original, atol=0, rtol=0)
    return result


@pytest.mark.parametrize("lengths,groups,slots,block_size", [
    ([1], 1, 4, 128), ([3, 5], 3, 5, 2), ([0, 3, 0, 2, 0], 2, 4, 2),
    ([127, 128, 129], 4, 5, 128), ([0, 0], 3, 5, 128), ([4, 2], 3, 0, 2),
])
def test_k2q_matches_oracle(lengths, groups, slots, block_size, device):
    generator = torch.Generator().manual_seed(951)
    max_blocks = (max(lengths) + block_size - 1) // block_size
    ids = torch.randint(-2, max_blocks + 4, (sum(lengths), groups, slots), generator=generator, dtype=torch.int32)
    _check_csr(ids, lengths, block_size, device)


def test_k2q_duplicates_and_block_reset(device):
    ids = torch.tensor(
        [[[0, 0, 1], [1, 0, -1]], [[0, -1, 8], [0, 0, 1]], [[1, 0, 1], [0, 1, -2]], [[0, 0, 1], [0, -1, 9]],
         [[0, 0, -1], [0, 0, -1]]], dtype=torch.int32)
    result = _check_csr(ids, [3, 2], 2, device)
    assert result.cu_block_lens.cpu().tolist() == [0, 2, 3]
    ptr = result.row_ptr.cpu().tolist()
    assert set(result.query_indices[ptr[4]:ptr[5]].cpu().tolist()) == {3, 4}


def test_k2q_hotspots_tail_block_noncontiguous_and_all_invalid(device):
    lengths, groups, slots, block_size = [9, 5], 4, 3, 4
    ids = torch.full((sum(lengths), groups, slots), -1, dtype=torch.int32)
    start = 0
    for length in lengths:
        for local in range(length):
            ids[start + local, :, 0] = local // block_size
            ids[start + local, :, 1] = 0
            if local // block_size > 0:
                ids[start + local, :, 2] = local // block_size - 1
        start += length
    _check_csr(ids, lengths, block_size, device)
    base = torch.tensor([[[0, 1, 2, -1], [0, -1, 9, 0]]] * 5, dtype=torch.int32)
    _check_csr(base.transpose(1, 2), [2, 3], 2, device)
    bad = torch.full((7, 2, 4), 99, dtype=torch.int32)
    bad[:, :, 0] = -1
    result = _check_csr(bad, [3, 4], 2, device)
    assert result.row_ptr.count_nonzero().item() == 0


def test_k2q_sequences_longer_than_1024_blocks(device):
    """Query blocks 1024 and later take the serial path of the scatter; earlier ones
    and the short second sequence the parallel one. Random ids include duplicates."""
    generator = torch.Generator().manual_seed(1100)
    lengths, groups, slots, block_size = [2200, 37], 2, 3, 2
    ids = torch.randint(-1, 1101, (sum(lengths), groups, slots), generator=generator, dtype=torch.int32)
    _check_csr(ids, lengths, block_size, device)


@pytest.mark.parametrize("lengths,groups,k,block", [
    ([8192], 4, 16, 128), ([2048, 3072, 5120, 6144], 4, 16, 128), ([32768], 4, 16, 128),
])
def test_k2q_baseline_sized(lengths, groups, k, block, device):
    gen = torch.Generator().manual_seed(len(lengths))
    total = sum(lengths)
    scores = torch.randn(total, groups, (max(lengths) + block - 1) // block, generator=gen)
    ids = msa.m3_topk(scores.to(device), cu_tensor(lengths, device), block_size=block, topk_blocks=k, local_blocks=1)
    _check_csr(ids.cpu(), lengths, block, device)


@pytest.mark.parametrize("length,block,k", [(1024, 4, 16), (512, 4, 12), (2048, 4, 32)])
def test_topk_winners_concentrated_in_one_lane(length, block, k, device):
    """Sixteen lanes share a row (lane j holds blocks j, j + 16, ...) and each keeps a
    cache of its four largest remaining keys: rows whose winners all sit in one lane
    (blocks b with b % 16 == row % 16 lead by 10) refill that cache several times;
    some leaders tie (ascending block order) and a few are -inf."""
    gen = torch.Generator().manual_seed(29)
    groups, nb = 2, (length + block - 1) // block
    scores = torch.randn(length, groups, nb, generator=gen)
    rows = torch.arange(length).view(-1, 1, 1)
    lead = (torch.arange(nb).view(1, 1, -1) % 16) == (rows % 16)
    scores = torch.where(lead, scores + 10.0, scores)
    scores[::5, :, ::32] = 12.5  # ties among the leaders (and among the other lanes' blocks)
    scores[::9, 1, 16::48] = float("-inf")
    cu = cu_tensor([length], device)
    for local in (0, 1, 3):
        got = msa.m3_topk(scores.to(device), cu, block_size=block, topk_blocks=k, local_blocks=local)
        ref = O.topk(scores.numpy(), [0, length], block_size=block, topk_blocks=k, local_blocks=local)
        np.testing.assert_array_equal(got.cpu().numpy(), ref)


@pytest.mark.parametrize("tokens,block,k,local", [(9000, 2, 24, 2), (4500, 1, 40, 1)])
def test_topk_rows_beyond_4096_blocks(tokens, block, k, local, device):
    """Rows of 4500 blocks: one wavefront per row with the row streamed from memory. In
    every row the blocks of one lane (b % 64 == row % 64) lead, so that lane's cache of
    eight keys empties and refills several times; integer scores tie, some are -inf."""
    gen = torch.Generator().manual_seed(tokens + k)
    groups, nb = 2, (tokens + block - 1) // block
    scores = torch.randint(-4, 5, (tokens, groups, nb), generator=gen).float()
    rows = torch.arange(tokens).view(-1, 1, 1)
    lead = (torch.arange(nb).view(1, 1, -1) % 64) == (rows % 64)
    scores = torch.where(lead, scores + 20.0, scores)
    scores[::7, 0, ::5] = float("-inf")
    got = msa.m3_topk(scores.to(device), cu_tensor([tokens], device), block_size=block, topk_blocks=k,
                      local_blocks=local)
    ref = O.topk(scores.numpy(), [0, tokens], block_size=block, topk_blocks=k, local_blocks=local)
    np.testing.assert_array_equal(got.cpu().numpy(), ref)
