"""Prepared packed-sequence metadata (host side, no GPU): validation, immutability
and the operator-side checks that run before any launch."""

from __future__ import annotations

import pytest
import torch

import msa_triton_amd as msa
from msa_triton_amd.k2q import build_k2q_csr
from msa_triton_amd.layout import prepared_for


def test_prepare_sequences_metadata():
    seqs = msa.prepare_sequences(torch.tensor([0, 3, 3, 10], dtype=torch.int32), block_size=4)
    assert isinstance(seqs, msa.PackedSequences)
    assert seqs.meta.lengths == (3, 0, 7) and seqs.meta.block_counts == (1, 0, 2)
    assert seqs.cu_block_lens.tolist() == [0, 1, 1, 3]
    # per-sequence start of the (query block, key block) causal tile counters: nb (nb + 1) / 2 each
    assert seqs.tile_prefix.tolist() == [0, 1, 1, 4] and seqs.tile_prefix.dtype == torch.int64
    assert seqs.total_tokens == 10 and seqs.max_seqlen == 7 and seqs.block_size == 4


def test_prepared_copies_are_private():
    cu = torch.tensor([0, 5, 9], dtype=torch.int32)
    seqs = msa.prepare_sequences(cu, block_size=2)
    cu[1] = 7
    assert seqs.cu_seqlens.tolist() == [0, 5, 9] and seqs.meta.bounds == (0, 5, 9)
    assert seqs.cu_seqlens.data_ptr() != cu.data_ptr()


@pytest.mark.parametrize("cu,block,exc,match", [
    (torch.tensor([0, 4], dtype=torch.int64), 2, TypeError, "int32"),
    (torch.tensor([1, 4], dtype=torch.int32), 2, ValueError, "start at zero"),
    (torch.tensor([0, 4, 3], dtype=torch.int32), 2, ValueError, "nondecreasing"),
    (torch.tensor([0], dtype=torch.int32), 2, ValueError, "at least two"),
    (torch.tensor([0, 4], dtype=torch.int32), 0, ValueError, "block_size"),
    (torch.tensor([0, 4], dtype=torch.int32), True, ValueError, "block_size"),
])
def test_prepare_sequences_rejects_bad_metadata(cu, block, exc, match):
    with pytest.raises(exc, match=match):
        msa.prepare_sequences(cu, block_size=block)


def test_prepared_for_checks_block_size_tokens_and_device():
    seqs = msa.prepare_sequences(torch.tensor([0, 6], dtype=torch.int32), block_size=4)
    assert prepared_for(seqs, block_size=4, total_tokens=6, device=torch.device("cpu")) is seqs.meta
    with pytest.raises(ValueError, match="block_size"):
        prepared_for(seqs, block_size=8, total_tokens=6, device=torch.device("cpu"))
    with pytest.raises(ValueError, match="total_tokens"):
        prepared_for(seqs, block_size=4, total_tokens=7, device=torch.device("cpu"))


def test_operators_check_prepared_metadata_before_launch():
    seqs = msa.prepare_sequences(torch.tensor([0, 6], dtype=torch.int32), block_size=4)
    scores = torch.zeros(6, 1, 2)
    with pytest.raises(ValueError, match="block_size"):
        msa.m3_topk(scores, seqs, block_size=2, topk_blocks=1)
    with pytest.raises(ValueError, match="block_size"):
        build_k2q_csr(torch.zeros(6, 1, 1, dtype=torch.int32), seqs, block_size=8)
    iq = torch.zeros(6, 1, 4, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="max_seqlen"):
        msa.m3_index_score(iq, torch.zeros(6, 1, 4, dtype=torch.bfloat16), seqs, 5, block_size=4)
    q = torch.zeros(6, 2, 8, dtype=torch.bfloat16)
    kv = torch.zeros(6, 1, 8, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="total_tokens"):
        msa.m3_sparse_attention(q[:5], kv[:5], kv[:5], torch.zeros(5, 1, 1, dtype=torch.int32), seqs, 6,
                                block_size=4)
