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


@pytest.mark.parametrize("bounds,block", [([0, 5, 9], 4), ([0, 3, 3, 10, 20], 4), ([0, 300], 128), ([0, 0], 7)])
def test_call_and_rescaled_sequences_match_prepared(bounds, block):
    """The call-scoped metadata (one packed host-to-device copy, the G-scaled k2q tile prefix
    included) and a prepared object re-described for another block size equal a fresh
    prepare_sequences of the same bounds."""
    from msa_triton_amd.layout import call_sequences, sequence_meta, tile_prefix_times, with_block_size

    cu = torch.tensor(bounds, dtype=torch.int32)
    fresh = msa.prepare_sequences(cu, block_size=block)
    call = call_sequences(cu, sequence_meta(bounds, block), 3)
    assert call.cu_seqlens is cu and call.meta == fresh.meta
    assert torch.equal(call.cu_block_lens, fresh.cu_block_lens) and call.cu_block_lens.dtype == torch.int32
    assert torch.equal(call.tile_prefix, fresh.tile_prefix) and call.tile_prefix.dtype == torch.int64
    for g in (3, 5):  # the copied G-scaled prefix, and one computed on request
        assert torch.equal(tile_prefix_times(call, g), fresh.tile_prefix * g)
        assert tile_prefix_times(fresh, g) is tile_prefix_times(fresh, g)
    other = with_block_size(msa.prepare_sequences(cu, block_size=2 * block), block)
    assert other.meta == fresh.meta
    assert torch.equal(other.cu_block_lens, fresh.cu_block_lens) and torch.equal(other.tile_prefix, fresh.tile_prefix)
    base = msa.prepare_sequences(cu, block_size=2 * block)
    assert with_block_size(base, block) is with_block_size(base, block)  # cached with its PackedSequences
    assert with_block_size(base, 2 * block) is base
