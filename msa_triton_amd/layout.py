"""Packed-sequence metadata validation (host side).

``sequence_lengths`` mirrors layout.py:12-24 of the reference (same checks, same
messages and exception types); its messages are part of the attention error
contract. ``SequenceMeta`` is the per-call host metadata every operator derives
from ``cu_seqlens`` (block counts, per-sequence block prefix ``cu_block_lens``),
computed once from the single host read of ``cu_seqlens``.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


def sequence_lengths(cu_seqlens: torch.Tensor, total_tokens: int) -> list[int]:
    """Validate packed boundaries and return sequence lengths on the host."""
    if cu_seqlens.ndim != 1 or cu_seqlens.numel() < 2:
        raise ValueError("cu_seqlens must be a vector with at least two entries")
    if cu_seqlens.dtype != torch.int32:
        raise TypeError("cu_seqlens must be int32")
    boundaries = cu_seqlens.detach().cpu().tolist()
    if boundaries[0] != 0 or boundaries[-1] != total_tokens:
        raise ValueError("cu_seqlens must start at zero and end at total_tokens")
    lengths = [end - start for start, end in zip(boundaries[:-1], boundaries[1:])]
    if min(lengths) < 0:
        raise ValueError("cu_seqlens must be nondecreasing")
    return lengths


@dataclass(frozen=True)
class SequenceMeta:
    """Host-side description of a packed batch for a given block size."""

    bounds: tuple[int, ...]
    lengths: tuple[int, ...]
    block_counts: tuple[int, ...]
    cu_block_lens: tuple[int, ...]
    block_size: int

    @property
    def num_seqs(self) -> int:
        return len(self.lengths)

    @property
    def total_blocks(self) -> int:
        return self.cu_block_lens[-1]

    @property
    def tri_prefix(self) -> list[int]:
        """Start of each sequence's tile-counter range in the k2q histogram (per group)."""
        out = [0]
        for nb in self.block_counts:
            out.append(out[-1] + nb * (nb + 1) // 2)
        return out


def sequence_meta(bounds: list[int], block_size: int) -> SequenceMeta:
    lengths = [end - start for start, end in zip(bounds[:-1], bounds[1:])]
    block_counts = [(length + block_size - 1) // block_size for length in lengths]
    cu_blocks = [0]
    for count in block_counts:
        cu_blocks.append(cu_blocks[-1] + count)
    return SequenceMeta(tuple(bounds), tuple(lengths), tuple(block_counts), tuple(cu_blocks), block_size)
