"""Packed-sequence metadata validation (host side).

``sequence_lengths`` mirrors layout.py:12-24 of the reference (same checks, same
messages and exception types); its messages are part of the attention error
contract. ``SequenceMeta`` is the per-call host metadata every operator derives
from ``cu_seqlens`` (block counts, per-sequence block prefix ``cu_block_lens``),
computed once from the single host read of ``cu_seqlens``.

``PackedSequences`` (from ``prepare_sequences``) is the prepared, immutable form:
validated once, with its own device copies of ``cu_seqlens``, ``cu_block_lens``
and the k2q tile prefix. Every operator accepts it in place of ``cu_seqlens`` and
then reads nothing back from the device, so a layer's score, top-k, attention and
backward issue no host synchronisation and can be captured in a HIP graph. Its
device tensors are private clones: later writes to the caller's ``cu_seqlens``
do not reach it (the stale-cache hazard of keying a cache on the caller's tensor).
"""

from __future__ import annotations

import weakref
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


@dataclass(frozen=True, eq=False)
class PackedSequences:
    """Validated packed-sequence metadata for one block size, with device copies.

    ``cu_seqlens`` (int32 ``[N+1]``), ``cu_block_lens`` (int32 ``[N+1]``) and
    ``tile_prefix`` (int64 ``[N+1]``, the per-sequence start of the k2q
    histogram's (query block, key block) counters, per group) live on the
    device; ``meta`` holds the same numbers on the host.
    """

    cu_seqlens: torch.Tensor
    cu_block_lens: torch.Tensor
    tile_prefix: torch.Tensor
    meta: SequenceMeta

    @property
    def device(self) -> torch.device:
        return self.cu_seqlens.device

    @property
    def block_size(self) -> int:
        return self.meta.block_size

    @property
    def total_tokens(self) -> int:
        return self.meta.bounds[-1]

    @property
    def max_seqlen(self) -> int:
        return max(self.meta.lengths)


def prepare_sequences(cu_seqlens: torch.Tensor, *, block_size: int = 128) -> PackedSequences:
    """Validate ``cu_seqlens`` once (one host read) and return ``PackedSequences``.

    The checks and messages are those of ``sequence_lengths`` (zero start,
    nondecreasing); the total token count is the last boundary.
    """
    if not isinstance(cu_seqlens, torch.Tensor):
        raise TypeError("cu_seqlens must be a tensor")
    if not isinstance(block_size, int) or isinstance(block_size, bool) or block_size <= 0:
        raise ValueError("block_size must be a positive integer")
    if cu_seqlens.ndim != 1 or cu_seqlens.numel() < 2:
        raise ValueError("cu_seqlens must be a vector with at least two entries")
    if cu_seqlens.dtype != torch.int32:
        raise TypeError("cu_seqlens must be int32")
    bounds = cu_seqlens.detach().cpu().tolist()
    if bounds[0] != 0:
        raise ValueError("cu_seqlens must start at zero and end at total_tokens")
    if any(b < a for a, b in zip(bounds, bounds[1:])):
        raise ValueError("cu_seqlens must be nondecreasing")
    meta = sequence_meta(bounds, block_size)
    device = cu_seqlens.device
    return PackedSequences(
        cu_seqlens=cu_seqlens.detach().clone().contiguous(),
        cu_block_lens=torch.tensor(meta.cu_block_lens, dtype=torch.int32, device=device),
        tile_prefix=torch.tensor(meta.tri_prefix, dtype=torch.int64, device=device),
        meta=meta,
    )


def call_sequences(cu_seqlens: torch.Tensor, meta: SequenceMeta, groups: int) -> PackedSequences:
    """``PackedSequences`` for one operator call whose ``cu_seqlens`` the host has read and
    validated already (``meta``): the block metadata, with the k2q tile prefix already
    multiplied by ``groups`` (``tile_prefix_times``), reaches the device in one
    host-to-device copy, and the rest of the call (CSR build, attention passes) reads
    nothing back. Its ``cu_seqlens`` is the caller's tensor, not a private clone: valid
    for that call only."""
    n = meta.num_seqs + 1
    words = list(meta.cu_block_lens)
    if n & 1:
        words.append(0)  # the int64 part starts 8-byte aligned
    pad = len(words)
    for x in meta.tri_prefix:
        words += (x & 0xFFFFFFFF, x >> 32)
    for x in meta.tri_prefix:
        x *= groups
        words += (x & 0xFFFFFFFF, x >> 32)
    # int32 words of nonnegative values below 2^63 (the high words stay below 2^31)
    dev = torch.tensor([w - (1 << 32) if w >= 1 << 31 else w for w in words], dtype=torch.int32).to(cu_seqlens.device)
    wide = dev[pad:].view(torch.int64)
    seqs = PackedSequences(cu_seqlens=cu_seqlens, cu_block_lens=dev[:n], tile_prefix=wide[:n], meta=meta)
    _TILE_PREFIX_TIMES.setdefault(seqs, {})[groups] = wide[n:]
    return seqs


# tile_prefix * groups per PackedSequences, kept with it.
_TILE_PREFIX_TIMES: "weakref.WeakKeyDictionary[PackedSequences, dict[int, torch.Tensor]]" = weakref.WeakKeyDictionary()


def tile_prefix_times(seqs: PackedSequences, groups: int) -> torch.Tensor:
    """``seqs.tile_prefix * groups`` on the device (the k2q build's per-sequence counter
    offsets), computed on the first request for a ``groups`` and kept with ``seqs``."""
    cache = _TILE_PREFIX_TIMES.setdefault(seqs, {})
    tri = cache.get(groups)
    if tri is None:
        tri = cache[groups] = seqs.tile_prefix * groups
    return tri


# PackedSequences re-described for other block sizes, kept with the original.
_OTHER_BLOCK_SIZES: "weakref.WeakKeyDictionary[PackedSequences, dict[int, PackedSequences]]" = weakref.WeakKeyDictionary()


def with_block_size(seqs: PackedSequences, block_size: int) -> PackedSequences:
    """``seqs`` for another block size: the same ``cu_seqlens`` tensor, block metadata
    recomputed on the host from ``seqs.meta`` (no device read) and copied to the device
    on the first request only; later requests return the cached object."""
    if block_size == seqs.block_size:
        return seqs
    cache = _OTHER_BLOCK_SIZES.setdefault(seqs, {})
    if block_size not in cache:
        meta = sequence_meta(list(seqs.meta.bounds), block_size)
        cache[block_size] = PackedSequences(
            cu_seqlens=seqs.cu_seqlens,
            cu_block_lens=torch.tensor(meta.cu_block_lens, dtype=torch.int32, device=seqs.device),
            tile_prefix=torch.tensor(meta.tri_prefix, dtype=torch.int64, device=seqs.device),
            meta=meta,
        )
    return cache[block_size]


def prepared_for(seqs: PackedSequences, *, block_size: int, total_tokens: int, device: torch.device) -> SequenceMeta:
    """Check that prepared metadata fits an operator call; return its host metadata."""
    if seqs.block_size != block_size:
        raise ValueError("block_size differs from the block_size the sequences were prepared with")
    if seqs.total_tokens != total_tokens:
        raise ValueError("cu_seqlens must start at zero and end at total_tokens")
    if seqs.device != device:
        raise ValueError("prepared sequences must be on the input device")
    return seqs.meta
