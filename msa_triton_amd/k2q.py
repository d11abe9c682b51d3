"""Block->query CSR ("k2q") for the KV-owned sparse backward.

Mirrors triton/k2q.py:20-128 of the reference: the ``K2QCSR`` record layout,
validation order, messages (``"span T"``, ``"nondecreasing"``, ``"block_size"``,
``OverflowError("... edge capacity")``) and the bit-level contract of the four
int32 outputs. The build runs as HIP kernels (``msa_k2q_build``): a per-query-
block histogram, a per-row prefix over tiles, a row-pointer scan and an ordered
scatter, instead of the reference's int64 argsort. Sequence metadata is read on
the host once, as in the reference, or taken from ``PackedSequences`` without a
host read.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib
from .layout import PackedSequences, prepared_for, sequence_meta, tile_prefix_times, with_block_size

_INT32_MAX = 2**31 - 1


@dataclass(frozen=True)
class K2QCSR:
    """Reverse sparse edges, with every tensor on the indices device.

    ``row_ptr`` has ``total_blocks * G + 1`` int32 elements. Row
    ``global_block * G + group`` holds global packed query token ids in
    ``query_indices`` and their selection slots in ``slot_indices``. Both edge
    arrays have capacity ``T * G * K``; entries beyond ``row_ptr[-1]`` are
    ``-1``. ``cu_block_lens`` is the int32 prefix sum of each sequence's block
    count. Within a row, edges are ordered by query token, then slot; duplicate
    selections keep one edge per slot.
    """

    row_ptr: torch.Tensor
    query_indices: torch.Tensor
    slot_indices: torch.Tensor
    cu_block_lens: torch.Tensor


@torch.no_grad()
def build_k2q_csr(indices: torch.Tensor, cu_seqlens: torch.Tensor, *, block_size: int) -> K2QCSR:
    """Invert ``indices[T,G,K]`` into deterministic block/group CSR rows.

    Negative, future and out-of-sequence block ids produce no edge. A query
    selecting its current block does produce an edge (the consumer applies the
    token-level causal mask). Empty sequences, T=0 and K=0 are supported.
    """
    if indices.ndim != 3 or indices.dtype != torch.int32:
        raise ValueError("indices must be an int32 tensor with shape [T,G,K]")
    total, groups, slots = indices.shape
    if groups <= 0:
        raise ValueError("indices must have at least one group")
    if not isinstance(block_size, int) or isinstance(block_size, bool) or block_size <= 0:
        raise ValueError("block_size must be a positive integer")
    seqs = cu_seqlens if isinstance(cu_seqlens, PackedSequences) else None
    cu = seqs.cu_seqlens if seqs is not None else cu_seqlens
    if cu.ndim != 1 or cu.dtype != torch.int32 or cu.numel() < 2:
        raise ValueError("cu_seqlens must be a rank-1 int32 tensor with at least two entries")
    if cu.device != indices.device:
        raise ValueError("cu_seqlens and indices must be on the same device")
    capacity = total * groups * slots
    # Protects the int32 CSR counts and positions.
    if capacity > _INT32_MAX:
        raise OverflowError("T * G * K exceeds int32 edge capacity")
    if seqs is None:
        bounds = cu.detach().cpu().tolist()
        lengths = [end - start for start, end in zip(bounds[:-1], bounds[1:])]
        if bounds[0] != 0 or bounds[-1] != total or any(length < 0 for length in lengths):
            raise ValueError("cu_seqlens must span T with nondecreasing boundaries starting at zero")
        meta = sequence_meta(bounds, block_size)
    else:  # prepared: no host read
        meta = prepared_for(seqs, block_size=block_size, total_tokens=total, device=indices.device)
    num_rows = meta.total_blocks * groups
    if num_rows >= _INT32_MAX:
        raise OverflowError("block/group row pointer length exceeds int32 indexing capacity")
    _lib.require_gpu(indices, "build_k2q_csr")
    return _build_device(indices.contiguous(), cu.contiguous(), meta, groups, slots, seqs)


def _build_device(indices, cu_seqlens, meta, groups, slots, seqs=None) -> K2QCSR:
    device = indices.device
    total = indices.shape[0]
    capacity = total * groups * slots
    num_rows = meta.total_blocks * groups
    if seqs is None:
        cu_block_lens = torch.tensor(meta.cu_block_lens, dtype=torch.int32, device=device)
        tri = torch.tensor([groups * x for x in meta.tri_prefix], dtype=torch.int64, device=device)
    else:  # prepared device copies (no host-to-device copy: capturable after the first call per G)
        cu_block_lens = seqs.cu_block_lens
        tri = tile_prefix_times(seqs, groups)
    counter_elems = groups * meta.tri_prefix[-1]
    row_ptr = torch.empty(num_rows + 1, dtype=torch.int32, device=device)
    query_indices = torch.empty(capacity, dtype=torch.int32, device=device)
    slot_indices = torch.empty(capacity, dtype=torch.int32, device=device)
    workspace = torch.empty(max(1, counter_elems + num_rows), dtype=torch.int32, device=device)
    with torch.cuda.device(device):
        status = _lib.lib().msa_k2q_build(
            indices.data_ptr(), cu_seqlens.data_ptr(), cu_block_lens.data_ptr(), tri.data_ptr(),
            meta.num_seqs, total, groups, slots, meta.block_size, meta.total_blocks, counter_elems,
            row_ptr.data_ptr(), query_indices.data_ptr(), slot_indices.data_ptr(), workspace.data_ptr(),
            _lib.stream_of(device),
        )
    _lib.check(status, "msa_k2q_build")
    return K2QCSR(row_ptr, query_indices, slot_indices, cu_block_lens)


# At most this many sub-blocks per block (partial records, CSR edges and work grow with
# the sub-block slot count).
MAX_SUB_BLOCKS = 8


def sub_block_selection(indices, meta, block_size, seqs, fits):
    """The selection with blocks of more than 128 keys (the MFMA kernels' tile) cut into
    f sub-blocks of ``block_size / f`` keys: (indices, meta, block_size, seqs).

    f is the smallest divisor of ``block_size`` in [ceil(block_size / 128), 8] for which
    ``fits(f, sub_block_size, sub_meta)`` holds; ``msa_split_block_indices`` maps id b to
    f b .. f b + f - 1, which hold exactly block b's keys (a sub-block that starts after
    the query is skipped by the same id <= query-block rule). Returned unchanged when
    ``block_size <= 128`` or no such f exists."""
    total, groups, slots = indices.shape
    if block_size <= 128 or not total:
        return indices, meta, block_size, seqs
    for factor in range(-(-block_size // 128), MAX_SUB_BLOCKS + 1):
        if block_size % factor:
            continue
        sub = block_size // factor
        sub_meta = sequence_meta(list(meta.bounds), sub)
        if not fits(factor, sub, sub_meta):
            break
        split = torch.empty((total, groups, slots * factor), dtype=torch.int32, device=indices.device)
        with torch.cuda.device(indices.device):
            status = _lib.lib().msa_split_block_indices(indices.data_ptr(), total * groups, slots, factor,
                                                        split.data_ptr(), _lib.stream_of(indices.device))
        _lib.check(status, "msa_split_block_indices")
        if seqs is None:
            return split, sub_meta, sub, None
        sub_seqs = with_block_size(seqs, sub)
        return split, sub_seqs.meta, sub, sub_seqs
    return indices, meta, block_size, seqs
