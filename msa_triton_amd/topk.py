"""Stage 2: causal top-k block selection with forced local blocks.

Mirrors triton/topk.py:11-47 of the reference: same signature, validation order,
messages and output contract (int32 ``[T,G,K]``, left-aligned distinct blocks,
``-1`` padding, no gradient, input never mutated). The selection itself runs in
one HIP kernel (``msa_topk``): one wavefront per (token, group) row, so no
masked ``[T,G,NB]`` temporaries are materialised.

Order contract: slots are in descending score order; equal values (including
several forced ``+inf`` local blocks) appear in ascending block order.
"""

from __future__ import annotations

import torch

from . import _lib
from .layout import PackedSequences, prepared_for


@torch.no_grad()
def m3_topk(scores, cu_seqlens, *, block_size=128, topk_blocks=16, local_blocks=1):
    if scores.ndim != 3 or scores.dtype != torch.float32:
        raise ValueError("scores must be FP32 [T,G,Bmax]")
    seqs = cu_seqlens if isinstance(cu_seqlens, PackedSequences) else None
    cu = seqs.cu_seqlens if seqs is not None else cu_seqlens
    if cu.ndim != 1 or cu.numel() < 2 or cu.dtype != torch.int32:
        raise ValueError("cu_seqlens must be an int32 vector with at least two entries")
    if cu.device != scores.device:
        raise ValueError("scores and cu_seqlens must share a device")
    if not isinstance(block_size, int) or block_size <= 0:
        raise ValueError("block_size must be a positive integer")
    if not isinstance(topk_blocks, int) or topk_blocks < 0:
        raise ValueError("topk_blocks must be a nonnegative integer")
    if not isinstance(local_blocks, int) or not 0 <= local_blocks <= topk_blocks:
        raise ValueError("local_blocks must satisfy 0 <= local_blocks <= topk_blocks")
    total, groups, blocks = scores.shape
    if seqs is None:
        boundaries = cu.detach().cpu().tolist()
        if boundaries[0] != 0 or boundaries[-1] != total or any(b < a for a, b in zip(boundaries, boundaries[1:])):
            raise ValueError("cu_seqlens must start at 0, be nondecreasing, and end at T")
    else:  # prepared: no host read
        boundaries = list(prepared_for(seqs, block_size=block_size, total_tokens=total, device=scores.device).bounds)
    if groups <= 0 or blocks <= 0 or any(b - a > blocks * block_size for a, b in zip(boundaries, boundaries[1:])):
        raise ValueError("scores need positive G and enough block slots for every sequence")
    _lib.require_gpu(scores, "m3_topk")
    result = torch.empty((total, groups, topk_blocks), dtype=torch.int32, device=scores.device)
    if total == 0 or topk_blocks == 0:
        return result.fill_(-1)
    scores = scores.contiguous()
    cu = cu.contiguous()
    with torch.cuda.device(scores.device):
        status = _lib.lib().msa_topk(
            scores.data_ptr(), cu.data_ptr(), len(boundaries) - 1, total, groups, blocks, block_size,
            topk_blocks, local_blocks, result.data_ptr(), _lib.stream_of(scores.device),
        )
    _lib.check(status, "msa_topk")
    return result
