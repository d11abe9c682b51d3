"""Stage 1: per-group causal block maxima of the indexer logits.

Mirrors triton/index_score.py:298-357 of the reference (signature, defaults,
validation order, messages and exception types) and its autograd contract
(:235-295): first-order gradients, with the winner state saved only when grad
is enabled and an input requires grad.

Numerics: each public score is the reference's fp32 form of the exact winning dot x
(index_score.py:121-127): hi = fl32(x), lo = fl32(x - hi), s = fl32(|scale|), score =
fl32(fl32(hi s) + fl32(lo s)), i.e. fl32(scale * x) when |scale| is 0, 1 or a power
of two. Winners are
decided on exact dot products (FP64 evaluation of bf16/fp16/fp32 products), so
ties are true mathematical ties and the backward splits ds*scale evenly across
them like ``torch.amax``. Saved state is one int32 tie/winner code per score
(offset+1, or -count), versus max_hi/max_lo/tie_info in the reference.
"""

from __future__ import annotations

import math

import torch

from . import _lib
from .layout import PackedSequences, prepared_for, sequence_meta


def _score_forward(q, k, cu, meta, max_seqlen, block_size, scale, save_state):
    """Forward launch on contiguous inputs: (scores, tie codes or None)."""
    total, groups, dim = q.shape
    blocks = (max_seqlen + block_size - 1) // block_size
    scores = torch.empty((total, groups, blocks), dtype=torch.float32, device=q.device)
    tie = torch.empty((total, groups, blocks), dtype=torch.int32, device=q.device) if save_state else None
    if total:
        lib = _lib.lib()
        workspace = torch.empty(lib.msa_score_fwd_workspace_bytes(total, groups, blocks), dtype=torch.uint8, device=q.device)
        with torch.cuda.device(q.device):
            status = lib.msa_score_fwd(
                q.data_ptr(), k.data_ptr(), _lib.DTYPE_CODE[q.dtype], cu.data_ptr(), meta.num_seqs,
                total, groups, dim, blocks, block_size, scale, scores.data_ptr(),
                None if tie is None else tie.data_ptr(), workspace.data_ptr(), _lib.stream_of(q.device),
            )
        _lib.check(status, "msa_score_fwd")
    return scores, tie


def _score_backward(q, k, cu, tie, grad_scores, meta, blocks, scale, need_q, need_k, cu_blocks=None):
    """Backward launch: (dq, dk), None where not needed."""
    total, groups, dim = q.shape
    dq = torch.empty_like(q) if need_q else None
    dk = torch.empty_like(k) if need_k else None
    if total and (dq is not None or dk is not None):
        ds = grad_scores.to(torch.float32).contiguous()
        if cu_blocks is None:
            cu_blocks = torch.tensor(meta.cu_block_lens, dtype=torch.int32, device=q.device)
        lib = _lib.lib()
        ws_bytes = (lib.msa_score_bwd_workspace_bytes(total, groups, blocks, dim, meta.block_size,
                                                     meta.total_blocks) if dk is not None else 0)
        workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
        with torch.cuda.device(q.device):
            status = lib.msa_score_bwd(
                q.data_ptr(), k.data_ptr(), _lib.DTYPE_CODE[q.dtype], cu.data_ptr(), cu_blocks.data_ptr(),
                tie.data_ptr(), ds.data_ptr(), meta.num_seqs, total, groups, dim, blocks,
                meta.block_size, meta.total_blocks, scale, _lib.ptr(dq), _lib.ptr(dk),
                workspace.data_ptr(), _lib.stream_of(q.device),
            )
        _lib.check(status, "msa_score_bwd")
    return dq, dk


class _IndexScore(torch.autograd.Function):
    @staticmethod
    def forward(ctx, index_q, index_k, cu_seqlens, max_seqlen, block_size, scale, save_state, meta, cu_blocks):
        q = index_q.contiguous()
        k = index_k.contiguous()
        cu = cu_seqlens.contiguous()
        scores, tie = _score_forward(q, k, cu, meta, max_seqlen, block_size, scale, save_state)
        if save_state:
            ctx.save_for_backward(q, k, cu, tie)
        ctx.meta = meta
        ctx.cu_blocks = cu_blocks  # prepared device copy of cu_block_lens, or None
        ctx.scale = scale
        ctx.blocks = scores.shape[2]
        return scores

    @staticmethod
    def backward(ctx, grad_scores):
        q, k, cu, tie = ctx.saved_tensors
        dq, dk = _score_backward(q, k, cu, tie, grad_scores, ctx.meta, ctx.blocks, ctx.scale,
                                 ctx.needs_input_grad[0], ctx.needs_input_grad[1], ctx.cu_blocks)
        return dq, dk, None, None, None, None, None, None, None


def _validate(index_q, index_k, cu_seqlens, max_seqlen, block_size, scale):
    """m3_index_score's checks, in the reference's order; returns (cu, meta, seqs, save_state)."""
    if index_q.ndim != 3 or index_k.ndim != 3:
        raise ValueError("index_q and index_k must be rank-3 TND tensors")
    total, groups, dim = index_q.shape
    if groups < 1 or dim < 1 or index_k.shape != (total, 1, dim):
        raise ValueError("expected index_q[T,G,Di] and index_k[T,1,Di] with G, Di > 0")
    if index_q.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError("index_q must have BF16, FP16, or FP32 dtype")
    if index_k.dtype != index_q.dtype or index_k.device != index_q.device:
        raise ValueError("index_q and index_k must share dtype and device")
    seqs = cu_seqlens if isinstance(cu_seqlens, PackedSequences) else None
    cu = seqs.cu_seqlens if seqs is not None else cu_seqlens
    if cu.ndim != 1 or cu.numel() < 2 or cu.dtype != torch.int32:
        raise ValueError("cu_seqlens must be a rank-1 int32 tensor with at least two entries")
    if cu.device != index_q.device:
        raise ValueError("cu_seqlens must be on the input device")
    if not isinstance(block_size, int) or block_size <= 0:
        raise ValueError("block_size must be a positive integer")
    if not isinstance(max_seqlen, int) or max_seqlen <= 0:
        raise ValueError("max_seqlen must be a positive integer")
    if total > 2147483647 or cu.numel() - 1 > 2147483647:
        raise ValueError("packed token and sequence counts must fit int32 metadata")
    if block_size > 2147483647 or max_seqlen > 2147483647:
        raise ValueError("block_size and max_seqlen must fit int32 metadata")
    if not math.isfinite(scale):
        raise ValueError("scale must be finite")
    if seqs is None:
        boundaries = cu.detach().cpu().tolist()
        lengths = [end - start for start, end in zip(boundaries, boundaries[1:])]
        if boundaries[0] != 0 or boundaries[-1] != total or any(n < 0 for n in lengths):
            raise ValueError("cu_seqlens must span T with nondecreasing boundaries starting at zero")
        meta = sequence_meta(boundaries, block_size)
    else:  # prepared: no host read
        meta = prepared_for(seqs, block_size=block_size, total_tokens=total, device=index_q.device)
        lengths = list(meta.lengths)
    if max(lengths) > max_seqlen:
        raise ValueError("max_seqlen is smaller than a packed sequence")
    _lib.require_gpu(index_q, "m3_index_score")
    save_state = torch.is_grad_enabled() and (index_q.requires_grad or index_k.requires_grad)
    return cu, meta, seqs, save_state


def m3_index_score(
    index_q: torch.Tensor,
    index_k: torch.Tensor,
    cu_seqlens: torch.Tensor,
    max_seqlen: int,
    *,
    block_size: int = 128,
    scale: float = 1.0,
) -> torch.Tensor:
    """Return per-group causal block maxima as FP32 ``[T, G, Bmax]``.

    ``index_q`` is ``[T,G,Di]`` and ``index_k`` is ``[T,1,Di]``. Blocks are
    relative to the start of each packed sequence. Future and out-of-sequence
    blocks return ``-inf`` and have zero derivative. Exact max ties share the
    gradient equally, matching ``torch.amax``. Inputs must be finite.
    Metadata validation reads ``cu_seqlens`` on the host.
    """
    cu, meta, seqs, save_state = _validate(index_q, index_k, cu_seqlens, max_seqlen, block_size, scale)
    return _IndexScore.apply(index_q, index_k, cu, max_seqlen, block_size, float(scale), save_state, meta,
                             None if seqs is None else seqs.cu_block_lens)



class _IndexScoreTopk(torch.autograd.Function):
    """Scores with the top-k selection from the same launch; indices carry no gradient."""

    @staticmethod
    def forward(ctx, index_q, index_k, cu_seqlens, max_seqlen, block_size, scale, save_state, meta, cu_blocks,
                topk_blocks, local_blocks):
        q = index_q.contiguous()
        k = index_k.contiguous()
        cu = cu_seqlens.contiguous()
        total, groups, dim = q.shape
        blocks = (max_seqlen + block_size - 1) // block_size
        scores = torch.empty((total, groups, blocks), dtype=torch.float32, device=q.device)
        tie = torch.empty((total, groups, blocks), dtype=torch.int32, device=q.device) if save_state else None
        indices = torch.empty((total, groups, topk_blocks), dtype=torch.int32, device=q.device)
        if total:
            lib = _lib.lib()
            workspace = torch.empty(lib.msa_score_fwd_workspace_bytes(total, groups, blocks), dtype=torch.uint8, device=q.device)
            with torch.cuda.device(q.device):
                status = lib.msa_index_score_topk(
                    q.data_ptr(), k.data_ptr(), _lib.DTYPE_CODE[q.dtype], cu.data_ptr(), meta.num_seqs,
                    total, groups, dim, blocks, block_size, scale, topk_blocks, local_blocks, scores.data_ptr(),
                    None if tie is None else tie.data_ptr(), indices.data_ptr(), workspace.data_ptr(),
                    _lib.stream_of(q.device),
                )
            _lib.check(status, "msa_index_score_topk")
        if save_state:
            ctx.save_for_backward(q, k, cu, tie)
        ctx.meta = meta
        ctx.cu_blocks = cu_blocks
        ctx.scale = scale
        ctx.blocks = blocks
        ctx.mark_non_differentiable(indices)
        return scores, indices

    @staticmethod
    def backward(ctx, grad_scores, grad_indices):
        q, k, cu, tie = ctx.saved_tensors
        dq, dk = _score_backward(q, k, cu, tie, grad_scores, ctx.meta, ctx.blocks, ctx.scale,
                                 ctx.needs_input_grad[0], ctx.needs_input_grad[1], ctx.cu_blocks)
        return dq, dk, None, None, None, None, None, None, None, None, None


def m3_index_score_topk(index_q, index_k, cu_seqlens, max_seqlen, *, block_size=128, scale=1.0, topk_blocks=16,
                        local_blocks=1):
    """``m3_index_score`` and ``m3_topk`` of its scores in one call: ``(scores, indices)``.

    Equal, bit for bit, to ``m3_topk(m3_index_score(...), ...)`` with the same
    arguments; the scores keep their gradient, the indices have none. One C call
    (``msa_index_score_topk``) launches both kernels back to back.
    """
    if not isinstance(topk_blocks, int) or topk_blocks < 0:
        raise ValueError("topk_blocks must be a nonnegative integer")
    if not isinstance(local_blocks, int) or not 0 <= local_blocks <= topk_blocks:
        raise ValueError("local_blocks must satisfy 0 <= local_blocks <= topk_blocks")
    cu, meta, seqs, save_state = _validate(index_q, index_k, cu_seqlens, max_seqlen, block_size, scale)
    return _IndexScoreTopk.apply(index_q, index_k, cu, max_seqlen, block_size, float(scale), save_state, meta,
                                 None if seqs is None else seqs.cu_block_lens, topk_blocks, local_blocks)
