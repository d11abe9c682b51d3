"""Indexer KL: the training branch that consumes the selection.

The reference describes this loss (docs/msa_training_flow.md:92-138) and leaves it
unimplemented (docs/implementation_plan.md:66-69); there is no reference signature,
so this operator follows the conventions of the three operators around it (TND
tensors, int32 ``cu_seqlens`` or ``PackedSequences``, ``block_size``, the score's
``scale`` as ``index_scale`` and the attention's ``scale``).

Over the causal tokens of each (token, group)'s selected blocks:

* student: softmax of the index token logits ``index_scale * index_q[t,g] . index_k[j]``
  (token logits, not block maxima, and no local ``+inf`` boost);
* teacher: the mean over the group's ``Hq / G`` query heads of the attention
  probabilities ``softmax(scale * q[t,h] . k[j,g])`` -- ``q`` and ``k`` are treated
  as detached (the teacher receives no gradient);
* loss: ``KL(teacher || student)`` averaged over the ``T * G`` (token, group) pairs
  (pairs without visible keys contribute 0).

Execution: ``msa_indexer_kl`` (two KV-major MFMA passes over the selection's k2q
CSR, deterministic). The forward also produces the fp32 gradients of the loss when
``index_q`` or ``index_k`` requires grad; the backward scales them by the incoming
gradient. bf16 or fp16 (all four inputs of one dtype), head and index dims of 32, 64 or
128, at most 8 query heads per group, block size up to 128 (larger blocks run as f <= 8
sub-blocks of at most 128 keys when f divides the block size: the same keys, so the same
loss); other configurations raise ``NotImplementedError``.
"""

from __future__ import annotations

import math

import torch

from . import _lib
from . import k2q as _k2q
from .layout import PackedSequences, prepared_for, sequence_lengths, sequence_meta


def _launch(iq, ik, q, k, indices, cu, meta, seqs, block_size, index_scale, scale, want_rows, need_q, need_k,
            teacher_lse=None):
    total, groups, dim_i = iq.shape
    heads, dim = q.shape[1], q.shape[2]
    lib = _lib.lib()
    if q.dtype != iq.dtype:  # the kernels take one input type for all four tensors
        raise NotImplementedError("m3_indexer_kl takes index_q / index_k and q / k of one dtype")

    def fits(factor, sub, sub_meta):
        return lib.msa_indexer_kl_workspace_bytes(_lib.DTYPE_CODE[iq.dtype], total, heads, groups, dim, dim_i,
                                                  indices.shape[2] * factor, sub_meta.total_blocks, sub) > 0

    # blocks above 128 keys as sub-blocks of the same keys (the loss is over keys, not blocks)
    indices, meta, block_size, seqs = _k2q.sub_block_selection(indices, meta, block_size, seqs, fits)
    slots = indices.shape[2]
    ws_bytes = lib.msa_indexer_kl_workspace_bytes(_lib.DTYPE_CODE[iq.dtype], total, heads, groups, dim, dim_i,
                                                  slots, meta.total_blocks, block_size)
    if total and ws_bytes == 0:
        raise NotImplementedError(
            "m3_indexer_kl supports bf16 or fp16 inputs with head and index dims of 32, 64 or 128, at most 8 "
            "query heads per group and block_size <= 128 (or a multiple of at most 8 sub-blocks of <= 128)")
    device = iq.device
    loss = torch.zeros(1, dtype=torch.float32, device=device)
    row_kl = torch.zeros((total, groups), dtype=torch.float32, device=device) if want_rows else None
    d_iq = torch.empty((total, groups, dim_i), dtype=torch.float32, device=device) if need_q else None
    d_ik = torch.empty((total, 1, dim_i), dtype=torch.float32, device=device) if need_k else None
    if total:
        csr = _k2q._build_device(indices, cu, meta, groups, slots, seqs)
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
        with torch.cuda.device(device):
            status = lib.msa_indexer_kl(
                iq.data_ptr(), ik.data_ptr(), q.data_ptr(), k.data_ptr(), _lib.DTYPE_CODE[iq.dtype],
                indices.data_ptr(), cu.data_ptr(), meta.num_seqs, total, heads, groups, dim, dim_i, slots,
                block_size, index_scale, scale, csr.cu_block_lens.data_ptr(), meta.total_blocks,
                csr.row_ptr.data_ptr(), _lib.ptr(csr.query_indices), _lib.ptr(csr.slot_indices),
                _lib.ptr(teacher_lse), loss.data_ptr(),
                _lib.ptr(row_kl), _lib.ptr(d_iq), _lib.ptr(d_ik), workspace.data_ptr(), ws_bytes,
                _lib.stream_of(device))
        _lib.check(status, "msa_indexer_kl")
    return loss[0], row_kl, d_iq, d_ik


class _IndexerKL(torch.autograd.Function):
    @staticmethod
    def forward(ctx, iq, ik, q, k, indices, cu, meta, seqs, block_size, index_scale, scale, want_rows, teacher_lse):
        need_q, need_k = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        loss, row_kl, d_iq, d_ik = _launch(iq.contiguous(), ik.contiguous(), q.detach().contiguous(),
                                           k.detach().contiguous(), indices.contiguous(), cu, meta, seqs, block_size,
                                           index_scale, scale, want_rows, need_q, need_k, teacher_lse)
        ctx.save_for_backward(d_iq, d_ik)
        ctx.dtypes = (iq.dtype, ik.dtype)
        if row_kl is None:
            row_kl = loss.new_zeros(0)
        ctx.mark_non_differentiable(row_kl)
        return loss, row_kl

    @staticmethod
    def backward(ctx, grad_loss, grad_rows):
        d_iq, d_ik = ctx.saved_tensors
        g = grad_loss.to(torch.float32)
        diq = (d_iq * g).to(ctx.dtypes[0]) if d_iq is not None else None
        dik = (d_ik * g).to(ctx.dtypes[1]) if d_ik is not None else None
        return diq, dik, None, None, None, None, None, None, None, None, None, None, None


def m3_indexer_kl(
    index_q: torch.Tensor,
    index_k: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    indices: torch.Tensor,
    cu_seqlens: torch.Tensor | PackedSequences,
    max_seqlen: int,
    *,
    block_size: int = 128,
    index_scale: float = 1.0,
    scale: float | None = None,
    return_rows: bool = False,
    teacher_lse: torch.Tensor | None = None,
):
    """KL(stopgrad(teacher) || student) over the selected causal tokens, averaged over
    (token, group) pairs: a differentiable fp32 scalar (gradients reach ``index_q`` and
    ``index_k`` only). With ``return_rows`` also the per-pair KL ``[T, G]`` (fp32,
    non-differentiable). ``teacher_lse``: the lse ``m3_sparse_attention(...,
    return_lse=True)`` returned for the same ``q``, ``k``, ``indices``, ``block_size``
    and ``scale`` (fp32 ``[T, Hq]``); the teacher's normalisers are then taken from it
    instead of being recomputed (about a quarter of the work)."""
    if index_q.ndim != 3 or index_k.ndim != 3 or q.ndim != 3 or k.ndim != 3:
        raise ValueError("expected index_q[T,G,Di], index_k[T,1,Di], q[T,Hq,D] and k[T,G,D]")
    total, groups, dim_i = index_q.shape
    if groups < 1 or dim_i < 1 or index_k.shape != (total, 1, dim_i):
        raise ValueError("expected index_q[T,G,Di] and index_k[T,1,Di] with G, Di > 0")
    if k.shape[:2] != (total, groups) or q.shape[0] != total or q.shape[2] != k.shape[2] or k.shape[2] < 1:
        raise ValueError("expected q[T,Hq,D] and k[T,G,D] matching index_q's tokens and groups")
    if q.shape[1] % groups or q.shape[1] == 0:
        raise ValueError("Hq must be a positive multiple of G")
    if indices.ndim != 3 or indices.shape[:2] != (total, groups) or indices.dtype != torch.int32:
        raise ValueError("indices must be int32 [T,G,K]")
    if index_q.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError("index_q must have BF16, FP16, or FP32 dtype")
    if index_k.dtype != index_q.dtype or q.dtype != k.dtype or q.dtype not in (torch.bfloat16, torch.float16,
                                                                               torch.float32):
        raise TypeError("index_q / index_k and q / k must each share a BF16, FP16, or FP32 dtype")
    seqs = cu_seqlens if isinstance(cu_seqlens, PackedSequences) else None
    cu = seqs.cu_seqlens if seqs is not None else cu_seqlens
    if cu.ndim != 1 or cu.numel() < 2 or cu.dtype != torch.int32:
        raise ValueError("cu_seqlens must be int32 [num_sequences + 1]")
    if any(x.device != index_q.device for x in (index_k, q, k, indices, cu)):
        raise ValueError("all inputs must reside on the same device")
    if not isinstance(block_size, int) or block_size <= 0:
        raise ValueError("block_size must be a positive integer")
    if not isinstance(max_seqlen, int) or max_seqlen <= 0:
        raise ValueError("max_seqlen must be a positive integer")
    effective_scale = q.shape[-1] ** -0.5 if scale is None else float(scale)
    if not math.isfinite(effective_scale) or not math.isfinite(index_scale):
        raise ValueError("scale and index_scale must be finite")
    if teacher_lse is not None:
        if teacher_lse.shape != q.shape[:2] or teacher_lse.dtype != torch.float32:
            raise ValueError("teacher_lse must be the fp32 [T, Hq] lse of the attention")
        if teacher_lse.device != index_q.device:
            raise ValueError("all inputs must reside on the same device")
        teacher_lse = teacher_lse.detach().contiguous()
    if seqs is None:
        lengths = sequence_lengths(cu, total)
    else:  # prepared: no host read
        lengths = list(prepared_for(seqs, block_size=block_size, total_tokens=total, device=index_q.device).lengths)
    if max(lengths) > max_seqlen:
        raise ValueError("max_seqlen is smaller than an actual sequence")
    _lib.require_gpu(index_q, "m3_indexer_kl")
    if seqs is None:
        bounds = [0]
        for length in lengths:
            bounds.append(bounds[-1] + length)
        meta = sequence_meta(bounds, block_size)
    else:
        meta = seqs.meta
    loss, rows = _IndexerKL.apply(index_q, index_k, q, k, indices, cu, meta, seqs, block_size, float(index_scale),
                                  effective_scale, return_rows, teacher_lse)
    return (loss, rows) if return_rows else loss
