"""torch.library registration of the three operators, for torch.compile.

The reference names this as follow-on work (docs/code_review.md:321-322; a
``torch.library`` custom op with fake/meta kernels). Here the HIP launches are
registered as opaque custom ops in the ``msa_mi355x`` namespace, each with a fake
implementation (output shapes and dtypes only, no data access) and, for score and
attention, a registered backward op, so ``torch.compile`` traces a layer without
graph breaks and AOTAutograd differentiates it:

    msa_mi355x::index_score(index_q, index_k, cu_seqlens, max_seqlen, block_size, scale, save_state)
        -> (scores, tie)           tie: int32 winner codes, or an empty tensor when not saved
    msa_mi355x::index_score_backward(index_q, index_k, cu_seqlens, tie, grad_scores, max_seqlen,
                                     block_size, scale, need_q, need_k) -> (dq, dk)
    msa_mi355x::topk(scores, cu_seqlens, block_size, topk_blocks, local_blocks) -> indices
    msa_mi355x::sparse_attention(q, k, v, indices, cu_seqlens, max_seqlen, block_size, scale, save_state)
        -> (out, lse, row_state, out_f32)   row_state: the fp64 per-row state the backward reads;
                                            out_f32: the fp32 output, or an empty tensor when not saved
    msa_mi355x::sparse_attention_backward(q, k, v, indices, cu_seqlens, out, row_state, out_f32, grad_out,
                                          block_size, scale, need_q, need_k, need_v) -> (dq, dk, dv)
    msa_mi355x::indexer_kl(index_q, index_k, q, k, indices, cu_seqlens, max_seqlen, block_size, index_scale,
                           scale, need_q, need_k, teacher_lse) -> (loss, row_kl, d_iq, d_ik)
                                               d_iq / d_ik: fp32 gradients of loss, empty when not wanted

A gradient that is not needed comes back as an empty tensor. ``m3_index_score``,
``m3_topk`` and ``m3_sparse_attention`` below keep the public signatures: their
static checks (ranks, dtypes, devices) run in Python, the metadata checks that read
``cu_seqlens`` run inside the ops when they execute, with the same messages.
Importing this module registers the ops; it does not load the HIP library.
"""

from __future__ import annotations

import math
from typing import Optional

import torch
from torch import Tensor

from . import _lib
from .index_score import _score_backward, _score_forward
from .indexer_kl import _launch as _kl_launch
from .layout import sequence_lengths, sequence_meta
from .sparse_attention import _attn_backward, _attn_forward
from .topk import m3_topk as _eager_topk

_NS = "msa_mi355x"


def _score_meta(cu_seqlens, total, max_seqlen, block_size):
    """The eager operator's metadata checks (index_score.py), at execution time."""
    boundaries = cu_seqlens.detach().cpu().tolist()
    lengths = [end - start for start, end in zip(boundaries, boundaries[1:])]
    if boundaries[0] != 0 or boundaries[-1] != total or any(n < 0 for n in lengths):
        raise ValueError("cu_seqlens must span T with nondecreasing boundaries starting at zero")
    if max(lengths) > max_seqlen:
        raise ValueError("max_seqlen is smaller than a packed sequence")
    return sequence_meta(boundaries, block_size)


def _attention_meta(cu_seqlens, total, max_seqlen, block_size):
    """The eager operator's metadata checks (sparse_attention.py), at execution time."""
    lengths = sequence_lengths(cu_seqlens, total)
    if max(lengths) > max_seqlen:
        raise ValueError("max_seqlen is smaller than an actual sequence.")
    bounds = [0]
    for length in lengths:
        bounds.append(bounds[-1] + length)
    return sequence_meta(bounds, block_size)


# ---------------------------------------------------------------------------- score

@torch.library.custom_op(f"{_NS}::index_score", mutates_args=())
def _index_score(index_q: Tensor, index_k: Tensor, cu_seqlens: Tensor, max_seqlen: int, block_size: int,
                 scale: float, save_state: bool) -> tuple[Tensor, Tensor]:
    _lib.require_gpu(index_q, "m3_index_score")
    q, k, cu = index_q.contiguous(), index_k.contiguous(), cu_seqlens.contiguous()
    meta = _score_meta(cu, q.shape[0], max_seqlen, block_size)
    scores, tie = _score_forward(q, k, cu, meta, max_seqlen, block_size, scale, save_state)
    return scores, tie if tie is not None else torch.empty(0, dtype=torch.int32, device=q.device)


@_index_score.register_fake
def _(index_q, index_k, cu_seqlens, max_seqlen, block_size, scale, save_state):
    total, groups, _ = index_q.shape
    blocks = (max_seqlen + block_size - 1) // block_size
    scores = index_q.new_empty((total, groups, blocks), dtype=torch.float32)
    tie = index_q.new_empty((total, groups, blocks) if save_state else (0,), dtype=torch.int32)
    return scores, tie


@torch.library.custom_op(f"{_NS}::index_score_backward", mutates_args=())
def _index_score_backward(index_q: Tensor, index_k: Tensor, cu_seqlens: Tensor, tie: Tensor, grad_scores: Tensor,
                          max_seqlen: int, block_size: int, scale: float, need_q: bool,
                          need_k: bool) -> tuple[Tensor, Tensor]:
    q, k, cu = index_q.contiguous(), index_k.contiguous(), cu_seqlens.contiguous()
    meta = _score_meta(cu, q.shape[0], max_seqlen, block_size)
    blocks = (max_seqlen + block_size - 1) // block_size
    dq, dk = _score_backward(q, k, cu, tie, grad_scores, meta, blocks, scale, need_q, need_k)
    empty = q.new_empty(0)
    return dq if dq is not None else empty, dk if dk is not None else empty


@_index_score_backward.register_fake
def _(index_q, index_k, cu_seqlens, tie, grad_scores, max_seqlen, block_size, scale, need_q, need_k):
    return (index_q.new_empty(index_q.shape if need_q else (0,)),
            index_k.new_empty(index_k.shape if need_k else (0,)))


def _score_setup(ctx, inputs, output):
    index_q, index_k, cu_seqlens, max_seqlen, block_size, scale, save_state = inputs
    ctx.save_for_backward(index_q, index_k, cu_seqlens, output[1])
    ctx.args = (max_seqlen, block_size, scale)
    ctx.mark_non_differentiable(output[1])


def _score_grad(ctx, grad_scores, grad_tie):
    index_q, index_k, cu_seqlens, tie = ctx.saved_tensors
    need_q, need_k = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
    dq, dk = torch.ops.msa_mi355x.index_score_backward(index_q, index_k, cu_seqlens, tie, grad_scores, *ctx.args,
                                                       need_q, need_k)
    return (dq if need_q else None, dk if need_k else None, None, None, None, None, None)


torch.library.register_autograd(f"{_NS}::index_score", _score_grad, setup_context=_score_setup)


# ---------------------------------------------------------------------------- top-k

@torch.library.custom_op(f"{_NS}::topk", mutates_args=())
def _topk(scores: Tensor, cu_seqlens: Tensor, block_size: int, topk_blocks: int, local_blocks: int) -> Tensor:
    return _eager_topk(scores, cu_seqlens, block_size=block_size, topk_blocks=topk_blocks, local_blocks=local_blocks)


@_topk.register_fake
def _(scores, cu_seqlens, block_size, topk_blocks, local_blocks):
    return scores.new_empty((scores.shape[0], scores.shape[1], topk_blocks), dtype=torch.int32)


# ---------------------------------------------------------------------------- attention

@torch.library.custom_op(f"{_NS}::sparse_attention", mutates_args=())
def _sparse_attention(q: Tensor, k: Tensor, v: Tensor, indices: Tensor, cu_seqlens: Tensor, max_seqlen: int,
                      block_size: int, scale: float, save_state: bool) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    _lib.require_gpu(q, "m3_sparse_attention")
    cu = cu_seqlens.contiguous()
    meta = _attention_meta(cu, q.shape[0], max_seqlen, block_size)
    out, lse, row_state, out_f32, _ = _attn_forward(q.contiguous(), k.contiguous(), v.contiguous(),
                                                    indices.contiguous(), cu, meta, block_size, scale, None,
                                                    save_f32=save_state)
    row_state[..., 2:].zero_()  # lse and mass are forward state; the rest is the backward's scratch
    return out, lse, row_state, (out_f32 if out_f32 is not None else q.new_empty(0, dtype=torch.float32))


@_sparse_attention.register_fake
def _(q, k, v, indices, cu_seqlens, max_seqlen, block_size, scale, save_state):
    total, heads, dim = q.shape
    return (q.new_empty(q.shape), q.new_empty((total, heads), dtype=torch.float32),
            q.new_empty((total, heads, 4), dtype=torch.float64),
            q.new_empty((total, heads, dim) if save_state else (0,), dtype=torch.float32))


@torch.library.custom_op(f"{_NS}::sparse_attention_backward", mutates_args=())
def _sparse_attention_backward(q: Tensor, k: Tensor, v: Tensor, indices: Tensor, cu_seqlens: Tensor, out: Tensor,
                               row_state: Tensor, out_f32: Tensor, grad_out: Tensor, block_size: int, scale: float,
                               need_q: bool, need_k: bool, need_v: bool) -> tuple[Tensor, Tensor, Tensor]:
    cu = cu_seqlens.contiguous()
    meta = _attention_meta(cu, q.shape[0], max(1, q.shape[0]), block_size)
    # the backward writes its center into the row state: work on a copy (inputs are not mutated)
    dq, dk, dv = _attn_backward(q.contiguous(), k.contiguous(), v.contiguous(), indices.contiguous(), cu,
                                out.contiguous(), row_state.clone(), grad_out, meta, block_size, scale, None,
                                need_q, need_k, need_v,
                                out_f32=out_f32.contiguous() if out_f32.numel() else None)
    empty = q.new_empty(0)
    return (dq if dq is not None else empty, dk if dk is not None else empty, dv if dv is not None else empty)


@_sparse_attention_backward.register_fake
def _(q, k, v, indices, cu_seqlens, out, row_state, out_f32, grad_out, block_size, scale, need_q, need_k, need_v):
    return (q.new_empty(q.shape if need_q else (0,)), k.new_empty(k.shape if need_k else (0,)),
            v.new_empty(v.shape if need_v else (0,)))


def _attention_setup(ctx, inputs, output):
    q, k, v, indices, cu_seqlens, max_seqlen, block_size, scale, save_state = inputs
    out, lse, row_state, out_f32 = output
    ctx.save_for_backward(q, k, v, indices, cu_seqlens, out, row_state, out_f32)
    ctx.args = (block_size, scale)
    ctx.mark_non_differentiable(lse, row_state, out_f32)


def _attention_grad(ctx, grad_out, grad_lse, grad_row_state, grad_out_f32):
    q, k, v, indices, cu_seqlens, out, row_state, out_f32 = ctx.saved_tensors
    need = [bool(x) for x in ctx.needs_input_grad[:3]]
    if grad_out is None:
        grad_out = torch.zeros_like(out)
    dq, dk, dv = torch.ops.msa_mi355x.sparse_attention_backward(q, k, v, indices, cu_seqlens, out, row_state,
                                                                out_f32, grad_out, *ctx.args, *need)
    return (dq if need[0] else None, dk if need[1] else None, dv if need[2] else None, None, None, None, None, None,
            None)


torch.library.register_autograd(f"{_NS}::sparse_attention", _attention_grad, setup_context=_attention_setup)


# ---------------------------------------------------------------------------- indexer KL

@torch.library.custom_op(f"{_NS}::indexer_kl", mutates_args=())
def _indexer_kl(index_q: Tensor, index_k: Tensor, q: Tensor, k: Tensor, indices: Tensor, cu_seqlens: Tensor,
                max_seqlen: int, block_size: int, index_scale: float, scale: float, need_q: bool, need_k: bool,
                teacher_lse: Optional[Tensor]) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    _lib.require_gpu(index_q, "m3_indexer_kl")
    cu = cu_seqlens.contiguous()
    meta = _attention_meta(cu, index_q.shape[0], max_seqlen, block_size)
    loss, rows, d_iq, d_ik = _kl_launch(index_q.contiguous(), index_k.contiguous(), q.contiguous(), k.contiguous(),
                                        indices.contiguous(), cu, meta, None, block_size, index_scale, scale, True,
                                        need_q, need_k,
                                        teacher_lse.contiguous() if teacher_lse is not None else None)
    empty = loss.new_empty(0)
    return loss.clone(), rows, d_iq if d_iq is not None else empty, d_ik if d_ik is not None else empty


@_indexer_kl.register_fake
def _(index_q, index_k, q, k, indices, cu_seqlens, max_seqlen, block_size, index_scale, scale, need_q, need_k,
      teacher_lse):
    total, groups, dim_i = index_q.shape
    f32 = torch.float32
    return (index_q.new_empty((), dtype=f32), index_q.new_empty((total, groups), dtype=f32),
            index_q.new_empty((total, groups, dim_i) if need_q else (0,), dtype=f32),
            index_k.new_empty((total, 1, dim_i) if need_k else (0,), dtype=f32))


def _kl_setup(ctx, inputs, output):
    ctx.save_for_backward(output[2], output[3])
    ctx.dtypes = (inputs[0].dtype, inputs[1].dtype)
    ctx.mark_non_differentiable(output[1], output[2], output[3])


def _kl_grad(ctx, grad_loss, grad_rows, grad_diq, grad_dik):
    d_iq, d_ik = ctx.saved_tensors
    need_q, need_k = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
    g = grad_loss.to(torch.float32)
    return ((d_iq * g).to(ctx.dtypes[0]) if need_q else None, (d_ik * g).to(ctx.dtypes[1]) if need_k else None,
            None, None, None, None, None, None, None, None, None, None, None)


torch.library.register_autograd(f"{_NS}::indexer_kl", _kl_grad, setup_context=_kl_setup)


# ---------------------------------------------------------------------------- public wrappers

def m3_index_score(index_q, index_k, cu_seqlens, max_seqlen, *, block_size=128, scale=1.0):
    """``msa_triton_amd.m3_index_score`` through the registered op (same arguments and checks)."""
    if index_q.ndim != 3 or index_k.ndim != 3:
        raise ValueError("index_q and index_k must be rank-3 TND tensors")
    total, groups, dim = index_q.shape
    if groups < 1 or dim < 1 or index_k.shape != (total, 1, dim):
        raise ValueError("expected index_q[T,G,Di] and index_k[T,1,Di] with G, Di > 0")
    if index_q.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError("index_q must have BF16, FP16, or FP32 dtype")
    if index_k.dtype != index_q.dtype or index_k.device != index_q.device:
        raise ValueError("index_q and index_k must share dtype and device")
    if cu_seqlens.ndim != 1 or cu_seqlens.numel() < 2 or cu_seqlens.dtype != torch.int32:
        raise ValueError("cu_seqlens must be a rank-1 int32 tensor with at least two entries")
    if cu_seqlens.device != index_q.device:
        raise ValueError("cu_seqlens must be on the input device")
    if not isinstance(block_size, int) or block_size <= 0:
        raise ValueError("block_size must be a positive integer")
    if not isinstance(max_seqlen, int) or max_seqlen <= 0:
        raise ValueError("max_seqlen must be a positive integer")
    if not math.isfinite(scale):
        raise ValueError("scale must be finite")
    save_state = torch.is_grad_enabled() and (index_q.requires_grad or index_k.requires_grad)
    scores, _ = torch.ops.msa_mi355x.index_score(index_q, index_k, cu_seqlens, max_seqlen, block_size,
                                                 float(scale), save_state)
    return scores


def m3_topk(scores, cu_seqlens, *, block_size=128, topk_blocks=16, local_blocks=1):
    """``msa_triton_amd.m3_topk`` through the registered op."""
    if scores.ndim != 3 or scores.dtype != torch.float32:
        raise ValueError("scores must be FP32 [T,G,Bmax]")
    if not isinstance(topk_blocks, int) or topk_blocks < 0:
        raise ValueError("topk_blocks must be a nonnegative integer")
    if not isinstance(local_blocks, int) or not 0 <= local_blocks <= topk_blocks:
        raise ValueError("local_blocks must satisfy 0 <= local_blocks <= topk_blocks")
    return torch.ops.msa_mi355x.topk(scores.detach(), cu_seqlens, block_size, topk_blocks, local_blocks)


def m3_sparse_attention(q, k, v, indices, cu_seqlens, max_seqlen, *, block_size=128, scale=None, return_lse=False):
    """``msa_triton_amd.m3_sparse_attention`` through the registered op (same arguments and checks)."""
    if q.ndim != 3 or k.ndim != 3 or v.shape != k.shape:
        raise ValueError("Expected q[T,Hq,D] and matching k/v[T,G,D].")
    if q.shape[0] != k.shape[0] or q.shape[2] != k.shape[2]:
        raise ValueError("q/k/v must have matching token and head dimensions.")
    if k.shape[1] <= 0 or q.shape[1] <= 0 or q.shape[1] % k.shape[1]:
        raise ValueError("Hq must be a positive multiple of G.")
    if q.shape[2] <= 0:
        raise ValueError("Head dimension must be positive.")
    if q.dtype not in (torch.bfloat16, torch.float16, torch.float32) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise TypeError("q/k/v must share a BF16, FP16, or FP32 dtype.")
    if indices.ndim != 3 or indices.shape[:2] != (q.shape[0], k.shape[1]) or indices.dtype != torch.int32:
        raise ValueError("indices must be int32 [T,G,K].")
    if cu_seqlens.ndim != 1 or cu_seqlens.numel() < 2 or cu_seqlens.dtype != torch.int32:
        raise ValueError("cu_seqlens must be int32 [num_sequences + 1].")
    if any(x.device != q.device for x in (k, v, indices, cu_seqlens)):
        raise ValueError("All inputs must reside on the same device.")
    if not isinstance(block_size, int) or block_size <= 0:
        raise ValueError("block_size must be a positive integer.")
    if not isinstance(max_seqlen, int) or max_seqlen <= 0:
        raise ValueError("max_seqlen must be a positive integer.")
    effective_scale = q.shape[-1] ** -0.5 if scale is None else float(scale)
    if not math.isfinite(effective_scale):
        raise ValueError("scale must be finite.")
    save_state = torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad)
    out, lse, _, _ = torch.ops.msa_mi355x.sparse_attention(q, k, v, indices, cu_seqlens, max_seqlen, block_size,
                                                           effective_scale, save_state)
    return (out, lse) if return_lse else out


def m3_indexer_kl(index_q, index_k, q, k, indices, cu_seqlens, max_seqlen, *, block_size=128, index_scale=1.0,
                  scale=None, return_rows=False, teacher_lse=None):
    """``msa_triton_amd.m3_indexer_kl`` through the registered op (same arguments and static checks)."""
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
    if cu_seqlens.ndim != 1 or cu_seqlens.numel() < 2 or cu_seqlens.dtype != torch.int32:
        raise ValueError("cu_seqlens must be int32 [num_sequences + 1]")
    if not isinstance(block_size, int) or block_size <= 0:
        raise ValueError("block_size must be a positive integer")
    if not isinstance(max_seqlen, int) or max_seqlen <= 0:
        raise ValueError("max_seqlen must be a positive integer")
    effective_scale = q.shape[-1] ** -0.5 if scale is None else float(scale)
    if not math.isfinite(effective_scale) or not math.isfinite(index_scale):
        raise ValueError("scale and index_scale must be finite")
    grad = torch.is_grad_enabled()
    loss, rows, _, _ = torch.ops.msa_mi355x.indexer_kl(index_q, index_k, q.detach(), k.detach(), indices, cu_seqlens,
                                                       max_seqlen, block_size, float(index_scale), effective_scale,
                                                       grad and index_q.requires_grad, grad and index_k.requires_grad,
                                                       None if teacher_lse is None else teacher_lse.detach())
    return (loss, rows) if return_rows else loss
