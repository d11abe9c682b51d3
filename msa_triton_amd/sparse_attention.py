"""Stage 3: TND sparse GQA attention over selected KV blocks, with autograd.

Mirrors triton/sparse_attention.py:429-485 of the reference (signature,
defaults, validation order, messages and exception types) and the
``_SparseAttention`` autograd contract (:334-395): per-input
``needs_input_grad``; the public ``build_k2q_csr`` is invoked by the backward
exactly when dK or dV is needed; lse is non-differentiable.

Execution: ``msa_attn_fwd`` and ``msa_attn_bwd``. For bf16 and fp16 both are KV-major
over the selection's k2q CSR (per-block partials merged in slot order, dK/dV
owned per key block, no floating-point atomics); the forward builds the CSR
itself and keeps it for a backward that needs only dQ. ``cu_seqlens`` may be a
``PackedSequences`` (``prepare_sequences``): then neither pass reads metadata
back from the device. Saved state is q, k, v,
out in the input dtype, an fp64 [T,Hq,4] per-row state (full-precision lse
and its normalisation, then the backward's center / delta) and the output in
fp32, from which the backward takes delta = O . dO directly instead of
recomputing the softmax statistics over every selected block (the reference's
centred recomputation, :119-158, remains the C path without the fp32 output).
"""

from __future__ import annotations

import math

import torch

from . import _lib
from . import k2q as _k2q
from .layout import PackedSequences, call_sequences, prepared_for, sequence_lengths, sequence_meta


def _sub_block_view(q, k, indices, meta, block_size, seqs):
    """The selection as the MFMA kernels take it: bf16 / fp16 blocks above 128 keys as
    sub-blocks (``k2q.sub_block_selection``); unchanged for other calls."""
    total, heads, dim = q.shape
    if q.dtype not in (torch.bfloat16, torch.float16):
        return indices, meta, block_size, seqs
    lib = _lib.lib()

    def fits(factor, sub, sub_meta):
        return lib.msa_attn_fwd_workspace_bytes(_lib.DTYPE_CODE[q.dtype], total, heads, k.shape[1], dim,
                                                indices.shape[2] * factor, sub_meta.total_blocks, sub) > 0

    return _k2q.sub_block_selection(indices, meta, block_size, seqs, fits)


def _attn_forward(q, k, v, indices, cu, meta, block_size, scale, seqs, public_csr=False, save_f32=False):
    """Forward launch on contiguous inputs: (out, lse, row_state, out_f32 or None,
    csr or None). With ``public_csr`` the KV-major path builds its CSR through the
    public builder; with ``save_f32`` it also returns the fp32 output for the backward."""
    total, heads, dim = q.shape
    groups = k.shape[1]
    out = torch.empty_like(q)
    lse = torch.empty((total, heads), device=q.device, dtype=torch.float32)
    # Private fp64 per-row state shared by forward and backward: lse, mass, center, delta.
    row_state = torch.empty((total, heads, 4), device=q.device, dtype=torch.float64)
    out_f32 = torch.empty((total, heads, dim), device=q.device, dtype=torch.float32) if save_f32 else None
    csr = None
    if total:
        indices, meta, block_size, seqs = _sub_block_view(q, k, indices, meta, block_size, seqs)
        lib = _lib.lib()
        dtype = _lib.DTYPE_CODE[q.dtype]
        slots = indices.shape[2]
        ws_bytes = lib.msa_attn_fwd_workspace_bytes(dtype, total, heads, groups, dim, slots,
                                                    meta.total_blocks, block_size)
        workspace = None
        if ws_bytes > 0:
            # The KV-major forward walks the block->query CSR of the selection.
            if public_csr:  # looked up through the module so the build stays observable
                csr = _k2q.build_k2q_csr(indices, cu if seqs is None else seqs, block_size=block_size)
            else:
                csr = _k2q._build_device(indices, cu, meta, groups, slots, seqs)
            workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
        with torch.cuda.device(q.device):
            status = lib.msa_attn_fwd(
                q.data_ptr(), k.data_ptr(), v.data_ptr(), dtype, indices.data_ptr(), cu.data_ptr(),
                meta.num_seqs, total, heads, groups, dim, slots, block_size, scale,
                _lib.ptr(None if csr is None else csr.cu_block_lens), meta.total_blocks,
                _lib.ptr(None if csr is None else csr.row_ptr),
                _lib.ptr(None if csr is None else csr.query_indices),
                _lib.ptr(None if csr is None else csr.slot_indices), _lib.ptr(workspace), ws_bytes,
                out.data_ptr(), lse.data_ptr(), row_state.data_ptr(), _lib.ptr(out_f32), _lib.stream_of(q.device),
            )
        _lib.check(status, "msa_attn_fwd")
    return out, lse, row_state, out_f32, csr


def _attn_backward(q, k, v, indices, cu, out, row_state, grad_output, meta, block_size, scale, seqs,
                   need_q, need_k, need_v, csr=None, out_f32=None):
    """Backward launch: (dq, dk, dv), None where not needed. ``row_state`` gets the
    backward's center; ``out_f32`` is the forward's fp32 output (None: the backward
    recomputes the statistics). ``csr`` (the forward's) is reused when given; otherwise a
    backward that needs dK or dV builds it through the public builder (as the
    reference does) and a dQ-only one privately."""
    need_kv = need_k or need_v
    dq = torch.empty_like(q) if need_q else None
    dk = torch.empty_like(k) if need_k else None
    dv = torch.empty_like(v) if need_v else None
    total, heads, dim = q.shape
    groups = k.shape[1]
    if total and (need_q or need_kv):
        indices, meta, block_size, seqs = _sub_block_view(q, k, indices, meta, block_size, seqs)
        slots = indices.shape[2]
        lib = _lib.lib()
        device = q.device
        dtype = _lib.DTYPE_CODE[q.dtype]
        if grad_output is None:
            grad_output = torch.zeros_like(out)
        dout = grad_output.to(q.dtype).contiguous()
        ws_bytes = lib.msa_attn_bwd_workspace_bytes(dtype, total, heads, groups, dim, slots, meta.total_blocks,
                                                    block_size)
        if csr is not None:
            pass
        elif need_kv:
            # Looked up through the module so the CSR build stays observable.
            csr = _k2q.build_k2q_csr(indices, cu if seqs is None else seqs, block_size=block_size)
        elif ws_bytes > 0:
            csr = _k2q._build_device(indices, cu, meta, groups, slots, seqs)
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=device) if ws_bytes > 0 else None
        with torch.cuda.device(device):
            status = lib.msa_attn_bwd(
                q.data_ptr(), k.data_ptr(), v.data_ptr(), dtype, out.data_ptr(), dout.data_ptr(),
                row_state.data_ptr(), _lib.ptr(out_f32), indices.data_ptr(), cu.data_ptr(), meta.num_seqs, total,
                heads, groups,
                dim, slots, block_size, scale,
                _lib.ptr(None if csr is None else csr.cu_block_lens), meta.total_blocks,
                _lib.ptr(None if csr is None else csr.row_ptr),
                _lib.ptr(None if csr is None else csr.query_indices),
                _lib.ptr(None if csr is None else csr.slot_indices), _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv),
                _lib.ptr(workspace), ws_bytes, _lib.stream_of(device),
            )
        _lib.check(status, "msa_attn_bwd")
    return dq, dk, dv


class _SparseAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, indices, cu_seqlens, block_size, scale, meta, seqs):
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        indices = indices.contiguous()
        cu = cu_seqlens.contiguous()
        # The KV-major forward needs the CSR anyway: when dK or dV will be needed it is
        # built through the public builder (the one build the reference makes, in its
        # backward) and the backward reuses it; a dQ-only backward reuses a private one.
        need_kv = ctx.needs_input_grad[1] or ctx.needs_input_grad[2]
        need_any = need_kv or ctx.needs_input_grad[0]
        out, lse, row_state, out_f32, csr = _attn_forward(q, k, v, indices, cu, meta, block_size, scale, seqs,
                                                          public_csr=need_kv, save_f32=need_any)
        ctx.save_for_backward(q, k, v, indices, cu, out, row_state, out_f32)
        ctx.csr = csr
        ctx.meta = meta
        ctx.seqs = seqs
        ctx.scale = scale
        ctx.block_size = block_size
        ctx.mark_non_differentiable(lse)
        return out, lse

    @staticmethod
    def backward(ctx, grad_output, grad_lse):
        q, k, v, indices, cu, out, row_state, out_f32 = ctx.saved_tensors
        need_q, need_k, need_v = ctx.needs_input_grad[:3]
        dq, dk, dv = _attn_backward(q, k, v, indices, cu, out, row_state, grad_output, ctx.meta, ctx.block_size,
                                    ctx.scale, ctx.seqs, need_q, need_k, need_v, ctx.csr, out_f32)
        ctx.csr = None
        return dq, dk, dv, None, None, None, None, None, None


def m3_sparse_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    indices: torch.Tensor,
    cu_seqlens: torch.Tensor,
    max_seqlen: int,
    *,
    block_size: int = 128,
    scale: float | None = None,
    return_lse: bool = False,
):
    """Apply causal block-sparse attention to packed TND tensors.

    ``indices[T, G, K]`` holds distinct sequence-local block ids with ``-1``
    padding. Each contiguous group of ``Hq / G`` query heads shares a
    selection. Empty selections produce zero output and zero input gradients.
    The optional natural-log LSE is FP32 and non-differentiable.
    """
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
    seqs = cu_seqlens if isinstance(cu_seqlens, PackedSequences) else None
    cu = seqs.cu_seqlens if seqs is not None else cu_seqlens
    if cu.ndim != 1 or cu.numel() < 2 or cu.dtype != torch.int32:
        raise ValueError("cu_seqlens must be int32 [num_sequences + 1].")
    if any(x.device != q.device for x in (k, v, indices, cu)):
        raise ValueError("All inputs must reside on the same device.")
    if not isinstance(block_size, int) or block_size <= 0:
        raise ValueError("block_size must be a positive integer.")
    if not isinstance(max_seqlen, int) or max_seqlen <= 0:
        raise ValueError("max_seqlen must be a positive integer.")
    if seqs is None:
        lengths = sequence_lengths(cu, q.shape[0])
    else:  # prepared: no host read
        lengths = list(prepared_for(seqs, block_size=block_size, total_tokens=q.shape[0], device=q.device).lengths)
    if max(lengths) > max_seqlen:
        raise ValueError("max_seqlen is smaller than an actual sequence.")
    effective_scale = q.shape[-1] ** -0.5 if scale is None else float(scale)
    if not math.isfinite(effective_scale):
        raise ValueError("scale must be finite.")
    _lib.require_gpu(q, "m3_sparse_attention")
    if seqs is None:
        bounds = [0]
        for length in lengths:
            bounds.append(bounds[-1] + length)
        meta = sequence_meta(bounds, block_size)
        # cu_seqlens was read once above: the rest of the call reads nothing back
        seqs = call_sequences(cu, meta, k.shape[1]) if q.shape[0] else None
    else:
        meta = seqs.meta
    output, lse = _SparseAttention.apply(q, k, v, indices, cu, block_size, effective_scale, meta, seqs)
    return (output, lse) if return_lse else output
