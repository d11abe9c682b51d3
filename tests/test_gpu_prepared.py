"""Prepared sequence metadata on the GPU: every operator gives bitwise the same
results with ``PackedSequences`` as with ``cu_seqlens``; with it a whole layer
(score -> top-k -> attention, forward and backward) runs without reading device
memory back on the host; and the attention forward + backward captured in a HIP
graph replays to the eager results."""

from __future__ import annotations

import pytest
import torch

import msa_triton_amd as msa
from msa_triton_amd.k2q import build_k2q_csr
from tests.helpers import cu_tensor

pytestmark = pytest.mark.gpu


def _layer_inputs(lengths, groups, ratio, dim, seed):
    gen = torch.Generator().manual_seed(seed)
    total = sum(lengths)
    iq = torch.randn(total, groups, dim, generator=gen).bfloat16()
    ik = torch.randn(total, 1, dim, generator=gen).bfloat16()
    q = torch.randn(total, groups * ratio, dim, generator=gen).bfloat16()
    k = torch.randn(total, groups, dim, generator=gen).bfloat16()
    v = torch.randn(total, groups, dim, generator=gen).bfloat16()
    g = torch.randn(total, groups * ratio, dim, generator=gen).bfloat16()
    return iq, ik, q, k, v, g


def _layer(tensors, meta_arg, max_seqlen, block, topk, local, device):
    """score -> top-k -> attention forward and backward; returns every output."""
    iq, ik, q, k, v, g = (x.to(device).clone().requires_grad_(x.dtype != torch.int32) for x in tensors)
    scores = msa.m3_index_score(iq, ik, meta_arg, max_seqlen, block_size=block)
    ids = msa.m3_topk(scores.detach(), meta_arg, block_size=block, topk_blocks=topk, local_blocks=local)
    out, lse = msa.m3_sparse_attention(q, k, v, ids, meta_arg, max_seqlen, block_size=block, return_lse=True)
    out.backward(g.detach())
    scores.backward(torch.ones_like(scores).masked_fill(torch.isinf(scores), 0.0))
    csr = build_k2q_csr(ids, meta_arg, block_size=block)
    return [scores.detach(), ids, out.detach(), lse, q.grad, k.grad, v.grad, iq.grad, ik.grad,
            csr.row_ptr, csr.query_indices, csr.slot_indices, csr.cu_block_lens]


@pytest.mark.parametrize("lengths,groups,ratio,dim,block,topk,local", [
    ([300, 0, 517, 64], 2, 4, 128, 64, 4, 1), ([1000], 4, 8, 128, 128, 4, 1), ([5, 0, 90], 1, 2, 64, 16, 3, 2),
])
def test_prepared_metadata_gives_identical_results(lengths, groups, ratio, dim, block, topk, local, device):
    tensors = _layer_inputs(lengths, groups, ratio, dim, sum(lengths) + block)
    cu = cu_tensor(lengths, device)
    seqs = msa.prepare_sequences(cu, block_size=block)
    plain = _layer(tensors, cu, max(lengths), block, topk, local, device)
    prepared = _layer(tensors, seqs, max(lengths), block, topk, local, device)
    for a, b in zip(plain, prepared):
        assert torch.equal(a, b)


def test_prepared_layer_reads_nothing_back(device, monkeypatch):
    """With PackedSequences no operator copies device data to the host or syncs."""
    lengths, block = [700, 0, 350], 64
    tensors = _layer_inputs(lengths, 2, 4, 128, 9)
    seqs = msa.prepare_sequences(cu_tensor(lengths, device), block_size=block)
    _layer(tensors, seqs, max(lengths), block, 4, 1, device)  # first call: library load, allocator warm-up
    torch.cuda.synchronize()

    def refuse(*args, **kwargs):
        raise AssertionError("host read of device data")

    inputs = [x.to(device) for x in tensors]
    for name in ("tolist", "item", "cpu", "numpy"):
        monkeypatch.setattr(torch.Tensor, name, refuse)
    torch.cuda.set_sync_debug_mode("error")
    try:
        iq, ik, q, k, v, g = (x.clone().requires_grad_() for x in inputs)
        scores = msa.m3_index_score(iq, ik, seqs, max(lengths), block_size=block)
        ids = msa.m3_topk(scores.detach(), seqs, block_size=block, topk_blocks=4, local_blocks=1)
        out = msa.m3_sparse_attention(q, k, v, ids, seqs, max(lengths), block_size=block)
        out.backward(g.detach())
        scores.backward(torch.zeros_like(scores))
    finally:
        torch.cuda.set_sync_debug_mode("default")
        monkeypatch.undo()
    torch.cuda.synchronize()
    assert q.grad is not None and k.grad is not None and iq.grad is not None


def test_attention_forward_backward_captured_in_a_graph(device):
    """Capture fwd + bwd once, then replay three times with new inputs copied into
    the static buffers (eager work and a synchronisation between replays); every
    replay must equal a fresh eager run bitwise."""
    lengths, groups, ratio, dim, block, topk = [600, 0, 424], 2, 4, 128, 64, 4
    total = sum(lengths)
    cu = cu_tensor(lengths, device)
    seqs = msa.prepare_sequences(cu, block_size=block)
    gen = torch.Generator().manual_seed(77)

    def draw():
        q = torch.randn(total, groups * ratio, dim, generator=gen).bfloat16().to(device)
        k = torch.randn(total, groups, dim, generator=gen).bfloat16().to(device)
        v = torch.randn(total, groups, dim, generator=gen).bfloat16().to(device)
        g = torch.randn(total, groups * ratio, dim, generator=gen).bfloat16().to(device)
        sc = torch.randn(total, groups, (max(lengths) + block - 1) // block, generator=gen).to(device)
        ids = msa.m3_topk(sc, seqs, block_size=block, topk_blocks=topk, local_blocks=1)
        return q, k, v, g, ids

    def eager(q, k, v, g, ids):
        q, k, v = (x.clone().requires_grad_() for x in (q, k, v))
        out = msa.m3_sparse_attention(q, k, v, ids, seqs, max(lengths), block_size=block)
        out.backward(g)
        return out.detach(), q.grad, k.grad, v.grad

    q0, k0, v0, g0, ids0 = draw()
    sq, sk, sv = (x.clone().requires_grad_() for x in (q0, k0, v0))
    sg, sids = g0.clone(), ids0.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up outside the capture
        for _ in range(2):
            msa.m3_sparse_attention(sq, sk, sv, sids, seqs, max(lengths), block_size=block).backward(sg)
            sq.grad = sk.grad = sv.grad = None
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        sout = msa.m3_sparse_attention(sq, sk, sv, sids, seqs, max(lengths), block_size=block)
        sout.backward(sg)
    for rep in range(3):
        q, k, v, g, ids = draw()
        with torch.no_grad():
            for dst, src in ((sq, q), (sk, k), (sv, v), (sg, g), (sids, ids)):
                dst.copy_(src)
        graph.replay()
        torch.cuda.synchronize()
        ref = eager(q, k, v, g, ids)
        torch.cuda.synchronize()
        for got, want in zip((sout, sq.grad, sk.grad, sv.grad), ref):
            assert torch.equal(got, want), f"replay {rep}"
