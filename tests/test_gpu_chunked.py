"""GPU parity of the sums that the kernels split across query-token chunks or row segments.

* The bf16 attention forward, backward and the indexer KL process query tokens in
  chunks whose per-(token, head, slot) partial records fit a byte budget. The
  backward carries dK / dV in fp32 accumulators across chunks (the first chunk
  stores, middle chunks add, the last writes bf16), the KL carries d_index_k the
  same way. Here the budgets are shrunk with the ``msa_set_chunk_budgets`` testing
  hook so that small packs, checked against the dense FP64 oracle, run through 4 to
  20 chunks: every early key then receives its gradient from several chunks.
* The score backward forms dk per (key block, 8192-row segment) and adds the
  segments in order; a pack with T * G > 3 * 8192 rows runs through 4 segments.

Tolerance: the stated bf16 tolerance of the large-output tests
(tests.helpers.check_bf16_stated); the KL uses its own stated bounds
(tests/test_gpu_indexer_kl.py).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import msa_triton_amd as msa
from msa_triton_amd import _lib
from msa_triton_amd.indexer_kl import _launch as kl_launch
from msa_triton_amd.layout import sequence_meta
from msa_triton_amd.sparse_attention import _attn_backward, _attn_forward
from oracle import msa_oracle as O
from tests.helpers import check_bf16_stated, cu_list, np64, random_selection

pytestmark = pytest.mark.gpu


def _chunks(total, per_token_bytes, budget):
    """Chunks the host makes for `budget` (kv_chunk_tokens: at least 64 tokens, balanced)."""
    tc = max(64, budget // per_token_bytes)
    return -(-total // tc) if total > tc else 1


def _within_one_ulp(a, b, what):
    """Two bf16 results of the same sums in a different order: at most one bf16 ulp apart
    (2^-7 |x|) or, for values whose sums cancel, within the oracle's 1e-4 absolute floor."""
    x, y = a.detach().float().cpu(), b.detach().float().cpu()
    diff = (x - y).abs()
    bound = 1e-4 + 2.0 ** -7 * torch.maximum(x.abs(), y.abs())
    differ = int((diff > 0).sum())
    print(f"{what}: {differ} of {diff.numel()} differ; worst diff/bound {float((diff / bound).max()):.3f}", flush=True)
    assert bool((diff <= bound).all()), f"{what}: results further apart than one ulp + 1e-4"


def _attn_case(lengths, groups, ratio, dim, block, topk, seed):
    gen = torch.Generator().manual_seed(seed)
    total = sum(lengths)
    q = torch.randn(total, groups * ratio, dim, generator=gen).bfloat16()
    k = torch.randn(total, groups, dim, generator=gen).bfloat16()
    v = torch.randn(total, groups, dim, generator=gen).bfloat16()
    grad = torch.randn(q.shape, generator=gen).bfloat16()
    ids = random_selection(total, groups, topk, lengths, block, 1, gen)
    cu = torch.tensor(cu_list(lengths), dtype=torch.int32)
    return q, k, v, grad, ids, cu


@pytest.mark.parametrize("with_f32", [True, False])
def test_attention_through_many_chunks(with_f32, device):
    lengths, groups, ratio, dim, block, topk = [300, 517, 211], 2, 4, 64, 32, 6
    q, k, v, grad, ids, cu = _attn_case(lengths, groups, ratio, dim, block, topk, 41)
    total, heads = q.shape[0], q.shape[1]
    out_r, lse_r, dq_r, dk_r, dv_r = O.sparse_attention(np64(q), np64(k), np64(v), ids.numpy(), cu.numpy(),
                                                        block_size=block, dout=np64(grad))
    fwd_budget = 1                                      # 64-token chunks
    bwd_budget = 100 * heads * topk * (dim * 4 + 8)     # ~100-token chunks
    assert _chunks(total, heads * topk * (dim + 2) * 4, fwd_budget) >= 16
    assert _chunks(total, heads * topk * (dim * 4 + 8), bwd_budget) >= 10
    meta = sequence_meta(cu.tolist(), block)
    scale = dim ** -0.5
    qd, kd, vd, gd, idd, cud = (x.to(device) for x in (q, k, v, grad, ids, cu))
    with _lib.chunk_budgets(fwd=fwd_budget, bwd=bwd_budget):
        out, lse, rs, o32, csr = _attn_forward(qd, kd, vd, idd, cud, meta, block, scale, None, save_f32=with_f32)
        dq, dk, dv = _attn_backward(qd, kd, vd, idd, cud, out, rs, gd, meta, block, scale, None, True, True, True,
                                    csr, o32)
    torch.cuda.synchronize()
    check_bf16_stated(out, out_r, "chunked out")
    fin = np.isfinite(lse_r)
    np.testing.assert_allclose(lse.cpu().numpy()[fin], lse_r[fin], atol=1e-4, rtol=1e-4)
    check_bf16_stated(dq, dq_r, "chunked dq")
    check_bf16_stated(dk, dk_r, "chunked dk")
    check_bf16_stated(dv, dv_r, "chunked dv")
    # the default (single-chunk) run: the same sums split differently, so equal but for one-ulp flips
    out1, _, rs1, o321, csr1 = _attn_forward(qd, kd, vd, idd, cud, meta, block, scale, None, save_f32=with_f32)
    _, dk1, dv1 = _attn_backward(qd, kd, vd, idd, cud, out1, rs1, gd, meta, block, scale, None, False, True, True,
                                 csr1, o321)
    _within_one_ulp(dk, dk1, "chunked vs single-chunk dk")
    _within_one_ulp(dv, dv1, "chunked vs single-chunk dv")


@pytest.mark.parametrize("need", [(True, False, False), (False, True, False), (False, False, True)])
def test_attention_gradient_subsets_through_many_chunks(need, device):
    lengths, groups, ratio, dim, block, topk = [450, 190], 1, 8, 128, 64, 4
    q, k, v, grad, ids, cu = _attn_case(lengths, groups, ratio, dim, block, topk, 43)
    _, _, dq_r, dk_r, dv_r = O.sparse_attention(np64(q), np64(k), np64(v), ids.numpy(), cu.numpy(),
                                                block_size=block, dout=np64(grad))
    meta = sequence_meta(cu.tolist(), block)
    qd, kd, vd, gd, idd, cud = (x.to(device) for x in (q, k, v, grad, ids, cu))
    with _lib.chunk_budgets(fwd=1, bwd=1):  # 64-token chunks in both passes
        out, _, rs, o32, csr = _attn_forward(qd, kd, vd, idd, cud, meta, block, dim ** -0.5, None, save_f32=True)
        grads = _attn_backward(qd, kd, vd, idd, cud, out, rs, gd, meta, block, dim ** -0.5, None, *need, csr, o32)
    torch.cuda.synchronize()
    for wanted, got, ref, what in zip(need, grads, (dq_r, dk_r, dv_r), ("dq", "dk", "dv")):
        if wanted:
            check_bf16_stated(got, ref, f"chunked {what} only")
        else:
            assert got is None


def test_indexer_kl_through_many_chunks(device):
    lengths, groups, ratio, dim, dim_i, block, topk = [300, 45, 500], 2, 4, 64, 64, 16, 5
    gen = torch.Generator().manual_seed(47)
    total = sum(lengths)
    iq = torch.randn(total, groups, dim_i, generator=gen).bfloat16()
    ik = torch.randn(total, 1, dim_i, generator=gen).bfloat16()
    q = torch.randn(total, groups * ratio, dim, generator=gen).bfloat16()
    k = torch.randn(total, groups, dim, generator=gen).bfloat16()
    ids = random_selection(total, groups, topk, lengths, block, 1, gen)
    cu = torch.tensor(cu_list(lengths), dtype=torch.int32)
    scale = dim ** -0.5
    ref = O.indexer_kl(*(x.double().numpy() for x in (iq, ik, q, k)), ids.numpy(), cu.numpy(), block_size=block,
                       index_scale=0.5, scale=scale)
    meta = sequence_meta(cu.tolist(), block)
    d = [x.to(device) for x in (iq, ik, q, k, ids, cu)]
    with _lib.chunk_budgets(kl=1):  # 64-token chunks: 14 of them
        loss, rows, d_iq, d_ik = kl_launch(*d, meta, None, block, 0.5, scale, True, True, True)
    torch.cuda.synchronize()
    assert float(loss) == pytest.approx(ref["loss"], rel=1e-5, abs=1e-6)
    np.testing.assert_allclose(rows.cpu().double().numpy(), ref["row_kl"], rtol=1e-5, atol=1e-6)
    for got, exp, what in ((d_iq, ref["d_iq"], "d_iq"), (d_ik, ref["d_ik"], "d_ik")):
        act = got.detach().cpu().double().numpy()
        bound = 1e-5 * max(np.abs(exp).max(), 1e-30) + 1e-4 * np.abs(exp)
        assert np.all(np.abs(act - exp) <= bound), f"{what}: max err/bound {float((np.abs(act - exp) / bound).max())}"


def test_score_backward_through_several_row_segments(device):
    """T * G = 26800 rows: the dk pass works on 4 segments of 8192 rows per key block."""
    lengths, groups, dim, block = [3000, 2500, 1200], 4, 64, 128
    gen = torch.Generator().manual_seed(53)
    total = sum(lengths)
    iq = torch.randn(total, groups, dim, generator=gen).bfloat16()
    ik = torch.randn(total, 1, dim, generator=gen).bfloat16()
    cu = torch.tensor(cu_list(lengths), dtype=torch.int32)
    a = iq.to(device).requires_grad_()
    b = ik.to(device).requires_grad_()
    scores = msa.m3_index_score(a, b, cu.to(device), max(lengths), block_size=block, scale=0.7)
    ds = torch.randn(scores.shape, generator=gen).masked_fill(torch.isinf(scores.detach().cpu()), 0)
    scores.backward(ds.to(device))
    torch.cuda.synchronize()
    dq_r, dk_r = O.index_score_backward(iq.double().numpy(), ik.double().numpy(), cu.numpy(), max(lengths),
                                        ds.double().numpy(), block_size=block, scale=0.7)
    check_bf16_stated(a.grad, dq_r, "segmented score dq")
    check_bf16_stated(b.grad, dk_r, "segmented score dk")


@pytest.mark.parametrize("chunked", [False, True])
def test_dispatch_order_leaves_results_bitwise_equal(chunked, device):
    """The KV-major passes launch their work items largest first (``kv_item_order``);
    every item writes only its own records and partial slot, so row-order dispatch (the
    ``msa_set_item_order`` testing hook) must give the same bits in every output."""
    lengths, groups, ratio, dim, block, topk = [2100, 1500, 37], 2, 8, 128, 64, 8
    q, k, v, grad, ids, cu = _attn_case(lengths, groups, ratio, dim, block, topk, 53)
    gen = torch.Generator().manual_seed(54)
    total = sum(lengths)
    iq = torch.randn(total, groups, 64, generator=gen).bfloat16()
    ik = torch.randn(total, 1, 64, generator=gen).bfloat16()
    meta = sequence_meta(cu.tolist(), block)
    scale = dim ** -0.5
    qd, kd, vd, gd, idd, cud, iqd, ikd = (x.to(device) for x in (q, k, v, grad, ids, cu, iq, ik))
    budgets = dict(fwd=1, bwd=1, kl=1) if chunked else {}

    def run():
        with _lib.chunk_budgets(**budgets):
            out, lse, rs, o32, csr = _attn_forward(qd, kd, vd, idd, cud, meta, block, scale, None, save_f32=True)
            dq, dk, dv = _attn_backward(qd, kd, vd, idd, cud, out, rs, gd, meta, block, scale, None, True, True,
                                        True, csr, o32)
            kl = kl_launch(iqd, ikd, qd, kd, idd, cud, meta, None, block, 0.5, scale, True, True, True)
        torch.cuda.synchronize()
        return [x.detach().clone() for x in (out, lse, dq, dk, dv, *kl)]

    ordered = run()
    with _lib.row_order():
        in_rows = run()
    ordered_again = run()
    names = ("out", "lse", "dq", "dk", "dv", "kl loss", "kl rows", "d_iq", "d_ik")
    for a, b, c, what in zip(ordered, in_rows, ordered_again, names):
        assert torch.equal(a, b), f"{what}: row-order dispatch changed the result"
        assert torch.equal(a, c), f"{what}: a second ordered run changed the result"
