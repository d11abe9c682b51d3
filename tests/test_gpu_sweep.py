"""Seeded random-shape sweep of the whole hot path against the FP64 oracle.

Each case draws a shape (sequence lengths including empty ones, groups, query heads
per group including non-powers of two, head and index dims on and off the MFMA
templates' 32-multiples, block sizes from 1 to 128, top-k and local blocks, scales)
and runs score -> top-k -> k2q CSR -> attention forward + backward through the
public API, then checks every stage at its stated bar:
  * scores and tie handling: bit-exact to the oracle (index_score.py:121-136),
  * top-k indices and the k2q CSR: bit-exact (topk.py:31-46, k2q.py:39-128),
  * score gradients: the reference gate (atol = rtol = 1e-4 after rounding the FP64
    values to bf16, tests/test_triton_score.py:42-77),
  * attention output and dQ / dK / dV: the stated bf16 tolerance for large outputs
    (check_bf16_stated: every element within 1e-4 + 2^-8 |x| of the FP64 value, at
    most 0.1 % outside the reference's gate, tests/test_triton_attention.py:58-97 --
    fp32 arithmetic leaves values within ~2^-22 of a bf16 rounding midpoint undecided,
    a few elements in 10^5 on these shapes); lse within 1e-4.
Smaller sweeps cover fp16 / fp32 inputs (fp16 on the MFMA kernels where the head dim
fits them, the FP64 kernels otherwise), head dims 136-256 on the MFMA kernels, and the
indexer KL (eager/ops.py:153-180 restated in the oracle).
The shapes are small enough for the oracle to finish in about a second each.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import msa_triton_amd as msa
from msa_triton_amd.k2q import build_k2q_csr
from oracle import msa_oracle as O
from tests.helpers import check_bf16_stated, cu_list, cu_tensor, np64, rounded

pytestmark = pytest.mark.gpu

CASES = int(os.environ.get("MSA_SWEEP_CASES", "24"))  # more for an occasional wider sweep


def _draw(seed):
    rng = np.random.default_rng(seed)
    nseq = int(rng.integers(1, 4))
    lengths = [int(rng.choice([0, int(rng.integers(1, 500))], p=[0.15, 0.85])) for _ in range(nseq)]
    if sum(lengths) == 0:
        lengths[0] = int(rng.integers(1, 300))
    groups = int(rng.integers(1, 4))
    ratio = int(rng.choice([1, 2, 3, 4, 8]))
    dim = int(rng.choice([8, 16, 24, 48, 64, 96, 128]))
    dim_i = int(rng.choice([8, 16, 40, 64, 128]))
    block = int(rng.choice([1, 3, 8, 16, 32, 64, 128]))
    topk = int(rng.integers(1, 7))
    local = int(rng.integers(0, min(topk, 2) + 1))
    scale = None if rng.random() < 0.5 else float(rng.choice([0.05, 0.3, 1.7]))
    index_scale = float(rng.choice([1.0, 0.5, -0.75] if seed < 8 else [1.0, 0.5, -0.75, 0.3, -1.7]))
    return dict(lengths=lengths, groups=groups, ratio=ratio, dim=dim, dim_i=dim_i, block=block, topk=topk,
                local=local, scale=scale, index_scale=index_scale)


@pytest.mark.parametrize("seed", range(CASES))
def test_random_shape_pipeline_against_oracle(seed, device):
    cfg = _draw(1000 + seed)
    print(f"sweep case {seed}: {cfg}", flush=True)
    lengths, groups, ratio, dim = cfg["lengths"], cfg["groups"], cfg["ratio"], cfg["dim"]
    block, topk, local = cfg["block"], cfg["topk"], cfg["local"]
    total, heads = sum(lengths), cfg["groups"] * cfg["ratio"]
    max_seqlen = max(lengths)
    g = torch.Generator().manual_seed(seed)
    iq = torch.randn(total, groups, cfg["dim_i"], generator=g).bfloat16()
    ik = torch.randn(total, 1, cfg["dim_i"], generator=g).bfloat16()
    q = torch.randn(total, heads, dim, generator=g).bfloat16()
    k = torch.randn(total, groups, dim, generator=g).bfloat16()
    v = torch.randn(total, groups, dim, generator=g).bfloat16()
    dout = torch.randn(total, heads, dim, generator=g).bfloat16()
    cu_h = cu_list(lengths)
    cu = cu_tensor(lengths, device)

    # ---- stage 1: scores (bit-exact) and their gradients
    iq_d, ik_d = iq.to(device).requires_grad_(), ik.to(device).requires_grad_()
    scores = msa.m3_index_score(iq_d, ik_d, cu, max_seqlen, block_size=block, scale=cfg["index_scale"])
    _, ref_scores, _ = O.index_score(iq.double().numpy(), ik.double().numpy(), cu_h, max_seqlen, block_size=block,
                                     scale=cfg["index_scale"])
    np.testing.assert_array_equal(scores.detach().cpu().numpy(), ref_scores)
    ds = torch.randn(scores.shape, generator=g).masked_fill(~torch.isfinite(scores.detach().cpu()), 0)
    scores.backward(ds.to(device))
    ref_dq, ref_dk = O.index_score_backward(iq.double().numpy(), ik.double().numpy(), cu_h, max_seqlen,
                                            ds.double().numpy(), block_size=block, scale=cfg["index_scale"])
    torch.testing.assert_close(iq_d.grad.cpu(), rounded(ref_dq, torch.bfloat16), atol=1e-4, rtol=1e-4)
    torch.testing.assert_close(ik_d.grad.cpu(), rounded(ref_dk, torch.bfloat16), atol=1e-4, rtol=1e-4)

    # ---- stage 2: top-k and the k2q CSR (bit-exact)
    ids = msa.m3_topk(scores.detach(), cu, block_size=block, topk_blocks=topk, local_blocks=local)
    ref_ids = O.topk(ref_scores, cu_h, block_size=block, topk_blocks=topk, local_blocks=local)
    np.testing.assert_array_equal(ids.cpu().numpy(), ref_ids)
    csr = build_k2q_csr(ids, cu, block_size=block)
    ref_csr = O.k2q_csr(ref_ids, cu_h, block_size=block)
    for got, ref in zip((csr.row_ptr, csr.query_indices, csr.slot_indices, csr.cu_block_lens), ref_csr):
        np.testing.assert_array_equal(got.cpu().numpy(), ref)

    # ---- stage 3: attention forward + backward (the reference gate)
    qd, kd, vd = (x.to(device).requires_grad_() for x in (q, k, v))
    out, lse = msa.m3_sparse_attention(qd, kd, vd, ids, cu, max_seqlen, block_size=block, scale=cfg["scale"],
                                       return_lse=True)
    r_out, r_lse, r_dq, r_dk, r_dv = O.sparse_attention(np64(q), np64(k), np64(v), ref_ids, np.asarray(cu_h),
                                                        block_size=block, scale=cfg["scale"], dout=np64(dout))
    check_bf16_stated(out, r_out, f"case {seed} out")
    got_lse = lse.detach().cpu()
    ref_lse = torch.from_numpy(r_lse).float()
    assert torch.equal(torch.isneginf(got_lse), torch.isneginf(ref_lse))
    finite = torch.isfinite(ref_lse)
    torch.testing.assert_close(got_lse[finite], ref_lse[finite], atol=1e-4, rtol=1e-4)
    out.backward(dout.to(device))
    for name, tensor, ref in (("dq", qd, r_dq), ("dk", kd, r_dk), ("dv", vd, r_dv)):
        check_bf16_stated(tensor.grad, ref, f"case {seed} {name}")


def _check_dtype_stated(actual, expected, dtype, what):
    """fp32: the reference gate (atol = rtol = 1e-4 after rounding the FP64 value to fp32).
    fp16: every element within 1e-4 + 2^-10 |x| (one fp16 ulp) of the FP64 value and at
    most 0.1 % (at least one) outside the gate -- the fp16 analogue of check_bf16_stated."""
    if dtype == torch.float32:
        torch.testing.assert_close(actual.detach().cpu(), rounded(expected, dtype), atol=1e-4, rtol=1e-4)
        return
    act = actual.detach().cpu().double().numpy().ravel()
    exp = np.asarray(expected, dtype=np.float64).ravel()
    ref_r = rounded(exp, dtype).double().numpy().ravel()
    bad = int((np.abs(act - ref_r) > 1e-4 + 1e-4 * np.abs(ref_r)).sum())
    err = np.abs(act - exp)
    bound = 1e-4 + 2.0 ** -10 * np.abs(exp)
    print(f"{what}: {bad} of {act.size} outside the gate; worst err/bound {float((err / bound).max()):.3f}", flush=True)
    assert bad <= max(1, act.size // 1000), f"{what}: {bad} elements outside the gate"
    assert np.all(err <= bound), f"{what}: error above 1e-4 + 2^-10 |x|"


@pytest.mark.parametrize("seed", range(max(8, CASES // 3)))
def test_random_shape_fp16_fp32_attention_against_oracle(seed, device):
    """fp16 / fp32 inputs, any head dim, on random shapes and selections (fp32 and head dims
    off the MFMA kernels' shapes on the FP64 kernels, fp16 otherwise on the MFMA ones)."""
    from tests.helpers import random_selection

    rng = np.random.default_rng(2000 + seed)
    dtype = torch.float16 if seed % 2 else torch.float32
    lengths = [int(rng.integers(1, 200)) for _ in range(int(rng.integers(1, 3)))]
    groups, ratio = int(rng.integers(1, 3)), int(rng.choice([1, 2, 3, 5]))
    dim = int(rng.choice([5, 12, 33, 80, 200] if seed < 8 else [5, 8, 12, 16, 32, 33, 64, 80, 128, 200]))
    block = int(rng.choice([1, 4, 16, 64]))
    topk, local = int(rng.integers(1, 5)), int(rng.integers(0, 2))
    scale = None if seed % 3 else 0.2
    print(f"case {seed}: {lengths} G={groups} R={ratio} D={dim} B={block} K={topk} L={local} {dtype}", flush=True)
    total = sum(lengths)
    g = torch.Generator().manual_seed(seed)
    ids = random_selection(total, groups, topk, lengths, block, local, g)
    q, k, v, dout = (torch.randn(total, h, dim, generator=g).to(dtype) for h in (groups * ratio, groups, groups,
                                                                                groups * ratio))
    cu_h = cu_list(lengths)
    qd, kd, vd = (x.to(device).requires_grad_() for x in (q, k, v))
    out, lse = msa.m3_sparse_attention(qd, kd, vd, ids.to(device), cu_tensor(lengths, device), max(lengths),
                                       block_size=block, scale=scale, return_lse=True)
    r_out, r_lse, r_dq, r_dk, r_dv = O.sparse_attention(np64(q), np64(k), np64(v), ids.numpy(), np.asarray(cu_h),
                                                        block_size=block, scale=scale, dout=np64(dout))
    assert out.dtype == dtype
    _check_dtype_stated(out, r_out, dtype, f"case {seed} out")
    finite = np.isfinite(r_lse)
    assert np.array_equal(np.isfinite(lse.cpu().numpy()), finite)
    np.testing.assert_allclose(lse.cpu().numpy()[finite], r_lse[finite], rtol=1e-4, atol=1e-4)
    out.backward(dout.to(device))
    for name, tensor, ref in (("dq", qd, r_dq), ("dk", kd, r_dk), ("dv", vd, r_dv)):
        _check_dtype_stated(tensor.grad, ref, dtype, f"case {seed} {name}")


@pytest.mark.parametrize("seed", range(max(6, CASES // 4)))
def test_random_shape_wide_head_attention_against_oracle(seed, device):
    """Head dims 136-256 on the MFMA kernels (bf16 for even seeds, fp16 for odd ones; the
    backward's main pass in its per-half launches) on random shapes and selections,
    within the stated tolerance of the dtype."""
    from tests.helpers import random_selection

    rng = np.random.default_rng(3000 + seed)
    dtype = torch.float16 if seed % 2 else torch.bfloat16
    lengths = [int(rng.integers(1, 300)) for _ in range(int(rng.integers(1, 3)))]
    groups, ratio = int(rng.integers(1, 3)), int(rng.choice([1, 2, 3, 8]))
    dim = int(rng.choice([136, 168, 200, 224, 256]))
    block = int(rng.choice([4, 16, 64, 128]))
    topk, local = int(rng.integers(1, 5)), int(rng.integers(0, 2))
    scale = None if seed % 3 else 0.2
    print(f"case {seed}: {lengths} G={groups} R={ratio} D={dim} B={block} K={topk} L={local} {dtype}", flush=True)
    total = sum(lengths)
    g = torch.Generator().manual_seed(seed)
    ids = random_selection(total, groups, topk, lengths, block, local, g)
    q, k, v, dout = (torch.randn(total, h, dim, generator=g).to(dtype) for h in (groups * ratio, groups, groups,
                                                                                groups * ratio))
    cu_h = cu_list(lengths)
    qd, kd, vd = (x.to(device).requires_grad_() for x in (q, k, v))
    out, lse = msa.m3_sparse_attention(qd, kd, vd, ids.to(device), cu_tensor(lengths, device), max(lengths),
                                       block_size=block, scale=scale, return_lse=True)
    r_out, r_lse, r_dq, r_dk, r_dv = O.sparse_attention(np64(q), np64(k), np64(v), ids.numpy(), np.asarray(cu_h),
                                                        block_size=block, scale=scale, dout=np64(dout))
    check = (lambda a, r, n: check_bf16_stated(a, r, n)) if dtype == torch.bfloat16 else (
        lambda a, r, n: _check_dtype_stated(a, r, dtype, n))
    check(out, r_out, f"case {seed} out")
    finite = np.isfinite(r_lse)
    assert np.array_equal(np.isfinite(lse.cpu().numpy()), finite)
    np.testing.assert_allclose(lse.cpu().numpy()[finite], r_lse[finite], rtol=1e-4, atol=1e-4)
    out.backward(dout.to(device))
    for name, tensor, ref in (("dq", qd, r_dq), ("dk", kd, r_dk), ("dv", vd, r_dv)):
        check(tensor.grad, ref, f"case {seed} {name}")


@pytest.mark.parametrize("seed", range(max(8, CASES // 3)))
def test_random_shape_indexer_kl_against_oracle(seed, device):
    """m3_indexer_kl (bf16, dims 32 / 64 / 128, up to 8 heads per group) on random shapes:
    loss and per-pair KL within 1e-6 + 1e-5 |x|, the fp32 gradients within
    1e-5 max |x| + 1e-4 |x| of the FP64 oracle (the KL tests' stated tolerance)."""
    from msa_triton_amd.indexer_kl import _launch
    from msa_triton_amd.layout import sequence_meta
    from tests.helpers import random_selection

    rng = np.random.default_rng(3000 + seed)
    lengths = [int(rng.choice([0, int(rng.integers(1, 400))], p=[0.1, 0.9])) for _ in range(int(rng.integers(1, 4)))]
    if sum(lengths) == 0:
        lengths[0] = 77
    groups, ratio = int(rng.integers(1, 4)), int(rng.choice([1, 2, 3, 8]))
    dim, dim_i = int(rng.choice([32, 64, 128])), int(rng.choice([32, 64, 128]))
    block = int(rng.choice([4, 16, 64, 128]))
    topk, local = int(rng.integers(1, 6)), int(rng.integers(0, 2))
    index_scale = float(rng.choice([1.0, 0.5]))
    scale = dim ** -0.5 if seed % 2 else 0.2
    print(f"case {seed}: {lengths} G={groups} R={ratio} D={dim} Di={dim_i} B={block} K={topk} L={local}", flush=True)
    total = sum(lengths)
    g = torch.Generator().manual_seed(seed)
    iq = torch.randn(total, groups, dim_i, generator=g).bfloat16()
    ik = torch.randn(total, 1, dim_i, generator=g).bfloat16()
    q = torch.randn(total, groups * ratio, dim, generator=g).bfloat16()
    k = torch.randn(total, groups, dim, generator=g).bfloat16()
    ids = random_selection(total, groups, topk, lengths, block, local, g)
    cu = torch.tensor(cu_list(lengths), dtype=torch.int32)
    ref = O.indexer_kl(*(x.double().numpy() for x in (iq, ik, q, k)), ids.numpy(), cu.numpy(), block_size=block,
                       index_scale=index_scale, scale=scale)
    meta = sequence_meta(cu.tolist(), block)
    d = [x.to(device) for x in (iq, ik, q, k, ids, cu)]
    loss, rows, d_iq, d_ik = _launch(*d[:6], meta, None, block, index_scale, scale, True, True, True)
    assert float(loss) == pytest.approx(ref["loss"], rel=1e-5, abs=1e-6)
    np.testing.assert_allclose(rows.cpu().double().numpy(), ref["row_kl"], rtol=1e-5, atol=1e-6)
    for name, got, exp in (("d_iq", d_iq, ref["d_iq"]), ("d_ik", d_ik, ref["d_ik"])):
        act = got.detach().cpu().double().numpy()
        bound = 1e-5 * max(np.abs(exp).max(), 1e-30) + 1e-4 * np.abs(exp)
        err = np.abs(act - exp)
        assert np.all(err <= bound), f"{name}: max err/bound {float((err / bound).max()):.3f}"
