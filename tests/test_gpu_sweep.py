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
The shapes are small enough for the oracle to finish in about a second each.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import msa_triton_amd as msa
from msa_triton_amd.k2q import build_k2q_csr
from oracle import msa_oracle as O
from tests.helpers import check_bf16_stated, cu_list, cu_tensor, np64, rounded

pytestmark = pytest.mark.gpu

CASES = 24


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
    index_scale = float(rng.choice([1.0, 0.5, -0.75]))
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
