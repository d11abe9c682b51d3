"""GPU parity of the indexer KL (m3_indexer_kl) against the FP64 oracle.

There is no reference kernel (docs/implementation_plan.md:66-69); the oracle is
the restatement in oracle/msa_oracle.py, pinned in tests/test_oracle_kl.py.
Stated tolerance: loss within 1e-6 + 1e-5 |x|; per-pair KL within 1e-6 + 1e-5 |x|;
fp32 gradients within 1e-5 * max |x| + 1e-4 |x| of the FP64 values (the teacher
and student probabilities come from fp32 logits, ~2^-22 relative); the bf16
gradients of the autograd path within one bf16 ulp (1e-6 + 2^-8 |x|).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import msa_triton_amd as msa
from msa_triton_amd.indexer_kl import _launch
from msa_triton_amd.layout import sequence_meta
from oracle import msa_oracle as O
from tests.helpers import cu_list, random_selection

pytestmark = pytest.mark.gpu


def _inputs(lengths, groups, ratio, dim, dim_i, block, topk, seed, q_scale=1.0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    total = sum(lengths)
    iq = torch.randn(total, groups, dim_i, generator=g).to(dtype)
    ik = torch.randn(total, 1, dim_i, generator=g).to(dtype)
    q = (q_scale * torch.randn(total, groups * ratio, dim, generator=g)).to(dtype)
    k = torch.randn(total, groups, dim, generator=g).to(dtype)
    ids = random_selection(total, groups, topk, lengths, block, 1, g)
    cu = torch.tensor(cu_list(lengths), dtype=torch.int32)
    return iq, ik, q, k, ids, cu


def _oracle(iq, ik, q, k, ids, cu, block, index_scale, scale):
    return O.indexer_kl(*(x.double().numpy() for x in (iq, ik, q, k)), ids.numpy(), cu.numpy(), block_size=block,
                        index_scale=index_scale, scale=scale)


def _close32(actual, expected, what):
    act = actual.detach().cpu().double().numpy()
    exp = np.asarray(expected, dtype=np.float64)
    bound = 1e-5 * max(np.abs(exp).max(), 1e-30) + 1e-4 * np.abs(exp)
    err = np.abs(act - exp)
    assert np.all(err <= bound), f"{what}: max err/bound {float((err / bound).max()):.3f}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("lengths,groups,ratio,dim,dim_i,block,topk,index_scale,scale", [
    ([37], 1, 1, 32, 32, 8, 3, 1.0, None),
    ([300, 45], 2, 4, 64, 64, 16, 5, 0.5, None),
    ([5, 0, 130, 77], 2, 8, 128, 64, 32, 4, 1.0, 0.1),
    ([257, 128], 1, 8, 128, 128, 128, 3, 0.2, None),
    ([64, 200], 4, 2, 64, 128, 64, 2, 1.0, 0.3),
    # blocks above 128 keys: 2 sub-blocks of 128, 2 of 96
    ([300, 45], 2, 4, 64, 64, 256, 2, 0.5, None),
    ([400], 1, 2, 32, 128, 192, 3, 1.0, None),
])
def test_matches_fp64_oracle(lengths, groups, ratio, dim, dim_i, block, topk, index_scale, scale, dtype, device):
    """bf16 and fp16 (fp16: dz = S - T enters the gradient products as fp16 terms of 2^15 dz)."""
    iq, ik, q, k, ids, cu = _inputs(lengths, groups, ratio, dim, dim_i, block, topk, 17, dtype=dtype)
    sc = dim ** -0.5 if scale is None else scale
    ref = _oracle(iq, ik, q, k, ids, cu, block, index_scale, sc)
    meta = sequence_meta(cu.tolist(), block)
    d = [x.to(device) for x in (iq, ik, q, k, ids, cu)]
    loss, rows, d_iq, d_ik = _launch(*d[:6], meta, None, block, index_scale, sc, True, True, True)
    assert float(loss) == pytest.approx(ref["loss"], rel=1e-5, abs=1e-6)
    np.testing.assert_allclose(rows.cpu().double().numpy(), ref["row_kl"], rtol=1e-5, atol=1e-6)
    _close32(d_iq, ref["d_iq"], "d_iq")
    _close32(d_ik, ref["d_ik"], "d_ik")
    # the autograd path: same loss, gradients of the loss in the input dtype (one ulp)
    a, b = d[0].clone().requires_grad_(), d[1].clone().requires_grad_()
    out = msa.m3_indexer_kl(a, b, d[2], d[3], d[4], d[5], max(lengths), block_size=block, index_scale=index_scale,
                            scale=scale)
    assert float(out.detach()) == float(loss)
    out.backward()
    ulp = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
    for grad, exp in ((a.grad, ref["d_iq"]), (b.grad, ref["d_ik"])):
        assert grad.dtype == dtype
        act = grad.float().cpu().double().numpy()
        assert np.all(np.abs(act - exp) <= 1e-6 + ulp * np.abs(exp))


def test_zero_when_student_equals_teacher(device):
    """One head per group, q = index_q, k = index_k, equal scales: the loss and its
    gradients vanish (up to fp32 rounding)."""
    iq, ik, _, _, ids, cu = _inputs([90, 150], 2, 1, 64, 64, 16, 4, 5)
    k = ik.expand(-1, 2, -1).contiguous()
    d = [x.to(device) for x in (iq, ik, iq, k, ids, cu)]
    meta = sequence_meta(cu.tolist(), 16)
    loss, rows, d_iq, d_ik = _launch(*d, meta, None, 16, 0.7, 0.7, True, True, True)
    assert abs(float(loss)) < 1e-6 and float(rows.abs().max()) < 1e-5
    assert float(d_iq.abs().max()) < 1e-7 and float(d_ik.abs().max()) < 1e-7


def test_empty_selection_and_empty_input(device):
    iq, ik, q, k, ids, cu = _inputs([20, 12], 2, 2, 32, 32, 8, 2, 9)
    ids[:] = -1
    a = iq.to(device).requires_grad_()
    loss, rows = msa.m3_indexer_kl(a, ik.to(device), q.to(device), k.to(device), ids.to(device), cu.to(device), 20,
                                   block_size=8, return_rows=True)
    loss.backward()
    assert float(loss.detach()) == 0.0 and float(rows.abs().max()) == 0.0 and float(a.grad.abs().max()) == 0.0
    e = torch.empty(0, 1, 32, dtype=torch.bfloat16, device=device)
    out = msa.m3_indexer_kl(e, e[:, :1], torch.empty(0, 2, 32, dtype=torch.bfloat16, device=device), e,
                            torch.empty(0, 1, 2, dtype=torch.int32, device=device),
                            torch.zeros(2, dtype=torch.int32, device=device), 1, block_size=8)
    assert float(out) == 0.0


def test_prepared_sequences_and_sampled_rows_at_c2_scale(device):
    """T = 2048 (16 blocks of 128, top-8): sampled rows and keys against the oracle,
    with prepared metadata; the result equals the cu_seqlens call bitwise."""
    lengths, groups, ratio, block = [2048], 4, 8, 128
    iq, ik, q, k, ids, cu = _inputs(lengths, groups, ratio, 128, 128, block, 8, 23)
    d = [x.to(device) for x in (iq, ik, q, k, ids, cu)]
    seqs = msa.prepare_sequences(d[5], block_size=block)
    l1, r1 = msa.m3_indexer_kl(*d[:5], seqs, 2048, block_size=block, return_rows=True)
    l2, r2 = msa.m3_indexer_kl(*d[:5], d[5], 2048, block_size=block, return_rows=True)
    assert torch.equal(l1, l2) and torch.equal(r1, r2)
    tokens = [0, 1, 127, 128, 1000, 2047]
    ref = O.indexer_kl_rows(*(x.double().numpy() for x in (iq, ik, q, k)), ids.numpy(), cu.numpy(), tokens,
                            block_size=block, index_scale=1.0, scale=128 ** -0.5)
    np.testing.assert_allclose(r1.cpu().double().numpy()[tokens], ref["row_kl"], rtol=1e-5, atol=1e-6)
    meta = sequence_meta(cu.tolist(), block)
    _, _, d_iq, d_ik = _launch(*d[:6], meta, None, block, 1.0, 128 ** -0.5, False, True, True)
    _close32(d_iq[tokens], ref["d_iq"], "d_iq rows")
    keys = [0, 130, 2047]
    ref_k = O.indexer_kl_key_rows(*(x.double().numpy() for x in (iq, ik, q, k)), ids.numpy(), cu.numpy(), keys,
                                  block_size=block, index_scale=1.0, scale=128 ** -0.5)
    _close32(d_ik[keys, 0], ref_k, "d_ik keys")


def test_unsupported_configurations_raise(device):
    iq, ik, q, k, ids, cu = _inputs([20], 1, 2, 32, 32, 8, 2, 1)
    d = [x.to(device) for x in (iq, ik, q, k, ids, cu)]
    with pytest.raises(NotImplementedError):
        msa.m3_indexer_kl(d[0].float(), d[1].float(), d[2].float(), d[3].float(), d[4], d[5], 20, block_size=8)
    with pytest.raises(NotImplementedError):
        q16 = torch.randn(20, 16, 32, device=device).bfloat16()
        msa.m3_indexer_kl(d[0], d[1], q16, d[3], d[4], d[5], 20, block_size=8)
    with pytest.raises(NotImplementedError):  # index inputs and attention inputs of different dtypes
        msa.m3_indexer_kl(d[0], d[1], d[2].half(), d[3].half(), d[4], d[5], 20, block_size=8)


def test_teacher_lse_from_the_attention(device):
    """The attention's lse as the teacher's normalisers (the teacher half of the
    statistics pass is skipped): the same oracle tolerances as the full pass."""
    lengths, groups, ratio, dim, block = [300, 0, 200], 2, 4, 64, 32
    iq, ik, q, k, ids, cu = _inputs(lengths, groups, ratio, dim, 64, block, 4, 31)
    ids[5, 1] = -1  # a pair with no visible key: lse -inf, KL 0
    d = [x.to(device) for x in (iq, ik, q, k, ids, cu)]
    v = torch.randn(k.shape, generator=torch.Generator().manual_seed(2)).bfloat16().to(device)
    _, lse = msa.m3_sparse_attention(d[2], d[3], v, d[4], d[5], 300, block_size=block, return_lse=True)
    sc = dim ** -0.5
    ref = _oracle(iq, ik, q, k, ids, cu, block, 1.0, sc)
    meta = sequence_meta(cu.tolist(), block)
    loss, rows, d_iq, d_ik = _launch(*d[:6], meta, None, block, 1.0, sc, True, True, True, teacher_lse=lse)
    assert float(loss) == pytest.approx(ref["loss"], rel=1e-5, abs=1e-6)
    np.testing.assert_allclose(rows.cpu().double().numpy(), ref["row_kl"], rtol=1e-5, atol=1e-6)
    assert float(rows[5, 1]) == 0.0
    _close32(d_iq, ref["d_iq"], "d_iq")
    _close32(d_ik, ref["d_ik"], "d_ik")
    a = d[0].clone().requires_grad_()
    out = msa.m3_indexer_kl(a, d[1], d[2], d[3], d[4], d[5], 300, block_size=block, teacher_lse=lse)
    assert float(out.detach()) == float(loss)
    out.backward()
    assert torch.equal(a.grad, d_iq.to(torch.bfloat16))
    with pytest.raises(ValueError, match="teacher_lse"):
        msa.m3_indexer_kl(a, d[1], d[2], d[3], d[4], d[5], 300, block_size=block, teacher_lse=lse[:, :1])
