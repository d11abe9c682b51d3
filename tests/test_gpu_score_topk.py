"""The fused first two stages (``m3_index_score_topk``): scores, indices and score
gradients equal, bit for bit, to ``m3_index_score`` followed by ``m3_topk``. Cases
cover the MFMA score path (bf16) and the exact one (fp16 / fp32), rows of up to
4500 blocks (above 4096 the selection streams each row from memory), varlen packs with empty sequences, forced local blocks, negative scale
and exact ties from small-integer inputs."""

from __future__ import annotations

import pytest
import torch

import msa_triton_amd as msa
from tests.helpers import cu_tensor

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("lengths,groups,dim,block,topk,local,scale,dtype,integer", [
    ([300, 0, 517, 64], 2, 128, 64, 4, 1, 1.0, torch.bfloat16, False),
    ([1000], 4, 64, 32, 8, 2, -1.0, torch.bfloat16, False),
    ([250, 7], 3, 32, 16, 16, 0, 0.5, torch.bfloat16, True),
    ([777], 2, 96, 128, 3, 1, 1.0, torch.bfloat16, False),
    ([2200, 37], 2, 64, 2, 8, 1, 1.0, torch.bfloat16, False),     # 1100 blocks per row
    ([400, 0, 90], 2, 64, 16, 5, 1, 1.0, torch.float16, False),
    ([300], 1, 40, 8, 6, 2, 1.0, torch.float32, True),
    ([129, 1], 2, 128, 128, 20, 1, 1.0, torch.bfloat16, False),   # K > blocks of the row
    ([9000, 37], 1, 32, 2, 12, 1, 1.0, torch.bfloat16, False),    # 4500 blocks per row
])
def test_fused_score_topk_equals_two_stages(lengths, groups, dim, block, topk, local, scale, dtype, integer, device):
    gen = torch.Generator().manual_seed(sum(lengths) + dim + topk)
    total = sum(lengths)
    if integer:
        iq = torch.randint(-2, 3, (total, groups, dim), generator=gen).to(dtype)
        ik = torch.randint(-2, 3, (total, 1, dim), generator=gen).to(dtype)
    else:
        iq = torch.randn(total, groups, dim, generator=gen).to(dtype)
        ik = torch.randn(total, 1, dim, generator=gen).to(dtype)
    cu = cu_tensor(lengths, device)
    maxlen = max(lengths)
    q1, k1 = (x.to(device).requires_grad_() for x in (iq, ik))
    s1 = msa.m3_index_score(q1, k1, cu, maxlen, block_size=block, scale=scale)
    i1 = msa.m3_topk(s1.detach(), cu, block_size=block, topk_blocks=topk, local_blocks=local)
    q2, k2 = (x.to(device).requires_grad_() for x in (iq, ik))
    s2, i2 = msa.m3_index_score_topk(q2, k2, cu, maxlen, block_size=block, scale=scale, topk_blocks=topk,
                                     local_blocks=local)
    assert torch.equal(s1, s2) and torch.equal(i1, i2)
    assert i2.dtype == torch.int32 and not i2.requires_grad and s2.requires_grad
    up = torch.randn(s1.shape, generator=gen).to(device)
    s1.backward(up)
    s2.backward(up)
    assert torch.equal(q1.grad, q2.grad) and torch.equal(k1.grad, k2.grad)


def test_fused_score_topk_with_prepared_sequences_and_k0(device):
    lengths, block = [500, 0, 260], 32
    gen = torch.Generator().manual_seed(4)
    iq = torch.randn(sum(lengths), 2, 64, generator=gen).bfloat16().to(device)
    ik = torch.randn(sum(lengths), 1, 64, generator=gen).bfloat16().to(device)
    seqs = msa.prepare_sequences(cu_tensor(lengths, device), block_size=block)
    s, i = msa.m3_index_score_topk(iq, ik, seqs, max(lengths), block_size=block, topk_blocks=6, local_blocks=1)
    ref = msa.m3_topk(msa.m3_index_score(iq, ik, seqs, max(lengths), block_size=block), seqs, block_size=block,
                      topk_blocks=6, local_blocks=1)
    assert torch.equal(i, ref)
    s0, i0 = msa.m3_index_score_topk(iq, ik, seqs, max(lengths), block_size=block, topk_blocks=0, local_blocks=0)
    assert i0.shape == (sum(lengths), 2, 0) and torch.equal(s0, s)
