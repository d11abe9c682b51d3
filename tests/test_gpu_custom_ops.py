"""GPU checks of the torch.library registration: ``torch.library.opcheck`` on each
op, and a score -> top-k -> attention layer compiled with ``torch.compile``
(AOTAutograd, ``fullgraph=True``) matching the eager operators bitwise."""

from __future__ import annotations

import pytest
import torch

import msa_triton_amd as msa
from msa_triton_amd import custom_ops as C
from tests.helpers import cu_tensor

pytestmark = pytest.mark.gpu


def _inputs(device, lengths=(200, 0, 137), groups=2, ratio=2, dim=64, seed=3):
    gen = torch.Generator().manual_seed(seed)
    total = sum(lengths)
    t = [torch.randn(total, groups, dim, generator=gen), torch.randn(total, 1, dim, generator=gen),
         torch.randn(total, groups * ratio, dim, generator=gen), torch.randn(total, groups, dim, generator=gen),
         torch.randn(total, groups, dim, generator=gen), torch.randn(total, groups * ratio, dim, generator=gen)]
    return [x.bfloat16().to(device) for x in t], cu_tensor(list(lengths), device), max(lengths)


def test_opcheck_each_op(device):
    (iq, ik, q, k, v, g), cu, maxlen = _inputs(device)
    block = 32
    iq.requires_grad_()
    ik.requires_grad_()
    torch.library.opcheck(torch.ops.msa_mi355x.index_score.default, (iq, ik, cu, maxlen, block, 1.0, True))
    scores = msa.m3_index_score(iq.detach(), ik.detach(), cu, maxlen, block_size=block)
    torch.library.opcheck(torch.ops.msa_mi355x.topk.default, (scores, cu, block, 3, 1))
    ids = msa.m3_topk(scores, cu, block_size=block, topk_blocks=3, local_blocks=1)
    q, k, v = (x.clone().requires_grad_() for x in (q, k, v))
    torch.library.opcheck(torch.ops.msa_mi355x.sparse_attention.default, (q, k, v, ids, cu, maxlen, block, 0.125, True))
    torch.library.opcheck(torch.ops.msa_mi355x.indexer_kl.default,
                          (iq, ik, q.detach(), k.detach(), ids, cu, maxlen, block, 1.0, 0.125, True, True, None))


def _forward(ops, iq, ik, q, k, v, g, cu, maxlen, block, topk):
    scores = ops.m3_index_score(iq, ik, cu, maxlen, block_size=block)
    ids = ops.m3_topk(scores.detach(), cu, block_size=block, topk_blocks=topk, local_blocks=1)
    out, lse = ops.m3_sparse_attention(q, k, v, ids, cu, maxlen, block_size=block, return_lse=True)
    kl = ops.m3_indexer_kl(iq, ik, q, k, ids, cu, maxlen, block_size=block)
    loss = (out.float() * g.float()).sum() + torch.where(torch.isinf(scores), 0.0, scores).sum() + kl
    return loss, scores, ids, out, lse


def _run(fn, tensors, cu, maxlen, block, topk):
    iq, ik, q, k, v = (x.clone().requires_grad_() for x in tensors[:5])
    loss, scores, ids, out, lse = fn(iq, ik, q, k, v, tensors[5], cu, maxlen, block, topk)
    loss.backward()
    return [scores.detach(), ids, out.detach(), lse, q.grad, k.grad, v.grad, iq.grad, ik.grad]


def test_compiled_layer_matches_eager(device):
    tensors, cu, maxlen = _inputs(device, lengths=(300, 0, 260), seed=11)
    block, topk = 32, 4
    eager = _run(lambda *a: _forward(msa, *a), tensors, cu, maxlen, block, topk)
    compiled_fn = torch.compile(lambda *a: _forward(C, *a), backend="aot_eager", fullgraph=True)
    compiled = _run(compiled_fn, tensors, cu, maxlen, block, topk)
    for a, b in zip(eager, compiled):
        assert torch.equal(a, b)
