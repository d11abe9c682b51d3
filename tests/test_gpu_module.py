"""A small trainable layer around the three operators, on the GPU: input projections ->
m3_index_score / m3_topk under no_grad (a frozen indexer) -> m3_sparse_attention ->
output projection, following the reference's module test (tests/test_pipeline.py:60-87).

The layer's output and the gradients of its input and of its four projection weights
are compared with float64 torch autograd of the same layer in which the attention is
the FP64 oracle (forward and backward of oracle.msa_oracle.sparse_attention, pinned
against torch autograd of an independent dense formulation in
tests/test_oracle_attention.py). The selection is the oracle's own (index_score ->
topk on the same index inputs) and must equal the GPU's bit for bit. The indexer
weights must receive no gradient.

fp32 layers use the reference test's gate (atol = rtol = 1e-4). bf16 layers round
every projection and every attention output and gradient to bf16, so their values
are compared within a bound of a few bf16 ulps of each gradient's scale.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import msa_triton_amd as msa
from oracle import msa_oracle as O
from tests.helpers import cu_list

pytestmark = pytest.mark.gpu


class _OracleAttention(torch.autograd.Function):
    """FP64 oracle attention as a torch autograd function (CPU, float64)."""

    @staticmethod
    def forward(ctx, q, k, v, ids, cu, block_size):
        out, _ = O.sparse_attention(q.numpy(), k.numpy(), v.numpy(), ids, cu, block_size=block_size)
        ctx.save_for_backward(q, k, v)
        ctx.ids, ctx.cu, ctx.block_size = ids, cu, block_size
        return torch.from_numpy(out)

    @staticmethod
    def backward(ctx, grad):
        q, k, v = ctx.saved_tensors
        _, _, dq, dk, dv = O.sparse_attention(q.numpy(), k.numpy(), v.numpy(), ctx.ids, ctx.cu,
                                              block_size=ctx.block_size, dout=grad.contiguous().numpy())
        return torch.from_numpy(dq), torch.from_numpy(dk), torch.from_numpy(dv), None, None, None


def _layer(x, wq, wk, wv, wo, ids, cu, max_len, shape, block_size, attention):
    total, groups, ratio, dim = shape
    q = (x @ wq).reshape(total, groups * ratio, dim)
    k = (x @ wk).reshape(total, groups, dim)
    v = (x @ wv).reshape(total, groups, dim)
    out = attention(q, k, v, ids, cu, max_len, block_size)
    return out.reshape(total, -1) @ wo


# (lengths, hidden, groups, ratio, dim, block, topk, local): the reference's layer
# (8 tokens, hidden 12, two groups of two heads, dim 4, block 2, top-2), and a larger
# one whose bf16 attention runs on the MFMA kernels (dim 64, 4 heads per group).
CASES = [
    ([5, 3], 12, 2, 2, 4, 2, 2, 1),
    ([180, 77], 64, 2, 4, 64, 16, 4, 1),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("case", CASES, ids=["reference", "mfma"])
def test_layer_parameter_gradients(case, dtype, device):
    lengths, hidden, groups, ratio, dim, block_size, topk, local = case
    total = sum(lengths)
    max_len = max(lengths)
    torch.manual_seed(54)
    base = [torch.randn(total, hidden), torch.randn(hidden, groups * ratio * dim) * 0.2,
            torch.randn(hidden, groups * dim) * 0.2, torch.randn(hidden, groups * dim) * 0.2,
            torch.randn(groups * ratio * dim, hidden) * 0.2]
    base = [a.to(dtype) for a in base]  # the layer's parameters and input in the tested dtype
    index_q_weight = torch.randn(hidden, groups * dim).to(dtype).to(device).requires_grad_()
    index_k_weight = torch.randn(hidden, dim).to(dtype).to(device).requires_grad_()
    cu_np = np.array(cu_list(lengths), dtype=np.int32)
    cu = torch.from_numpy(cu_np).to(device)

    # ---- the layer on the GPU
    x, wq, wk, wv, wo = [a.to(device).detach().clone().requires_grad_() for a in base]
    with torch.no_grad():
        iq = (x @ index_q_weight).reshape(total, groups, dim)
        ik = (x @ index_k_weight).reshape(total, 1, dim)
        score = msa.m3_index_score(iq, ik, cu, max_len, block_size=block_size)
        ids = msa.m3_topk(score, cu, block_size=block_size, topk_blocks=topk, local_blocks=local)
    gpu_attention = lambda q, k, v, i, c, m, b: msa.m3_sparse_attention(q, k, v, i, c, m, block_size=b)
    output = _layer(x, wq, wk, wv, wo, ids, cu, max_len, (total, groups, ratio, dim), block_size, gpu_attention)
    output.float().square().mean().backward()
    torch.cuda.synchronize()
    got = [output.detach().float().cpu()] + [a.grad.float().cpu() for a in (x, wq, wk, wv, wo)]
    assert index_q_weight.grad is None
    assert index_k_weight.grad is None

    # ---- the oracle's selection from the same index inputs (bf16 / fp32 values as the GPU saw them)
    iq64, ik64 = iq.double().cpu().numpy(), ik.double().cpu().numpy()
    _, ref_scores, _ = O.index_score(iq64, ik64, cu_np, max_len, block_size=block_size)
    ref_ids = O.topk(ref_scores, cu_np, block_size=block_size, topk_blocks=topk, local_blocks=local)
    np.testing.assert_array_equal(ids.cpu().numpy(), ref_ids)

    # ---- float64 autograd of the same layer with the oracle attention
    xr, wqr, wkr, wvr, wor = [a.double().detach().clone().requires_grad_() for a in base]
    if dtype == torch.bfloat16:
        # the GPU layer rounds the projections to bf16 before the attention: so does the reference
        def oracle_attention(q, k, v, i, c, m, b):
            r = [t.detach().to(torch.bfloat16).double() + (t - t.detach()) for t in (q, k, v)]  # rounded, identity gradient
            return _OracleAttention.apply(*r, ref_ids, cu_np, b)
    else:
        def oracle_attention(q, k, v, i, c, m, b):
            return _OracleAttention.apply(q, k, v, ref_ids, cu_np, b)
    ref_out = _layer(xr, wqr, wkr, wvr, wor, None, None, max_len, (total, groups, ratio, dim), block_size,
                     oracle_attention)
    ref_out.square().mean().backward()
    want = [ref_out.detach()] + [a.grad for a in (xr, wqr, wkr, wvr, wor)]

    names = ["output", "x.grad", "wq.grad", "wk.grad", "wv.grad", "wo.grad"]
    for name, a, b in zip(names, got, want):
        a = a.double()
        assert torch.isfinite(a).all(), name
        if dtype == torch.float32:
            torch.testing.assert_close(a, b, atol=1e-4, rtol=1e-4, msg=name)
        else:
            # bf16 projections, attention outputs and gradient products each round to 8 significant
            # bits: a few bf16 ulps of the value, plus a few ulps of the gradient's largest entry
            scale = float(b.abs().max())
            err = (a - b).abs()
            bound = 2.0 ** -6 * b.abs() + 2.0 ** -6 * scale
            worst = float((err / bound).max())
            print(f"{name}: max err {float(err.max()):.3g} (scale {scale:.3g}), worst err/bound {worst:.3f}", flush=True)
            assert bool((err <= bound).all()), f"{name}: error {float(err.max()):.3g} above the bf16 bound"
