"""bf16 and fp16 attention with blocks of more than 128 keys, on the MFMA kernels through
sub-blocks: ``msa_split_block_indices`` maps block id b to sub-blocks f b .. f b + f - 1
of block_size / f keys, which hold the same keys (triton/sparse_attention.py:35-84: a
selected block b covers keys [b B, b B + B) of the sequence, clipped at the query).

The split itself is compared with a numpy statement of that map (including -1 padding,
future blocks and ids near INT32_MAX); the attention forward and backward with the
FP64 oracle at the original block size, within the stated tolerance of the dtype; the prepared
(PackedSequences) call bit for bit with the plain one.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import msa_triton_amd as msa
from msa_triton_amd import _lib
from msa_triton_amd import sparse_attention as SA
from oracle import msa_oracle as O
from tests.helpers import check_bf16_stated, cu_tensor, np64, random_selection

pytestmark = pytest.mark.gpu


def _split_np(ids, factor):
    """out[r, s f + i] = f ids[r, s] + i, -1 for negative ids and where f id + i passes INT32_MAX."""
    ids = ids.astype(np.int64)
    sub = ids[..., None] * factor + np.arange(factor)
    ok = (ids[..., None] >= 0) & (ids[..., None] <= (2**31 - 1 - (factor - 1)) // factor)
    return np.where(ok, sub, -1).reshape(ids.shape[0], ids.shape[1], -1).astype(np.int32)


@pytest.mark.parametrize("factor", [1, 2, 3, 8])
def test_split_block_indices_match_the_map(factor, device):
    rng = np.random.default_rng(factor)
    ids = rng.integers(-1, 50, size=(37, 3, 5)).astype(np.int32)
    limit = (2**31 - 1 - (factor - 1)) // factor  # the largest id whose sub-blocks fit int32
    ids[0, 0, :] = [2**31 - 1, limit, min(limit + 1, 2**31 - 1), -7, 0]
    src = torch.from_numpy(ids).to(device)
    out = torch.full((37, 3, 5 * factor), 99, dtype=torch.int32, device=device)
    status = _lib.lib().msa_split_block_indices(src.data_ptr(), 37 * 3, 5, factor, out.data_ptr(),
                                                _lib.stream_of(device))
    assert status == 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), _split_np(ids, factor))


# (lengths, groups, ratio, dim, block, topk): blocks of 256 (2 x 128), 192 (2 x 96) and
# 384 (3 x 128), with a ragged packing and a causal tail in each; one case at head dim 256
CASES = [
    ([700, 300], 2, 2, 64, 256, 2),
    ([650], 1, 4, 32, 192, 3),
    ([900, 5], 2, 1, 128, 384, 2),
    ([420, 33], 1, 2, 256, 256, 2),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("lengths,groups,ratio,dim,block,topk", CASES)
def test_large_blocks_run_sub_blocks_on_mfma(lengths, groups, ratio, dim, block, topk, dtype, device, monkeypatch):
    from tests.test_gpu_sweep import _check_dtype_stated

    check = check_bf16_stated if dtype == torch.bfloat16 else (
        lambda a, r, n: _check_dtype_stated(a, r, torch.float16, n))
    total = sum(lengths)
    gen = torch.Generator().manual_seed(block + dim)
    q = torch.randn(total, groups * ratio, dim, generator=gen).to(dtype)
    k = torch.randn(total, groups, dim, generator=gen).to(dtype)
    v = torch.randn(total, groups, dim, generator=gen).to(dtype)
    grad = torch.randn(total, groups * ratio, dim, generator=gen).to(dtype)
    ids = random_selection(total, groups, topk, lengths, block, 1, gen)
    cu = cu_tensor(lengths)

    seen = []
    view = SA._sub_block_view

    def spy(*args):
        result = view(*args)
        seen.append(result[2])
        return result

    monkeypatch.setattr(SA, "_sub_block_view", spy)
    tensors = [x.to(device).requires_grad_() for x in (q, k, v)]
    out, lse = msa.m3_sparse_attention(*tensors, ids.to(device), cu.to(device), max(lengths), block_size=block,
                                       return_lse=True)
    out.backward(grad.to(device))
    torch.cuda.synchronize()
    assert seen and all(b < block and block % b == 0 and b <= 128 for b in seen), seen  # forward and backward split

    ref_out, ref_lse, dq, dk, dv = O.sparse_attention(np64(q), np64(k), np64(v), ids.numpy(), cu.numpy(),
                                                      block_size=block, dout=np64(grad))
    check(out, ref_out, "out")
    finite = np.isfinite(ref_lse)
    np.testing.assert_array_equal(np.isneginf(lse.detach().cpu().numpy()), np.isneginf(ref_lse))
    np.testing.assert_allclose(lse.detach().cpu().numpy()[finite], ref_lse[finite], atol=1e-4, rtol=1e-4)
    for name, t, ref in zip(("dq", "dk", "dv"), tensors, (dq, dk, dv)):
        check(t.grad, ref, name)

    # the prepared form takes the same sub-blocks: identical results
    seqs = msa.prepare_sequences(cu.to(device), block_size=block)
    again = [x.detach().clone().requires_grad_() for x in tensors]
    out2 = msa.m3_sparse_attention(*again, ids.to(device), seqs, max(lengths), block_size=block)
    out2.backward(grad.to(device))
    assert torch.equal(out2, out)
    for a, b in zip(again, tensors):
        assert torch.equal(a.grad, b.grad)
