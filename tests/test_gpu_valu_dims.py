"""The FP64 attention kernels' row-parallel forms (attn_fwd_rows, attn_bwd_dq_rows,
attn_bwd_dkdv_rows: head dims 8, 16, 32, 64, 128 with 16-byte aligned rows) on fp16 and
fp32 inputs, forward and backward against the FP64 oracle: fp32 within the reference's
gate, fp16 within its stated analogue (every element within one fp16 ulp of the FP64
value, at most 0.1 % outside the gate). Head ratio 3 makes a KV-pass step span edges
(3 heads per edge against 4 to 16 rows per step); ragged lengths and blocks of 16 leave
partly visible blocks, and the blocks of 128 keys fill the forward's 64-key steps.
fp16 takes these kernels only for shapes outside the MFMA kernels: its cases use blocks
of 131 and 257 keys (primes above 128, so no sub-block split applies)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import msa_triton_amd as msa
from oracle import msa_oracle as O
from tests.helpers import cu_list, cu_tensor, np64, random_selection
from tests.test_gpu_sweep import _check_dtype_stated

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("block_index", [0, 1], ids=["short", "long"])
@pytest.mark.parametrize("dim", [8, 16, 32, 64, 128])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32], ids=["fp16", "fp32"])
def test_row_parallel_fp64_kernels_against_oracle(dtype, dim, block_index, device):
    from msa_triton_amd import _lib

    block = ([131, 257] if dtype == torch.float16 else [16, 128])[block_index]
    lengths, groups, ratio, topk = [150, 61], 2, 3, 4
    total = sum(lengths)
    nblocks = sum((n + block - 1) // block for n in lengths)
    assert _lib.lib().msa_attn_fwd_workspace_bytes(_lib.DTYPE_CODE[dtype], total, groups * ratio, groups, dim, topk,
                                                   nblocks, block) == 0  # the FP64 kernels
    g = torch.Generator().manual_seed(dim + block)
    ids = random_selection(total, groups, topk, lengths, block, 1, g)
    q, k, v, dout = (torch.randn(total, h, dim, generator=g).to(dtype) for h in (groups * ratio, groups, groups,
                                                                                groups * ratio))
    qd, kd, vd = (x.to(device).requires_grad_() for x in (q, k, v))
    out, lse = msa.m3_sparse_attention(qd, kd, vd, ids.to(device), cu_tensor(lengths, device), max(lengths),
                                       block_size=block, return_lse=True)
    r_out, r_lse, r_dq, r_dk, r_dv = O.sparse_attention(np64(q), np64(k), np64(v), ids.numpy(),
                                                        np.asarray(cu_list(lengths)), block_size=block,
                                                        dout=np64(dout))
    _check_dtype_stated(out, r_out, dtype, f"D={dim} B={block} out")
    finite = np.isfinite(r_lse)
    assert np.array_equal(np.isfinite(lse.cpu().numpy()), finite)
    np.testing.assert_allclose(lse.cpu().numpy()[finite], r_lse[finite], rtol=1e-4, atol=1e-4)
    out.backward(dout.to(device))
    for name, tensor, ref in (("dq", qd, r_dq), ("dk", kd, r_dk), ("dv", vd, r_dv)):
        _check_dtype_stated(tensor.grad, ref, dtype, f"D={dim} B={block} {name}")
