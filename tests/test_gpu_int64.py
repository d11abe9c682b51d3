"""Element offsets past 2^31 in the attention kernels.

The reference forms TND element offsets (token * heads + head) * dim and CSR cursors
in int64 (triton/_addressing.py:11-18) and tests offsets past 2^31
(tests/test_index_addressing.py:24-40). Here a pack of T = 327,680 tokens with
Hq = 64, G = 8, D = 128 puts q, dO, out and dQ at 2.68e9 elements (5 GiB in bf16;
the fp32 output copy, 10 GiB). Its last two sequences start at tokens 320,000 and
324,096, i.e. past element offset 2^31 = 2,147,483,648 (token 262,144). Their
query rows, gradients and keys are checked against the FP64 oracle on host copies
of those sequences alone (every token of a sequence sees only its own sequence).
Selections (current block plus one random earlier block per token and group) are
drawn on the device.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import msa_triton_amd as msa
from oracle import msa_oracle as O
from tests.helpers import check_bf16_stated

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(600)]


def test_attention_rows_past_int32_offsets(device):
    lengths = [320000, 4096, 3584]
    heads, groups, dim, block, topk = 64, 8, 128, 128, 2
    total = sum(lengths)
    bounds = np.cumsum([0] + lengths)
    assert bounds[1] * heads * dim > 2**31  # sequences 1 and 2 lie wholly past offset 2^31
    gen = torch.Generator(device=device).manual_seed(97)
    q = torch.randn(total, heads, dim, device=device, generator=gen).bfloat16()
    k = torch.randn(total, groups, dim, device=device, generator=gen).bfloat16()
    v = torch.randn(total, groups, dim, device=device, generator=gen).bfloat16()
    dout = torch.randn(total, heads, dim, device=device, generator=gen).bfloat16()
    starts = torch.repeat_interleave(torch.tensor(bounds[:-1], device=device),
                                     torch.tensor(lengths, device=device))
    qb = (torch.arange(total, device=device) - starts) // block
    ids = torch.empty(total, groups, topk, dtype=torch.int32, device=device)
    ids[:, :, 0] = qb[:, None].int()
    earlier = (torch.rand(total, groups, device=device, generator=gen) * qb[:, None]).floor().int()
    ids[:, :, 1] = torch.where(qb[:, None] > 0, earlier, torch.full_like(earlier, -1))
    cu = torch.tensor(bounds, dtype=torch.int32, device=device)
    print(f"T={total} Hq={heads} G={groups} D={dim}: q holds {total * heads * dim} elements", flush=True)

    qg, kg, vg = (x.requires_grad_() for x in (q, k, v))
    out, lse = msa.m3_sparse_attention(qg, kg, vg, ids, cu, max(lengths), block_size=block, return_lse=True)
    out.backward(dout)
    torch.cuda.synchronize()

    rng = np.random.default_rng(3)
    for s in (1, 2):
        a, b = int(bounds[s]), int(bounds[s + 1])
        n = b - a
        host = [x[a:b].detach().double().cpu().numpy() for x in (q, k, v, dout)]
        ids_s = ids[a:b].cpu().numpy()
        toks = np.unique(np.concatenate([[0, 1, block - 1, block, n // 2, n - 2, n - 1], rng.integers(0, n, 12)]))
        rows = O.attention_rows(*host[:3], ids_s, [0, n], toks, block_size=block, dout=host[3])
        check_bf16_stated(out[a + toks], rows["out"], f"seq {s} out")
        check_bf16_stated(qg.grad[a + toks], rows["dq"], f"seq {s} dq")
        got_lse = lse[a + toks].cpu().numpy()
        np.testing.assert_allclose(got_lse, rows["lse"], atol=1e-4, rtol=1e-4)
        keys = np.unique(np.array([0, 5, block + 7, n // 2, n - block, n - 1]))
        dk_ref, dv_ref = O.attention_kv_rows(*host[:3], ids_s, [0, n], host[3], keys, block_size=block)
        check_bf16_stated(kg.grad[a + keys], dk_ref, f"seq {s} dk")
        check_bf16_stated(vg.grad[a + keys], dv_ref, f"seq {s} dv")
