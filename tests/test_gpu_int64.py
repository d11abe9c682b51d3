"""Element offsets past 2^31 in the attention kernels, and (token, head, slot) counts past 2^31.

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

The capacity limit of the KV-major kernels is the CSR's T * G * K < 2^31 edges
(triton/k2q.py:65-69), so a pack may hold T * Hq * K >= 2^31 (token, head, slot)
triples -- the index space of the per-slot partial records of the attention and of
the indexer KL. test_token_head_slot_triples_past_int32 runs such a pack (T = 69,632,
Hq = 64, G = 8, K = 512: 2.28e9 triples, 2.85e8 edges) through attention forward +
backward and the indexer KL at the default chunk budgets and checks the sequence whose
triples all lie past 2^31 against the oracle.
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


def _stratified_selection(bounds, lengths, groups, topk, block, device, gen):
    """K distinct causal blocks per (token, group), local block included: block s of the
    row is drawn uniformly from [s nb / K, (s + 1) nb / K) (nb = causal blocks of the
    token), so no two slots collide; rows with nb <= K take every causal block."""
    total = int(bounds[-1])
    starts = torch.repeat_interleave(torch.tensor(bounds[:-1], device=device), torch.tensor(lengths, device=device))
    qb = (torch.arange(total, device=device) - starts) // block  # [T]
    nb = qb + 1
    s = torch.arange(topk, device=device)
    lo = (s[None, :] * nb[:, None]) // topk
    hi = ((s[None, :] + 1) * nb[:, None]) // topk
    u = torch.rand(total, groups, topk, device=device, generator=gen)
    ids = lo[:, None, :] + (u * (hi - lo)[:, None, :]).floor().long()
    ids[:, :, topk - 1] = qb[:, None]  # the last stratum ends at qb: the local block
    few = (nb <= topk)[:, None, None]
    dense = torch.where(s[None, None, :] < nb[:, None, None], s[None, None, :], torch.full_like(ids, -1))
    return torch.where(few, dense, ids).int()


def test_token_head_slot_triples_past_int32(device):
    lengths = [65536, 4096]
    heads, groups, dim, dim_i, block, topk = 64, 8, 32, 32, 2, 512
    total = sum(lengths)
    bounds = np.cumsum([0] + lengths)
    assert bounds[1] * heads * topk >= 2**31  # every triple of sequence 1 lies past 2^31
    assert total * groups * topk < 2**31  # within the CSR's edge limit
    gen = torch.Generator(device=device).manual_seed(131)
    q = torch.randn(total, heads, dim, device=device, generator=gen).bfloat16()
    k = torch.randn(total, groups, dim, device=device, generator=gen).bfloat16()
    v = torch.randn(total, groups, dim, device=device, generator=gen).bfloat16()
    dout = torch.randn(total, heads, dim, device=device, generator=gen).bfloat16()
    iq = torch.randn(total, groups, dim_i, device=device, generator=gen).bfloat16()
    ik = torch.randn(total, 1, dim_i, device=device, generator=gen).bfloat16()
    ids = _stratified_selection(bounds, lengths, groups, topk, block, device, gen)
    cu = torch.tensor(bounds, dtype=torch.int32, device=device)
    print(f"T={total} Hq={heads} G={groups} K={topk}: {total * heads * topk} (token, head, slot) triples", flush=True)

    qg, kg, vg = (x.clone().requires_grad_() for x in (q, k, v))
    out, lse = msa.m3_sparse_attention(qg, kg, vg, ids, cu, max(lengths), block_size=block, return_lse=True)
    out.backward(dout)
    iqg, ikg = iq.clone().requires_grad_(), ik.clone().requires_grad_()
    loss, row_kl = msa.m3_indexer_kl(iqg, ikg, q, k, ids, cu, max(lengths), block_size=block, return_rows=True)
    loss.backward()
    torch.cuda.synchronize()
    print("attention and indexer KL done", flush=True)

    a, b = int(bounds[1]), int(bounds[2])
    n = b - a
    host = [x[a:b].detach().double().cpu().numpy() for x in (q, k, v, dout, iq, ik)]
    ids_s = ids[a:b].cpu().numpy()
    toks = np.array([0, 1, 2, 1023, 1024, 1025, n // 2, n - 2, n - 1])
    rows = O.attention_rows(*host[:3], ids_s, [0, n], toks, block_size=block, dout=host[3])
    check_bf16_stated(out[a + toks], rows["out"], "seq 1 out")
    check_bf16_stated(qg.grad[a + toks], rows["dq"], "seq 1 dq")
    np.testing.assert_allclose(lse[a + toks].cpu().numpy(), rows["lse"], atol=1e-4, rtol=1e-4)
    keys = np.array([n - 64, n - 5, n - 1])
    dk_ref, dv_ref = O.attention_kv_rows(*host[:3], ids_s, [0, n], host[3], keys, block_size=block)
    check_bf16_stated(kg.grad[a + keys], dk_ref, "seq 1 dk")
    check_bf16_stated(vg.grad[a + keys], dv_ref, "seq 1 dv")

    # indexer KL: per-pair KL and the loss gradients (the loss averages over all T * G pairs
    # of the pack; the oracle on the sequence alone averages over its own, hence the factor)
    kl_args = (host[4], host[5], host[0], host[1], ids_s, [0, n])
    ref = O.indexer_kl_rows(*kl_args, toks, block_size=block)
    np.testing.assert_allclose(row_kl[a + toks].cpu().double().numpy(), ref["row_kl"], rtol=1e-5, atol=1e-6)
    factor = (n * groups) / (total * groups)
    ref_k = O.indexer_kl_key_rows(*kl_args, keys, block_size=block) * factor
    for what, got, want in (("d_iq", iqg.grad[a + toks], ref["d_iq"] * factor), ("d_ik", ikg.grad[a + keys, 0], ref_k)):
        act = got.detach().double().cpu().numpy()
        err = np.abs(act - want)
        bound = 2.0 ** -8 * np.abs(want) + 2.0 ** -10 * np.abs(want).max()
        print(f"seq 1 {what}: worst err/bound {float((err / bound).max()):.3f}", flush=True)
        assert np.all(err <= bound), f"seq 1 {what}: max err/bound {float((err / bound).max()):.3f}"
