"""GPU parity of stage 1 (m3_index_score) against the CPU oracle.

Forward: scores bit-exact to the reference's public form of the exact winning dot
(oracle.public_score: fl32(scale * dot) when |scale| is 0, 1 or a power of two, the
reference's two-term fp32 form otherwise), -inf pattern exact. Backward: within the reference gate (atol=rtol=1e-4 after rounding the
FP64 oracle to the input dtype, tests/test_triton_score.py:32-77). Cases
mirror tests/test_triton_score.py, including the low-bit winner known answers.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import msa_triton_amd as msa
from oracle import msa_oracle as O
from tests.helpers import cu_list, cu_tensor, rounded

pytestmark = pytest.mark.gpu


def _run(q_cpu, k_cpu, lengths, max_seqlen, block_size, scale, upstream, device):
    q = q_cpu.to(device).clone().requires_grad_()
    k = k_cpu.to(device).clone().requires_grad_()
    cu = cu_tensor(lengths, device)
    actual = msa.m3_index_score(q, k, cu, max_seqlen, block_size=block_size, scale=scale)
    _, exp32, _ = O.index_score(q_cpu.double().numpy(), k_cpu.double().numpy(), cu_list(lengths), max_seqlen,
                                block_size=block_size, scale=scale)
    got = actual.detach().cpu().numpy()
    assert got.dtype == np.float32
    np.testing.assert_array_equal(got, exp32)
    actual.backward(upstream.to(device))
    dq, dk = O.index_score_backward(q_cpu.double().numpy(), k_cpu.double().numpy(), cu_list(lengths), max_seqlen,
                                    upstream.double().numpy(), block_size=block_size, scale=scale)
    dtype = q_cpu.dtype
    torch.testing.assert_close(q.grad.cpu(), rounded(dq, dtype), atol=1e-4, rtol=1e-4)
    torch.testing.assert_close(k.grad.cpu(), rounded(dk, dtype), atol=1e-4, rtol=1e-4)
    return actual


@pytest.mark.parametrize("lengths,groups,dim,block_size,scale", [
    ([1], 1, 1, 4, 1.0), ([0, 0], 2, 7, 4, 1.0), ([0, 3, 0, 2, 0], 2, 7, 4, 1.0), ([3, 7], 2, 7, 4, 1.0),
    ([7, 11], 4, 16, 8, 0.5), ([9], 2, 64, 4, 1.0), ([5], 4, 128, 128, 1.0),
    # scales that are not powers of two: exact path (Di 16) and MFMA path (Di 64, 128)
    ([7, 11], 4, 16, 8, 0.3), ([90, 41], 2, 64, 16, -1.7), ([300], 2, 128, 64, 0.1),
])
def test_score_forward_backward_fp64(lengths, groups, dim, block_size, scale, device):
    generator = torch.Generator().manual_seed(731)
    q_cpu = torch.randn(sum(lengths), groups, dim, generator=generator).to(torch.bfloat16)
    k_cpu = torch.randn(sum(lengths), 1, dim, generator=generator).to(torch.bfloat16)
    max_seqlen = max(lengths) + block_size
    nb = (max_seqlen + block_size - 1) // block_size
    upstream = torch.randn((sum(lengths), groups, nb), generator=generator).to(torch.bfloat16).float()
    _run(q_cpu, k_cpu, lengths, max_seqlen, block_size, scale, upstream, device)


@pytest.mark.parametrize("dim,dtype", [(128, torch.bfloat16), (128, torch.float16), (64, torch.bfloat16)],
                         ids=["bf16-128", "fp16-128", "bf16-64"])
def test_score_backward_many_exact_ties_in_one_segment(dim, dtype, device):
    """One index_k vector for every token makes every visible key of every block an exact
    tie: 380 tied (row, block) pairs per key block, all in one 8192-row segment of the
    key-block (dk) pass, more than its list of tied rows holds, so that pass takes its
    rescan path; each ds is split evenly over the tied keys. Scores bit-exact; gradients
    within the stated tolerance against the FP64 oracle (the products of one repeated key
    vector land exactly on rounding midpoints of the output type far more often than
    random data does, where the last bit of the FP64 sum of the split weights decides)."""
    from tests.helpers import check_bf16_stated
    from tests.test_gpu_sweep import _check_dtype_stated

    lengths, groups, block, scale = [150, 40], 2, 128, 1.0
    gen = torch.Generator().manual_seed(11)
    q_cpu = torch.randn(sum(lengths), groups, dim, generator=gen).to(dtype)
    k_cpu = torch.randn(1, 1, dim, generator=gen).to(dtype).expand(sum(lengths), 1, dim).contiguous()
    max_seqlen = max(lengths)
    nb = (max_seqlen + block - 1) // block
    upstream = torch.randn((sum(lengths), groups, nb), generator=gen).to(torch.bfloat16).float()
    q = q_cpu.to(device).clone().requires_grad_()
    k = k_cpu.to(device).clone().requires_grad_()
    cu = cu_tensor(lengths, device)
    scores = msa.m3_index_score(q, k, cu, max_seqlen, block_size=block, scale=scale)
    _, exp32, tie = O.index_score(q_cpu.double().numpy(), k_cpu.double().numpy(), cu_list(lengths), max_seqlen,
                                  block_size=block, scale=scale)
    np.testing.assert_array_equal(scores.detach().cpu().numpy(), exp32)
    assert int((tie[:lengths[0], :, 0] < 0).sum()) > 64  # block 0 of the first sequence: 298 tied rows
    scores.backward(upstream.to(device))
    dq, dk = O.index_score_backward(q_cpu.double().numpy(), k_cpu.double().numpy(), cu_list(lengths), max_seqlen,
                                    upstream.double().numpy(), block_size=block, scale=scale)
    for got, ref, what in ((q.grad, dq, "tied dq"), (k.grad, dk, "tied dk")):
        if dtype == torch.bfloat16:
            check_bf16_stated(got, ref, what)
        else:
            _check_dtype_stated(got, ref, dtype, what)


@pytest.mark.parametrize("lengths", [[127], [128], [129], [1, 129, 257]])
def test_score_causal_block_and_packing_boundaries(lengths, device):
    generator = torch.Generator().manual_seed(97)
    q = torch.randn(sum(lengths), 2, 4, generator=generator).to(torch.bfloat16)
    k = torch.randn(sum(lengths), 1, 4, generator=generator).to(torch.bfloat16)
    actual = msa.m3_index_score(q.to(device), k.to(device), cu_tensor(lengths, device), max(lengths), block_size=128)
    _, exp32, _ = O.index_score(q.double().numpy(), k.double().numpy(), cu_list(lengths), max(lengths), block_size=128)
    np.testing.assert_array_equal(actual.cpu().numpy(), exp32)


@pytest.mark.parametrize("scale", [1.0, 0.0, -1.0])
def test_score_ties_split_backward_and_invalid_blocks_have_zero_gradient(scale, device):
    q_cpu = torch.ones(5, 2, 3, dtype=torch.bfloat16)
    k_cpu = torch.ones(5, 1, 3, dtype=torch.bfloat16)
    _run(q_cpu, k_cpu, [2, 3], 8, 4, scale, torch.ones(5, 2, 2), device)


def test_score_groups_remain_independent(device):
    q = torch.tensor([[[1., 0.], [0., 1.]]] * 4, dtype=torch.bfloat16, device=device)
    k = torch.tensor([[[9., 1.]], [[1., 8.]], [[0., 0.]], [[0., 0.]]], dtype=torch.bfloat16, device=device)
    scores = msa.m3_index_score(q, k, cu_tensor([4], device), 4, block_size=1)
    assert scores.shape == (4, 2, 4)
    assert scores[-1, 0].argmax().item() == 0 and scores[-1, 1].argmax().item() == 1


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("scale", [1.0, -1.0, 0.0])
@pytest.mark.parametrize("case", ["cancellation_unique", "cancellation_tie", "rounded_score_tie"])
def test_score_winners_retain_low_bits(case, scale, dtype, device):
    small = 2**-12
    if case.startswith("cancellation"):
        query, key0 = [1.0, small, 1.0], [1.0, small, -1.0]
        key1 = [0.0, small if case.endswith("tie") else 0.0, 0.0]
    else:
        query, key0, key1 = [1.0, 1.0], [1.0, 2**-24], [1.0, 0.0]
    q_cpu = torch.tensor([[query], [query]], dtype=dtype)
    k_cpu = torch.tensor([[key0], [key1]], dtype=dtype)
    grad = torch.zeros(2, 1, 1)
    grad[1] = 1
    _run(q_cpu, k_cpu, [2], 2, 2, scale, grad, device)


@pytest.mark.parametrize("exact_tie", [False, True])
def test_fp32_product_residual_changes_winner(exact_tie, device):
    query = [1 + 2**-12, 1.0]
    q_cpu = torch.tensor([[query], [query]], dtype=torch.float32)
    k_cpu = torch.tensor([[[1 + 2**-12, -1 - 2**-11]], [[0.0, 2**-24 if exact_tie else 0.0]]], dtype=torch.float32)
    grad = torch.zeros(2, 1, 1)
    grad[1] = 1
    _run(q_cpu, k_cpu, [2], 2, 2, 1.0, grad, device)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_score_dtype_and_packed_backward(dtype, device):
    generator = torch.Generator().manual_seed(928)
    q_cpu = torch.randn(6, 2, 7, generator=generator).to(dtype)
    k_cpu = torch.randn(6, 1, 7, generator=generator).to(dtype)
    grad = torch.randn((6, 2, 2), generator=generator)
    _run(q_cpu, k_cpu, [2, 0, 4], 8, 4, 0.3, grad, device)


def test_no_grad_with_trainable_inputs_preserves_score_values(device):
    q = torch.tensor([[[1.0, 2**-12, 1.0]]] * 2, dtype=torch.bfloat16, device=device, requires_grad=True)
    k = torch.tensor([[[1.0, 2**-12, -1.0]], [[0.0, 0.0, 0.0]]], dtype=torch.bfloat16, device=device,
                     requires_grad=True)
    cu = cu_tensor([2], device)
    trainable = msa.m3_index_score(q, k, cu, 4, block_size=2)
    with torch.no_grad():
        inference = msa.m3_index_score(q, k, cu, 4, block_size=2)
    assert trainable.requires_grad and not inference.requires_grad
    torch.testing.assert_close(trainable, inference, atol=0, rtol=0)


@pytest.mark.parametrize("scale", [1.0, -1.0, 0.5])
@pytest.mark.parametrize("dim", [32, 64, 128])
def test_score_mfma_path_exact_ties(dim, scale, device):
    """Small-integer bf16 inputs make exact ties and near-ties common, so the MFMA
    path's ambiguous-row branch (full FP64 re-evaluation of the block) and its tie
    codes are exercised; the backward consumes those codes."""
    gen = torch.Generator().manual_seed(dim + int(4 * scale))
    lengths = [300, 77]
    q_cpu = torch.randint(-2, 3, (sum(lengths), 2, dim), generator=gen).to(torch.bfloat16)
    k_cpu = torch.randint(-2, 3, (sum(lengths), 1, dim), generator=gen).to(torch.bfloat16)
    block = 32
    nb = (max(lengths) + block - 1) // block
    upstream = torch.randn((sum(lengths), 2, nb), generator=gen).to(torch.bfloat16).float()
    _run(q_cpu, k_cpu, lengths, max(lengths), block, scale, upstream, device)


@pytest.mark.parametrize("integer", [False, True])
def test_score_backward_blocks_wider_than_128_keys(integer, device):
    """Key blocks of 200 keys (two key chunks in the dK pass); small-integer inputs
    add exact ties in both chunks."""
    gen = torch.Generator().manual_seed(200 + integer)
    lengths, groups, dim, block = [450, 130], 2, 16, 200
    if integer:
        q_cpu = torch.randint(-1, 2, (sum(lengths), groups, dim), generator=gen).to(torch.bfloat16)
        k_cpu = torch.randint(-1, 2, (sum(lengths), 1, dim), generator=gen).to(torch.bfloat16)
    else:
        q_cpu = torch.randn(sum(lengths), groups, dim, generator=gen).to(torch.bfloat16)
        k_cpu = torch.randn(sum(lengths), 1, dim, generator=gen).to(torch.bfloat16)
    nb = (max(lengths) + block - 1) // block
    upstream = torch.randn((sum(lengths), groups, nb), generator=gen).to(torch.bfloat16).float()
    _run(q_cpu, k_cpu, lengths, max(lengths), block, 1.0, upstream, device)


@pytest.mark.parametrize("lengths,groups,dim,block,seed", [
    ([1280 - 512, 512], 2, 64, 128, 71), ([2048], 4, 128, 128, 3), ([300, 1, 777], 3, 96, 64, 4),
])
def test_score_medium_sizes_bit_exact(lengths, groups, dim, block, seed, device):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(sum(lengths), groups, dim, generator=gen).bfloat16()
    k = torch.randn(sum(lengths), 1, dim, generator=gen).bfloat16()
    got = msa.m3_index_score(q.to(device), k.to(device), cu_tensor(lengths, device), max(lengths), block_size=block)
    _, exp32, _ = O.index_score(q.double().numpy(), k.double().numpy(), cu_list(lengths), max(lengths), block_size=block)
    np.testing.assert_array_equal(got.cpu().numpy(), exp32)


@pytest.mark.parametrize("scale", [1.0, -0.75])
def test_score_extreme_magnitudes_bit_exact(scale, device):
    """Query rows and keys with elements outside [2^-60, 2^55) (tiny rows, huge keys,
    bf16 subnormals mixed into normal rows): the MFMA pass cannot take their fp32
    products as exact, so these pairs are settled by the FP64 resolve pass; the FP64
    sums of the subnormal rows round, so the fixed summation order is what is checked."""
    gen = torch.Generator().manual_seed(61 + int(4 * scale))
    lengths, groups, dim, block = [700, 333], 2, 128, 128
    total = sum(lengths)
    q = torch.randn(total, groups, dim, generator=gen)
    k = torch.randn(total, 1, dim, generator=gen)
    q[0:40] *= 2.0 ** -70                      # tiny rows
    q[100:140, :, ::3] = 2.0 ** -130           # bf16 subnormals among normal elements
    q[150:160] *= 2.0 ** 62                    # huge rows
    k[5:9] *= 2.0 ** 64                        # huge keys in block 0 of sequence 0
    k[300:310, :, ::5] = 2.0 ** -128           # subnormal elements in block 2
    k[760:765] *= 2.0 ** -66                   # tiny keys in sequence 1
    q, k = q.bfloat16(), k.bfloat16()
    got = msa.m3_index_score(q.to(device), k.to(device), cu_tensor(lengths, device), max(lengths), block_size=block,
                             scale=scale)
    with np.errstate(over="ignore"):  # huge rows x huge keys overflow fp32 (inf), as on the GPU
        _, exp32, _ = O.index_score(q.double().numpy(), k.double().numpy(), cu_list(lengths), max(lengths),
                                    block_size=block, scale=scale)
    np.testing.assert_array_equal(got.cpu().numpy(), exp32)


@pytest.mark.parametrize("dim", [64, 40])
def test_score_nan_keys_mfma_and_exact_paths_agree(dim, device):
    """Keys holding NaN elements. No reference fixture pins NaN (numpy's max, like the
    eager path's amax, propagates it; fmax-style maxima skip it), so this checks that
    the two GPU paths agree bitwise on scores and tie codes: the bf16 MFMA pass with its
    FP64 resolve, and the FP64 exact kernel on the same values as fp32. NaN dots are
    skipped; a block whose visible dots are all NaN scores -inf with code 0. Cases: a
    block whose only unsafe key is NaN and whose other keys are zero (its stored norm is
    -0), a block of NaN keys, single NaN keys among normal ones; dim 40 puts the second
    query half 8 bytes into a 16-byte unit."""
    from msa_triton_amd.index_score import _score_forward
    from msa_triton_amd.layout import sequence_meta

    lengths, groups, block = [300, 200], 2, 32
    total = sum(lengths)
    gen = torch.Generator().manual_seed(5)
    q = torch.randn(total, groups, dim, generator=gen)
    k = torch.randn(total, 1, dim, generator=gen)
    k[0:32] = 0.0
    k[3, 0, 7] = float("nan")        # sequence 0, block 0: zero keys and one NaN key
    k[64:96, 0, 5] = float("nan")    # block 2: every key NaN
    k[130, 0, :] = float("nan")      # block 4: one NaN key among normal keys
    k[340, 0, 1] = float("nan")      # sequence 1, block 1
    qb, kb = q.bfloat16(), k.bfloat16()
    bounds = cu_list(lengths)
    meta = sequence_meta(bounds, block)
    cu = cu_tensor(lengths, device)
    out = {}
    for name, dtype in (("mfma", torch.bfloat16), ("exact", torch.float32)):
        sc, tie = _score_forward(qb.to(dtype).to(device).contiguous(), kb.to(dtype).to(device).contiguous(), cu, meta,
                                 max(lengths), block, 1.0, True)
        out[name] = (sc.cpu().numpy(), tie.cpu().numpy())
    np.testing.assert_array_equal(out["mfma"][0], out["exact"][0])
    np.testing.assert_array_equal(out["mfma"][1], out["exact"][1])
    sc, tie = out["mfma"]
    assert np.isneginf(sc[64:300, :, 2]).all() and (tie[64:300, :, 2] == 0).all()  # block 2: all dots NaN
    assert (sc[32:300, :, 0] == 0.0).all() and (tie[32:300, :, 0] == -31).all()  # 31 zero keys tie
    # every other (row, block) pair of the pack against the oracle (NaN keys excluded there)
    kk = kb.double().numpy()
    assert not np.isnan(sc).any()
    _, exp32, exp_tie = O.index_score(qb.double().numpy(), np.nan_to_num(kk, nan=0.0), bounds, max(lengths),
                                      block_size=block)
    clean = np.ones(sc.shape, dtype=bool)
    for a, blk in ((0, 0), (0, 2), (0, 4), (300, 1)):
        s_idx = 0 if a == 0 else 1
        lo = a + blk * block
        clean[lo:bounds[s_idx + 1], :, blk] = False  # rows that see a NaN key's block
    np.testing.assert_array_equal(sc[clean], exp32[clean])
    np.testing.assert_array_equal(tie[clean], exp_tie[clean])


@pytest.mark.parametrize("dim,dtype", [(640, torch.bfloat16), (1100, torch.float32)])
def test_score_index_dims_beyond_512(dim, dtype, device):
    """Index dims above 512 (no cap upstream): the exact forward, and the backward in
    passes of 512 dims; bit-exact scores, gradients within the reference gate."""
    gen = torch.Generator().manual_seed(dim)
    lengths, groups, block = [70, 45], 2, 16
    q_cpu = torch.randn(sum(lengths), groups, dim, generator=gen).to(dtype)
    k_cpu = torch.randn(sum(lengths), 1, dim, generator=gen).to(dtype)
    nb = (max(lengths) + block - 1) // block
    upstream = torch.randn((sum(lengths), groups, nb), generator=gen).to(torch.bfloat16).float()
    _run(q_cpu, k_cpu, lengths, max(lengths), block, 1.0, upstream, device)
