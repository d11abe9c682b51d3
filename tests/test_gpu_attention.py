"""GPU parity of stage 3 (m3_sparse_attention forward + backward) against the FP64 oracle.

Gate: the reference's own, atol=rtol=1e-4 after rounding the FP64 oracle to the
public dtype (tests/test_triton_attention.py:58-97). Cases mirror
tests/test_triton_attention.py: the 8 shape cases, empty selection,
non-contiguous inputs, future-only selections, empty packing, scale/metadata
errors, the 257-token rounding regression, hot KV rows, slot-order invariance,
the 7 needs-grad combinations with the CSR spy, fp16/fp32 and GQA=16.
"""

from __future__ import annotations

import importlib

import numpy as np
import pytest
import torch

import msa_triton_amd as msa
from oracle import msa_oracle as O
from tests.helpers import attention_inputs, check_bf16_stated, np64, rounded

pytestmark = pytest.mark.gpu


def _to(device, tensors, indices, cu):
    return tuple(x.to(device).detach().requires_grad_() for x in tensors), indices.to(device), cu.to(device)


def _oracle(tensors, indices, cu, block_size, scale=None, dout=None):
    return O.sparse_attention(*(np64(x) for x in tensors), indices.cpu().numpy(), cu.cpu().numpy(),
                              block_size=block_size, scale=scale,
                              dout=None if dout is None else np64(dout))


def _close(actual, expected_np, dtype=torch.bfloat16):
    torch.testing.assert_close(actual.detach().cpu(), rounded(expected_np, dtype), atol=1e-4, rtol=1e-4)


def _assert_lse(actual, expected):
    actual = actual.detach().cpu()
    expected = torch.from_numpy(expected).float()
    assert torch.equal(torch.isneginf(actual), torch.isneginf(expected))
    finite = torch.isfinite(expected)
    torch.testing.assert_close(actual[finite], expected[finite], atol=1e-4, rtol=1e-4)


# The reference's attention test shapes (tests/test_triton_attention.py:58-93).
REFERENCE_SHAPES = [
    ([1], 1, 1, 5, 128, 1, None),
    ([7, 3], 2, 2, 8, 3, 3, None),
    ([17, 5], 3, 1, 16, 8, 2, 0.2),
    ([129, 1], 1, 2, 8, 128, 3, None),
    ([127, 128, 257], 1, 1, 8, 128, 3, None),
    ([5, 1, 9], 2, 4, 32, 4, 4, None),
    ([5, 3], 2, 2, 128, 4, 2, None),
    ([0, 3, 0, 2, 0], 2, 2, 8, 2, 2, None),
]


@pytest.mark.parametrize("lengths,groups,ratio,dimension,block_size,topk,scale", REFERENCE_SHAPES)
def test_forward_backward_against_fp64(lengths, groups, ratio, dimension, block_size, topk, scale, device):
    cpu, indices, cu = attention_inputs(lengths, groups, ratio, dimension, block_size, topk)
    tensors, indices_d, cu_d = _to(device, cpu, indices, cu)
    grad = torch.randn(cpu[0].shape, generator=torch.Generator().manual_seed(5678)).bfloat16()
    out, lse, dq, dk, dv = _oracle(cpu, indices, cu, block_size, scale, grad)
    actual, actual_lse = msa.m3_sparse_attention(*tensors, indices_d, cu_d, max(lengths), block_size=block_size,
                                                 scale=scale, return_lse=True)
    assert actual.dtype == torch.bfloat16 and actual_lse.dtype == torch.float32 and not actual_lse.requires_grad
    _close(actual, out)
    _assert_lse(actual_lse, lse)
    actual.backward(grad.to(device))
    for tensor, ref in zip(tensors, (dq, dk, dv)):
        _close(tensor.grad, ref)


@pytest.mark.parametrize("lengths,groups,ratio,dimension,block_size,topk,scale", REFERENCE_SHAPES)
def test_fp16_forward_backward_against_fp64(lengths, groups, ratio, dimension, block_size, topk, scale, device):
    """The reference's test shapes with fp16 inputs (the reference's q / k / v values, cast
    to fp16): the MFMA kernels wherever the shape fits them (all but head dim 5), against
    the FP64 oracle within the stated fp16 tolerance -- every element within
    1e-4 + 2^-10 |x| of the FP64 value, at most 0.1 % (at least one) outside the gate.
    fp16 has 3 more significant bits than bf16, so a value is about 8 times likelier to
    fall within fp32 arithmetic's reach of an fp16 rounding midpoint."""
    from msa_triton_amd import _lib
    from tests.test_gpu_sweep import _check_dtype_stated

    cpu, indices, cu = attention_inputs(lengths, groups, ratio, dimension, block_size, topk)
    cpu = tuple(x.to(torch.float16) for x in cpu)
    total, heads = sum(lengths), groups * ratio
    blocks = sum((n + block_size - 1) // block_size for n in lengths)
    on_mfma = _lib.lib().msa_attn_fwd_workspace_bytes(1, total, heads, groups, dimension, topk, blocks,
                                                      block_size) > 0
    assert on_mfma == (dimension % 8 == 0)
    tensors, indices_d, cu_d = _to(device, cpu, indices, cu)
    grad = torch.randn(cpu[0].shape, generator=torch.Generator().manual_seed(5678)).to(torch.float16)
    out, lse, dq, dk, dv = _oracle(cpu, indices, cu, block_size, scale, grad)
    actual, actual_lse = msa.m3_sparse_attention(*tensors, indices_d, cu_d, max(lengths), block_size=block_size,
                                                 scale=scale, return_lse=True)
    assert actual.dtype == torch.float16
    _check_dtype_stated(actual, out, torch.float16, "out")
    _assert_lse(actual_lse, lse)
    actual.backward(grad.to(device))
    for tensor, ref, name in zip(tensors, (dq, dk, dv), ("dq", "dk", "dv")):
        _check_dtype_stated(tensor.grad, ref, torch.float16, name)


def test_fp16_gradients_follow_power_of_two_output_gradients(device):
    """fp16 on the MFMA kernels carries dS into dK under a per-key power-of-two scale (from
    the running maximum of |dS|) and P under a fixed 2^15. Scaling dO by 2^s (exact: every
    |dO| in [2^-2, 2^2), s = -10 .. 5) scales every fp32 / fp64 quantity of the backward
    exactly, so dQ, dK and dV must come out as 2^s times the s = 0 gradients bit for bit
    (where those stay in fp16's normal range; within a subnormal step, scaled, below it). A
    peaked softmax (scale 0.5) spreads dS over many binades within each tile. The s = 0
    run is checked against the FP64 oracle within the stated fp16 tolerance."""
    from tests.test_gpu_sweep import _check_dtype_stated

    lengths, groups, ratio, dim, block, topk, scale = [300, 45], 2, 4, 64, 16, 5, 0.5
    cpu, indices, cu = attention_inputs(lengths, groups, ratio, dim, block, topk)
    cpu = tuple(x.to(torch.float16) for x in cpu)
    g = torch.Generator().manual_seed(77)
    mag = 2.0 ** (torch.rand(cpu[0].shape, generator=g) * 4 - 2)  # [2^-2, 2^2)
    sign = torch.where(torch.rand(cpu[0].shape, generator=g) < 0.5, -1.0, 1.0)
    dout = (sign * mag).to(torch.float16)
    out_ref, _, dq_ref, dk_ref, dv_ref = _oracle(cpu, indices, cu, block, scale, dout)
    results = {}
    for shift in (0, -10, 5):
        tensors, indices_d, cu_d = _to(device, cpu, indices, cu)
        out = msa.m3_sparse_attention(*tensors, indices_d, cu_d, max(lengths), block_size=block, scale=scale)
        out.backward((dout.double() * 2.0 ** shift).to(torch.float16).to(device))
        results[shift] = [t.grad.detach().cpu().double() for t in tensors]
        if shift == 0:
            _check_dtype_stated(out, out_ref, torch.float16, "out")
            for grad, ref, name in zip(results[0], (dq_ref, dk_ref, dv_ref), ("dq", "dk", "dv")):
                _check_dtype_stated(grad, ref, torch.float16, name)
    for shift in (-10, 5):
        for base, got, name in zip(results[0], results[shift], ("dq", "dk", "dv")):
            want = base * 2.0 ** shift
            normal = (want.abs() >= 2.0 ** -14) & (base.abs() >= 2.0 ** -14)
            assert torch.equal(got[normal], want[normal]), f"{name} at 2^{shift}: not an exact power-of-two image"
            # below the normal range one of the two roundings lands on the subnormal grid (step 2^-24)
            limit = 2.0 ** -24 * max(1.0, 2.0 ** shift)
            assert float((got - want).abs().max()) <= limit, f"{name} at 2^{shift}: subnormal outputs"
            print(f"{name} at 2^{shift}: {int(normal.sum())} of {base.numel()} compared bit for bit", flush=True)
            assert int(normal.sum()) > 0.5 * base.numel()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("lengths,groups,ratio,dimension,block_size,topk,scale", [
    ([300, 45], 2, 4, 256, 16, 5, None),
    ([127, 128, 257], 1, 3, 200, 128, 3, 0.1),
    ([5, 1, 9], 2, 2, 136, 4, 4, None),
])
def test_head_dims_to_256_on_mfma_against_fp64(lengths, groups, ratio, dimension, block_size, topk, scale, dtype,
                                               device):
    """Head dims above 128 (up to 256) on the MFMA kernels: the forward with 8 waves of 16
    rows, the backward's main pass as two launches over the two 128-dim halves of dK, dV and
    dQ (each recomputing S and dP over every dim). Against the FP64 oracle within the
    stated tolerance of the dtype (bf16: 1e-4 + 2^-8 |x|, fp16: 1e-4 + 2^-10 |x|; at most
    0.1 %, at least one, outside the gate)."""
    from msa_triton_amd import _lib
    from tests.test_gpu_sweep import _check_dtype_stated

    cpu, indices, cu = attention_inputs(lengths, groups, ratio, dimension, block_size, topk)
    cpu = tuple(x.to(dtype) for x in cpu)
    total, heads = sum(lengths), groups * ratio
    blocks = sum((n + block_size - 1) // block_size for n in lengths)
    lib = _lib.lib()
    code = _lib.DTYPE_CODE[dtype]
    assert lib.msa_attn_fwd_workspace_bytes(code, total, heads, groups, dimension, topk, blocks, block_size) > 0
    assert lib.msa_attn_bwd_workspace_bytes(code, total, heads, groups, dimension, topk, blocks, block_size) > 0
    tensors, indices_d, cu_d = _to(device, cpu, indices, cu)
    grad = torch.randn(cpu[0].shape, generator=torch.Generator().manual_seed(256)).to(dtype)
    out, lse, dq, dk, dv = _oracle(cpu, indices, cu, block_size, scale, grad)
    actual, actual_lse = msa.m3_sparse_attention(*tensors, indices_d, cu_d, max(lengths), block_size=block_size,
                                                 scale=scale, return_lse=True)
    check = (lambda a, r, n: check_bf16_stated(a, r, n)) if dtype == torch.bfloat16 else (
        lambda a, r, n: _check_dtype_stated(a, r, torch.float16, n))
    check(actual, out, "out")
    _assert_lse(actual_lse, lse)
    actual.backward(grad.to(device))
    for tensor, ref, name in zip(tensors, (dq, dk, dv), ("dq", "dk", "dv")):
        check(tensor.grad, ref, name)


@pytest.mark.parametrize("topk", [0, 3])
def test_empty_selection_has_zero_output_and_gradients(topk, device):
    cpu, indices, cu = attention_inputs([3, 2], 2, 2, 7, 2, topk)
    tensors, indices, cu = _to(device, cpu, indices, cu)
    indices.fill_(-1)
    output, lse = msa.m3_sparse_attention(*tensors, indices, cu, 3, block_size=2, return_lse=True)
    assert torch.count_nonzero(output) == 0 and torch.isneginf(lse).all()
    output.sum().backward()
    for tensor in tensors:
        assert tensor.grad is not None and torch.count_nonzero(tensor.grad) == 0


def test_noncontiguous_inputs_and_masked_queries(device):
    cpu, indices, cu = attention_inputs([5, 2], 2, 2, 5, 3, 2)
    indices[1] = -1
    tensors, indices_d, cu_d = _to(device, cpu, indices, cu)
    tensors = tuple(x.detach().transpose(1, 2).contiguous().transpose(1, 2).requires_grad_() for x in tensors)
    assert not tensors[0].is_contiguous()
    grad = torch.randn(cpu[0].shape, generator=torch.Generator().manual_seed(73)).bfloat16()
    out, lse, dq, dk, dv = _oracle(cpu, indices, cu, 3, None, grad)
    actual, actual_lse = msa.m3_sparse_attention(*tensors, indices_d, cu_d, 5, block_size=3, return_lse=True)
    _close(actual, out)
    _assert_lse(actual_lse, lse)
    actual.backward(grad.to(device))
    for tensor, ref in zip(tensors, (dq, dk, dv)):
        _close(tensor.grad, ref)
    assert torch.count_nonzero(tensors[0].grad[1]) == 0


def test_default_return_is_output_tensor(device):
    cpu, indices, cu = attention_inputs([2], 1, 1, 4, 2, 1)
    tensors, indices, cu = _to(device, cpu, indices, cu)
    output = msa.m3_sparse_attention(*tensors, indices, cu, 2, block_size=2)
    assert isinstance(output, torch.Tensor) and output.shape == tensors[0].shape


def test_future_only_selected_blocks_are_safely_masked(device):
    cpu, indices, cu = attention_inputs([5, 2], 1, 2, 8, 3, 1)
    indices.fill_(1)
    tensors, indices_d, cu_d = _to(device, cpu, indices, cu)
    ones = torch.ones(cpu[0].shape, dtype=torch.bfloat16)
    out, lse, dq, dk, dv = _oracle(cpu, indices, cu, 3, None, ones)
    actual, actual_lse = msa.m3_sparse_attention(*tensors, indices_d, cu_d, 5, block_size=3, return_lse=True)
    _close(actual, out)
    _assert_lse(actual_lse, lse)
    actual.sum().backward()
    for tensor, ref in zip(tensors, (dq, dk, dv)):
        _close(tensor.grad, ref)


def test_empty_packed_input(device):
    cpu, indices, cu = attention_inputs([0, 0], 1, 2, 8, 4, 1)
    tensors, indices, cu = _to(device, cpu, indices, cu)
    output, lse = msa.m3_sparse_attention(*tensors, indices, cu, 4, block_size=4, return_lse=True)
    assert output.shape == (0, 2, 8) and lse.shape == (0, 2)
    output.sum().backward()
    for tensor in tensors:
        assert tensor.grad is not None and tensor.grad.shape == tensor.shape


def test_rejects_invalid_sequence_metadata_on_device(device):
    cpu, indices, cu = attention_inputs([2], 1, 1, 4, 2, 1)
    tensors, indices, cu = _to(device, cpu, indices, cu)
    with pytest.raises(ValueError, match="scale must be finite"):
        msa.m3_sparse_attention(*tensors, indices, cu, 2, block_size=2, scale=float("nan"))
    with pytest.raises(ValueError, match="smaller"):
        msa.m3_sparse_attention(*tensors, indices, cu, 1, block_size=2)
    cu[-1] = 1
    with pytest.raises(ValueError, match="end at total_tokens"):
        msa.m3_sparse_attention(*tensors, indices, cu, 2, block_size=2)


def test_long_key_accumulation_bf16_rounding_regression(device):
    rng = np.random.default_rng(1234)
    cpu = tuple(torch.from_numpy(rng.standard_normal((512, 1, 8))).float().bfloat16()[255:] for _ in range(3))
    grad = torch.from_numpy(rng.standard_normal((512, 1, 8))).float().bfloat16()[255:]
    indices = torch.full((257, 1, 3), -1, dtype=torch.int32)
    for token in range(257):
        current = token // 128
        chosen = [current] + [b for b in range(current) if b % 2 == 0]
        indices[token, 0, : len(chosen)] = torch.tensor(chosen, dtype=torch.int32)
    cu = torch.tensor([0, 257], dtype=torch.int32)
    tensors, indices_d, cu_d = _to(device, cpu, indices, cu)
    out, _, dq, dk, dv = _oracle(cpu, indices, cu, 128, None, grad)
    actual = msa.m3_sparse_attention(*tensors, indices_d, cu_d, 257)
    _close(actual, out)
    actual.backward(grad.to(device))
    for tensor, ref in zip(tensors, (dq, dk, dv)):
        _close(tensor.grad, ref)


def test_hot_kv_rows_match_fp64(device):
    lengths, groups, ratio, dim, block_size = [41, 5], 2, 4, 16, 8
    cpu, _, cu = attention_inputs(lengths, groups, ratio, dim, block_size, 2)
    selected = torch.full((sum(lengths), groups, 2), -1, dtype=torch.int32)
    start = 0
    for length in lengths:
        for position in range(length):
            selected[start + position, 0, 0] = 0
            selected[start + position, 1, 0] = position // block_size
        start += length
    tensors, indices_d, cu_d = _to(device, cpu, selected, cu)
    grad = torch.randn(cpu[0].shape, generator=torch.Generator().manual_seed(819)).bfloat16()
    out, _, dq, dk, dv = _oracle(cpu, selected, cu, block_size, None, grad)
    actual = msa.m3_sparse_attention(*tensors, indices_d, cu_d, max(lengths), block_size=block_size)
    _close(actual, out)
    actual.backward(grad.to(device))
    for tensor, ref in zip(tensors, (dq, dk, dv)):
        _close(tensor.grad, ref)


def test_selected_block_order_preserves_output_and_gradients(device):
    cpu, indices, cu = attention_inputs([9, 3], 2, 2, 7, 3, 3)
    reordered = torch.full(indices.shape, -1, dtype=torch.int32)
    for token in range(indices.shape[0]):
        for group in range(indices.shape[1]):
            valid = indices[token, group]
            valid = valid[valid >= 0].flip(0)
            reordered[token, group, : valid.numel()] = valid
    grad = torch.randn(cpu[0].shape, generator=torch.Generator().manual_seed(127)).bfloat16()
    out, _, dq, dk, dv = _oracle(cpu, indices, cu, 3, None, grad)
    for selected in (indices, reordered):
        tensors, sel_d, cu_d = _to(device, cpu, selected, cu)
        actual = msa.m3_sparse_attention(*tensors, sel_d, cu_d, 9, block_size=3)
        _close(actual, out)
        actual.backward(grad.to(device))
        for tensor, ref in zip(tensors, (dq, dk, dv)):
            _close(tensor.grad, ref)


@pytest.mark.parametrize("needs_grad", [
    (True, False, False), (False, True, False), (False, False, True),
    (True, True, False), (True, False, True), (False, True, True), (True, True, True),
])
def test_independent_input_gradients_and_q_only_skips_csr(needs_grad, device, monkeypatch):
    cpu, indices, cu = attention_inputs([0, 5, 0, 3, 0], 2, 2, 8, 3, 2)
    indices[2] = -1
    tensors = tuple(x.to(device).detach().requires_grad_(need) for x, need in zip(cpu, needs_grad))
    saved_inputs = tuple(x.detach().clone() for x in tensors)
    k2q_module = importlib.import_module("msa_triton_amd.k2q")
    original_build = k2q_module.build_k2q_csr
    csr_calls = []

    def checked_build(*args, **kwargs):
        assert needs_grad[1] or needs_grad[2], "Q-only backward must not build CSR"
        csr_calls.append(True)
        return original_build(*args, **kwargs)

    monkeypatch.setattr(k2q_module, "build_k2q_csr", checked_build)
    grad = torch.randn(cpu[0].shape, generator=torch.Generator().manual_seed(190)).bfloat16()
    out, _, dq, dk, dv = _oracle(cpu, indices, cu, 3, None, grad)
    actual = msa.m3_sparse_attention(*tensors, indices.to(device), cu.to(device), 5, block_size=3)
    _close(actual, out)
    actual.backward(grad.to(device))
    assert len(csr_calls) == int(needs_grad[1] or needs_grad[2])
    for tensor, saved in zip(tensors, saved_inputs):
        torch.testing.assert_close(tensor.detach(), saved, atol=0, rtol=0)
    for tensor, ref, need in zip(tensors, (dq, dk, dv), needs_grad):
        if need:
            _close(tensor.grad, ref)
        else:
            assert tensor.grad is None


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_dtype_and_gqa16_forward_backward_against_fp64(dtype, device):
    _, indices, cu = attention_inputs([5, 3], 1, 16, 8, 3, 2)
    generator = torch.Generator().manual_seed(320)
    shapes = ((8, 16, 8), (8, 1, 8), (8, 1, 8))
    cpu = tuple(torch.randn(s, generator=generator).to(dtype) for s in shapes)
    grad = torch.randn(cpu[0].shape, generator=generator).to(dtype)
    out, lse, dq, dk, dv = _oracle(cpu, indices, cu, 3, None, grad)
    tensors, indices_d, cu_d = _to(device, cpu, indices, cu)
    actual, actual_lse = msa.m3_sparse_attention(*tensors, indices_d, cu_d, 5, block_size=3, return_lse=True)
    _close(actual, out, dtype)
    _assert_lse(actual_lse, lse)
    actual.backward(grad.to(device))
    for tensor, ref in zip(tensors, (dq, dk, dv)):
        _close(tensor.grad, ref, dtype)


@pytest.mark.parametrize("lengths,groups,ratio,dimension,block_size,topk,scale,stated", [
    ([5, 1, 9], 2, 4, 32, 4, 4, None, False),
    ([300, 45], 2, 4, 64, 16, 5, 0.02, True),
    ([127, 128, 257], 1, 8, 128, 128, 3, 0.02, True),
    ([127, 128, 257], 1, 8, 128, 128, 3, 0.5, True),
])
def test_backward_with_and_without_fp32_output(lengths, groups, ratio, dimension, block_size, topk, scale, stated,
                                               device):
    """The C-ABI backward both ways, each against the FP64 oracle: with the forward's
    fp32 output (flat rows take delta = O . dO, rows the forward marked peaked take
    the statistics pass; the autograd function's path) and without it (the
    reference's centred statistics pass for every row). With the small scale about
    a quarter to a half of the rows are flat (rows with few visible keys stay
    peaked); the large scale peaks them all. These use the stated tolerance; the
    small case meets the reference's gate."""
    from msa_triton_amd.layout import sequence_meta
    from msa_triton_amd.sparse_attention import _attn_backward, _attn_forward

    cpu, indices, cu = attention_inputs(lengths, groups, ratio, dimension, block_size, topk)
    grad = torch.randn(cpu[0].shape, generator=torch.Generator().manual_seed(4321)).bfloat16()
    out_ref, _, dq, dk, dv = _oracle(cpu, indices, cu, block_size, scale, grad)
    q, k, v = (x.to(device).contiguous() for x in cpu)
    ids, cu_d = indices.to(device), cu.to(device)
    meta = sequence_meta(cu.tolist(), block_size)
    sc = dimension ** -0.5 if scale is None else scale
    out, _, row_state, out_f32, _ = _attn_forward(q, k, v, ids, cu_d, meta, block_size, sc, None, save_f32=True)
    torch.testing.assert_close(out_f32.to(torch.bfloat16), out, atol=0, rtol=0)
    peaked = row_state[..., 1] < 0
    assert bool(peaked.any())
    if scale is not None and scale < 0.1:
        assert not bool(peaked.all())
    runs = {}
    for name, saved in (("fp32", out_f32), ("stats", None)):
        grads = _attn_backward(q, k, v, ids, cu_d, out, row_state.clone(), grad.to(device), meta, block_size, sc,
                               None, True, True, True, out_f32=saved)
        runs[name] = grads
        for actual, ref, what in zip(grads, (dq, dk, dv), ("dq", "dk", "dv")):
            if stated:
                check_bf16_stated(actual, ref, f"{name} {what}")
            else:
                _close(actual, ref)
    # rows that take the statistics pass either way get the same dQ bit for bit
    torch.testing.assert_close(runs["fp32"][0][peaked], runs["stats"][0][peaked], atol=0, rtol=0)


@pytest.mark.parametrize("dimension,dtype", [(640, torch.bfloat16), (1100, torch.float32), (2048, torch.float16)])
def test_head_dims_beyond_512_against_fp64(dimension, dtype, device):
    """Head dims above 512 run the VALU kernels in passes of 512 output dims (the logits
    always cover every dim); forward, lse and all gradients within the reference gate."""
    _, indices, cu = attention_inputs([9, 6], 2, 2, 8, 4, 2)
    generator = torch.Generator().manual_seed(dimension)
    shapes = ((15, 4, dimension), (15, 2, dimension), (15, 2, dimension))
    cpu = tuple((0.25 * torch.randn(s, generator=generator)).to(dtype) for s in shapes)
    grad = torch.randn(cpu[0].shape, generator=generator).to(dtype)
    out, lse, dq, dk, dv = _oracle(cpu, indices, cu, 4, None, grad)
    tensors, indices_d, cu_d = _to(device, cpu, indices, cu)
    actual, actual_lse = msa.m3_sparse_attention(*tensors, indices_d, cu_d, 9, block_size=4, return_lse=True)
    _close(actual, out, dtype)
    _assert_lse(actual_lse, lse)
    actual.backward(grad.to(device))
    for tensor, ref in zip(tensors, (dq, dk, dv)):
        _close(tensor.grad, ref, dtype)
