"""GPU parity of the whole pipeline at the BASELINE.json configurations.

Inputs are the benchmark's (bench.make_inputs: seed 71, the reference
benchmark's draw order, c4's per-group index_q jitter). For every config:

* scores: bit-exact against the FP64 oracle (rounded once to fp32) on sampled
  query tokens (all of them for c1);
* top-k: bit-exact against the oracle selection applied to the GPU scores of the
  sampled tokens (all tokens for c1-c4);
* k2q CSR: all four arrays bit-exact against the oracle restatement;
* attention: out / lse / dQ on sampled query tokens and dK / dV on sampled keys
  against the sparse FP64 oracle (oracle.attention_rows / attention_kv_rows);
  c1 also checks every attention output and gradient against the dense FP64
  oracle and the score backward against the dense FP64 amax subgradient.

Tolerance for bf16 outputs (stated): every element within 1e-4 + 2^-8 |x| of
the FP64 value x (one bf16 ulp relative, or 1e-4 absolute near zero), and at
most 0.1% of the elements outside the reference's own gate (atol = rtol = 1e-4
after rounding x to bf16). lse (fp32) uses the gate. The bf16 rounding of a
value that fp32 arithmetic puts within ~2^-24 of a rounding midpoint can go
either way; at 10^5 - 10^6 outputs a few such one-ulp flips are expected from
any fp32 implementation, the reference's included (its own tests use ~10^3
outputs per case, where the gate is met exactly; so do ours).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import bench
import msa_triton_amd as msa
from msa_triton_amd import _lib
from msa_triton_amd.k2q import build_k2q_csr
from oracle import msa_oracle as O
from tests.helpers import check_bf16_stated as _check_bf16

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(600)]  # c5 oracle work takes ~1 min on the host


def _bounds(lengths):
    b = [0]
    for n in lengths:
        b.append(b[-1] + n)
    return b


def _sample_tokens(lengths, block, rng, extra=4):
    """First / block-boundary / last tokens of every sequence plus a few random ones."""
    out = set()
    bounds = _bounds(lengths)
    for a, n in zip(bounds[:-1], lengths):
        if n == 0:
            continue
        for p in (0, 1, block - 1, block, 2 * block - 1, n // 2, n - block, n - 2, n - 1):
            if 0 <= p < n:
                out.add(a + p)
        out.update(int(x) for x in a + rng.integers(0, n, size=extra))
    return np.array(sorted(out), dtype=np.int64)


# Backward chunk budget per config: the default (3 GiB) except c3, set to 2 GiB so that its
# third sequence's keys are summed across three chunks.
BWD_BUDGET = {"c3": 2 << 30}


def _bwd_chunk_tokens(cfg, total, budget):
    """Query tokens per backward chunk at `budget` bytes (kv_chunk_tokens: records of
    D * 4 + 8 bytes per (token, head, slot), at least 64 tokens, balanced chunks)."""
    per_token = cfg["hq"] * cfg["topk"] * (cfg["d"] * 4 + 8)
    tc = max(64, budget // per_token)
    if total <= tc:
        return total
    nch = -(-total // tc)
    return -(-total // nch)


def _sample_keys(lengths, block, name):
    """Keys of the last blocks of the longest sequence (few query tokens see them), and
    early keys whose blocks are selected by query tokens of several backward chunks, so
    that their dK / dV are sums the backward carries across chunks: c3's third sequence
    (tokens 5120-10239 straddle the chunk boundary at 5462 at its 2 GiB budget), c4 blocks
    0, 40 and 120 (three chunks), c5 blocks 0 and 3 (22 chunks)."""
    bounds = _bounds(lengths)
    s = int(np.argmax(lengths))
    a, n = bounds[s], lengths[s]
    keys = {a + n - 1, a + n - block, a + max(0, n - 3 * block) + 5}
    if name in ("c1", "c2", "c3"):
        keys.update({a, a + block // 2, a + n // 2})
    if name == "c3":
        keys.update({bounds[2], bounds[2] + 77, bounds[2] + 10 * block + 3})
    if name == "c4":
        keys.update({0, 5, 40 * block + 3, 120 * block + 77})
    if name == "c5":
        keys.update({0, 3 * block + 50})
    return np.array(sorted(keys), dtype=np.int64)


def _assert_multi_chunk_keys(cfg, name, ids_np, bounds, keys):
    """Each early key of c3-c5 gets edges from at least two backward chunks."""
    tc = _bwd_chunk_tokens(cfg, bounds[-1], BWD_BUDGET.get(name, 3 << 30))
    spanning = 0
    for j in keys:
        s = int(np.searchsorted(bounds, j, side="right") - 1)
        blk = (int(j) - bounds[s]) // cfg["block"]
        hit = np.nonzero((ids_np[j:bounds[s + 1]] == blk).any(-1).any(-1))[0] + j
        spanning += len(np.unique(hit // tc)) >= 2
    if name in ("c3", "c4", "c5"):
        assert spanning >= 2, f"{name}: only {spanning} sampled keys span several backward chunks"


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c4", "c5"])
def test_pipeline_against_oracle(name, device):
    cfg = bench.CONFIGS[name]
    lengths, B, K, L = cfg["lengths"], cfg["block"], cfg["topk"], cfg["local"]
    bounds = _bounds(lengths)
    T, max_len = bounds[-1], max(lengths)
    nb = (max_len + B - 1) // B
    cu_np = np.array(bounds, dtype=np.int32)
    iq, ik, q, k, v, dout = bench.make_inputs(cfg)
    cu = torch.tensor(bounds, dtype=torch.int32, device=device)
    rng = np.random.default_rng(2024)
    print(f"[{name}] T={T} Hq={cfg['hq']} G={cfg['g']} K={K} L={L}", flush=True)

    # ---- stage 1 and 2
    with torch.no_grad():
        scores = msa.m3_index_score(iq.to(device), ik.to(device), cu, max_len, block_size=B)
        ids = msa.m3_topk(scores, cu, block_size=B, topk_blocks=K, local_blocks=L)
    scores_np = scores.cpu().numpy()
    ids_np = ids.cpu().numpy()
    tokens = np.arange(T) if name == "c1" else _sample_tokens(lengths, B, rng)
    iq64, ik64 = iq.double().numpy(), ik.double().numpy()
    _, ref32 = O.index_score_rows(iq64, ik64, cu_np, tokens, nb, block_size=B)
    np.testing.assert_array_equal(scores_np[tokens], ref32, err_msg=f"{name}: scores")
    if name == "c5":
        starts = np.array(bounds)[np.searchsorted(bounds, tokens, side="right") - 1]
        ref_ids = O.topk_rows(scores_np[tokens], tokens - starts, block_size=B, topk_blocks=K, local_blocks=L)
        np.testing.assert_array_equal(ids_np[tokens], ref_ids, err_msg=f"{name}: top-k")
    else:
        ref_ids = O.topk(scores_np, cu_np, block_size=B, topk_blocks=K, local_blocks=L)
        np.testing.assert_array_equal(ids_np, ref_ids, err_msg=f"{name}: top-k")

    # ---- k2q CSR, all edges
    csr = build_k2q_csr(ids, cu, block_size=B)
    ref = O.k2q_csr(ids_np, cu_np, block_size=B)
    for got, want, what in zip((csr.row_ptr, csr.query_indices, csr.slot_indices, csr.cu_block_lens), ref,
                               ("row_ptr", "query_indices", "slot_indices", "cu_block_lens")):
        np.testing.assert_array_equal(got.cpu().numpy(), want, err_msg=f"{name}: {what}")

    # ---- stage 3 forward + backward
    qd, kd, vd = (x.to(device).requires_grad_() for x in (q, k, v))
    with _lib.chunk_budgets(bwd=BWD_BUDGET.get(name)):
        out, lse = msa.m3_sparse_attention(qd, kd, vd, ids, cu, max_len, block_size=B, return_lse=True)
        out.backward(dout.to(device))
        torch.cuda.synchronize()
    q64, k64, v64, do64 = (x.double().numpy() for x in (q, k, v, dout))
    if name == "c1":
        # dense FP64 oracle over every token and key
        o_ref, lse_ref, dq_ref, dk_ref, dv_ref = O.sparse_attention(q64, k64, v64, ids_np, cu_np, block_size=B,
                                                                    dout=do64)
        rows = {"out": o_ref, "lse": lse_ref, "dq": dq_ref}
        keys = np.arange(T)
    else:
        rows = O.attention_rows(q64, k64, v64, ids_np, cu_np, tokens, block_size=B, dout=do64)
        keys = _sample_keys(lengths, B, name)
        _assert_multi_chunk_keys(cfg, name, ids_np, bounds, keys)
        dk_ref, dv_ref = O.attention_kv_rows(q64, k64, v64, ids_np, cu_np, do64, keys, block_size=B)
    _check_bf16(out[tokens], rows["out"], f"{name}: out")
    _check_bf16(qd.grad[tokens], rows["dq"], f"{name}: dq")
    lse_np = lse.cpu().numpy()[tokens]
    assert np.array_equal(np.isneginf(lse_np), np.isneginf(rows["lse"]))
    fin = np.isfinite(rows["lse"])
    np.testing.assert_allclose(lse_np[fin], rows["lse"][fin], atol=1e-4, rtol=1e-4, err_msg=f"{name}: lse")
    _check_bf16(kd.grad[keys], dk_ref, f"{name}: dk")
    _check_bf16(vd.grad[keys], dv_ref, f"{name}: dv")

    # ---- stage 1 backward (dense FP64 oracle)
    if name == "c1":
        a = iq.to(device).requires_grad_()
        b = ik.to(device).requires_grad_()
        sc = msa.m3_index_score(a, b, cu, max_len, block_size=B)
        g = torch.randn(sc.shape, generator=torch.Generator().manual_seed(9)).masked_fill(torch.isinf(sc.cpu()), 0)
        sc.backward(g.to(device))
        dq_ref, dk_ref = O.index_score_backward(iq64, ik64, cu_np, max_len, g.double().numpy(), block_size=B)
        _check_bf16(a.grad, dq_ref, f"{name}: score dq")
        _check_bf16(b.grad, dk_ref, f"{name}: score dk")


@pytest.mark.parametrize("name", ["c2", "c3", "c4", "c5"])
def test_score_backward_against_oracle(name, device):
    """Stage-1 backward at the large configs with an N(0,1) upstream gradient: dq of sampled
    query tokens and dk of sampled keys (early blocks: heavy fan-in over many 8192-row
    segments; late blocks) against the FP64 amax subgradient (index_score_backward_rows /
    _keys, pinned against the dense restatement on the CPU)."""
    cfg = bench.CONFIGS[name]
    lengths, B = cfg["lengths"], cfg["block"]
    bounds = _bounds(lengths)
    max_len = max(lengths)
    cu_np = np.array(bounds, dtype=np.int32)
    iq, ik = bench.make_inputs(cfg)[:2]
    cu = torch.tensor(bounds, dtype=torch.int32, device=device)
    print(f"[{name}] score backward T={bounds[-1]} G={cfg['g']}", flush=True)
    a = iq.to(device).requires_grad_()
    b = ik.to(device).requires_grad_()
    sc = msa.m3_index_score(a, b, cu, max_len, block_size=B)
    g = torch.randn(sc.shape, generator=torch.Generator().manual_seed(9)).masked_fill(torch.isinf(sc.detach().cpu()), 0)
    sc.backward(g.to(device))
    torch.cuda.synchronize()
    g_np = g.numpy()
    iq64, ik64 = iq.double().numpy(), ik.double().numpy()
    tokens = _sample_tokens(lengths, B, np.random.default_rng(2025))
    dq_ref = O.index_score_backward_rows(iq64, ik64, cu_np, g_np, tokens, block_size=B)
    _check_bf16(a.grad[tokens], dq_ref, f"{name}: score dq")
    s = int(np.argmax(lengths))
    keys = {bounds[s], bounds[s] + 77, bounds[s] + lengths[s] // 2, bounds[s + 1] - 1}
    keys.update(bounds[i] + 3 for i in range(len(lengths)))
    keys = np.array(sorted(keys), dtype=np.int64)
    dk_ref = O.index_score_backward_keys(iq64, ik64, cu_np, g_np, keys, block_size=B)
    _check_bf16(b.grad[keys], dk_ref, f"{name}: score dk")


@pytest.mark.parametrize("name,dtype", [("c2", torch.float16), ("c4", torch.float16), ("c2", torch.float32)],
                         ids=["c2-fp16", "c4-fp16", "c2-fp32"])
def test_fp16_fp32_attention_at_baseline_configs(name, dtype, device):
    """The FP64 attention kernels at BASELINE sizes: the benchmark's q / k / v / dO in fp16
    or fp32 with the benchmark's selection (bf16 score and top-k); out / lse / dQ of sampled
    query tokens and dK / dV of sampled keys against the sparse FP64 oracle, fp32 within
    the reference's gate, fp16 within its stated analogue (one fp16 ulp, at most 0.1 %
    outside the gate)."""
    from tests.test_gpu_sweep import _check_dtype_stated

    cfg = bench.CONFIGS[name]
    lengths, B, K, L = cfg["lengths"], cfg["block"], cfg["topk"], cfg["local"]
    bounds = _bounds(lengths)
    max_len = max(lengths)
    cu_np = np.array(bounds, dtype=np.int32)
    iq, ik, q, k, v, dout = bench.make_inputs(cfg)
    q, k, v, dout = (x.to(dtype) for x in (q, k, v, dout))
    cu = torch.tensor(bounds, dtype=torch.int32, device=device)
    print(f"[{name} {dtype}] T={bounds[-1]} Hq={cfg['hq']} G={cfg['g']} K={K}", flush=True)
    with torch.no_grad():
        ids = msa.m3_topk(msa.m3_index_score(iq.to(device), ik.to(device), cu, max_len, block_size=B), cu,
                          block_size=B, topk_blocks=K, local_blocks=L)
    qd, kd, vd = (x.to(device).requires_grad_() for x in (q, k, v))
    out, lse = msa.m3_sparse_attention(qd, kd, vd, ids, cu, max_len, block_size=B, return_lse=True)
    out.backward(dout.to(device))
    torch.cuda.synchronize()
    assert out.dtype == dtype and qd.grad.dtype == dtype
    ids_np = ids.cpu().numpy()
    tokens = _sample_tokens(lengths, B, np.random.default_rng(2025))
    keys = _sample_keys(lengths, B, name)
    q64, k64, v64, do64 = (x.double().numpy() for x in (q, k, v, dout))
    rows = O.attention_rows(q64, k64, v64, ids_np, cu_np, tokens, block_size=B, dout=do64)
    dk_ref, dv_ref = O.attention_kv_rows(q64, k64, v64, ids_np, cu_np, do64, keys, block_size=B)
    _check_dtype_stated(out[tokens], rows["out"], dtype, f"{name}: out")
    _check_dtype_stated(qd.grad[tokens], rows["dq"], dtype, f"{name}: dq")
    _check_dtype_stated(kd.grad[keys], dk_ref, dtype, f"{name}: dk")
    _check_dtype_stated(vd.grad[keys], dv_ref, dtype, f"{name}: dv")
    lse_np = lse.cpu().numpy()[tokens]
    assert np.array_equal(np.isneginf(lse_np), np.isneginf(rows["lse"]))
    fin = np.isfinite(rows["lse"])
    np.testing.assert_allclose(lse_np[fin], rows["lse"][fin], atol=1e-4, rtol=1e-4, err_msg=f"{name}: lse")


@pytest.mark.parametrize("name,dtype", [("c2", torch.bfloat16), ("c4", torch.bfloat16), ("c2", torch.float16)],
                         ids=["c2-bf16", "c4-bf16", "c2-fp16"])
def test_head_dim_256_attention_at_baseline_configs(name, dtype, device):
    """Head dim 256 on the MFMA kernels at BASELINE sizes: the config's tokens, heads and
    selection (bf16 score and top-k from the benchmark's index inputs) with seeded N(0, 1)
    q / k / v / dO of 256 dims; out / lse / dQ of sampled query tokens and dK / dV of
    sampled keys against the sparse FP64 oracle within the dtype's stated tolerance."""
    from tests.test_gpu_sweep import _check_dtype_stated

    cfg = bench.CONFIGS[name]
    lengths, B, K, L = cfg["lengths"], cfg["block"], cfg["topk"], cfg["local"]
    bounds = _bounds(lengths)
    max_len = max(lengths)
    cu_np = np.array(bounds, dtype=np.int32)
    iq, ik = bench.make_inputs(cfg)[:2]
    T = bounds[-1]
    g = torch.Generator().manual_seed(2560)
    q, k, v, dout = (torch.randn(T, h, 256, generator=g).to(dtype) for h in (cfg["hq"], cfg["g"], cfg["g"], cfg["hq"]))
    cu = torch.tensor(bounds, dtype=torch.int32, device=device)
    print(f"[{name} {dtype} D=256] T={T} Hq={cfg['hq']} G={cfg['g']} K={K}", flush=True)
    with torch.no_grad():
        ids = msa.m3_topk(msa.m3_index_score(iq.to(device), ik.to(device), cu, max_len, block_size=B), cu,
                          block_size=B, topk_blocks=K, local_blocks=L)
    qd, kd, vd = (x.to(device).requires_grad_() for x in (q, k, v))
    out, lse = msa.m3_sparse_attention(qd, kd, vd, ids, cu, max_len, block_size=B, return_lse=True)
    out.backward(dout.to(device))
    torch.cuda.synchronize()
    ids_np = ids.cpu().numpy()
    tokens = _sample_tokens(lengths, B, np.random.default_rng(256))
    keys = _sample_keys(lengths, B, name)
    q64, k64, v64, do64 = (x.double().numpy() for x in (q, k, v, dout))
    rows = O.attention_rows(q64, k64, v64, ids_np, cu_np, tokens, block_size=B, dout=do64)
    dk_ref, dv_ref = O.attention_kv_rows(q64, k64, v64, ids_np, cu_np, do64, keys, block_size=B)
    check = _check_bf16 if dtype == torch.bfloat16 else (lambda a, r, n: _check_dtype_stated(a, r, dtype, n))
    check(out[tokens], rows["out"], f"{name}: out")
    check(qd.grad[tokens], rows["dq"], f"{name}: dq")
    check(kd.grad[keys], dk_ref, f"{name}: dk")
    check(vd.grad[keys], dv_ref, f"{name}: dv")
    lse_np = lse.cpu().numpy()[tokens]
    assert np.array_equal(np.isneginf(lse_np), np.isneginf(rows["lse"]))
    fin = np.isfinite(rows["lse"])
    np.testing.assert_allclose(lse_np[fin], rows["lse"][fin], atol=1e-4, rtol=1e-4, err_msg=f"{name}: lse")
