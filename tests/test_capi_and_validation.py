"""CPU checks of the drop-in boundary: the C-ABI library and the host validation.

* the built library loads and exports every entry point include/msa_mi355x.h
  declares, with the argument counts the ctypes bindings use;
* the public operators raise the reference's exception types and messages
  (triton/index_score.py:325-355, triton/topk.py:13-30, triton/k2q.py:54-81,
  triton/sparse_attention.py:452-483, layout.py:12-24) before any device work;
* valid CPU tensors are refused (there is no CPU execution path).
"""

from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest
import torch

import msa_triton_amd as msa
from msa_triton_amd import _lib
from msa_triton_amd.k2q import build_k2q_csr

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "msa_mi355x.h")


def _declared():
    text = open(HEADER).read()
    decls = {}
    for match in re.finditer(r"^(?:int|int64_t)\s+(msa_\w+)\(([^;]*)\);", text, flags=re.M | re.S):
        params = [p for p in match.group(2).split(",") if p.strip() and p.strip() != "void"]
        decls[match.group(1)] = len(params)
    return decls


def test_library_exports_every_declared_symbol():
    decls = _declared()
    assert len(decls) >= 10
    handle = _lib.lib()
    for name, nparams in decls.items():
        assert hasattr(handle, name), name
        assert name in _lib.SIGNATURES, name
        assert len(_lib.SIGNATURES[name][1]) == nparams, name
    assert set(_lib.SIGNATURES) == set(decls)


def test_host_only_helpers():
    handle = _lib.lib()
    cb = np.array([0, 2, 3], dtype=np.int32)
    assert handle.msa_k2q_counter_elems(2, cb.ctypes.data, 4) == 4 * (3 + 1)
    # block-major (tie, ds) copies plus FP64 dk partials: 3 blocks x 1 key group x 1 segment x 8 keys x 128 dims
    assert handle.msa_score_bwd_workspace_bytes(10, 2, 3, 8, 4, 3) >= 10 * 2 * 3 * 8 + 3 * 8 * 128 * 8
    # bf16 and fp16 run the KV-major MFMA kernels (same workspace layout for both)
    for code in (1, 2):
        assert handle.msa_attn_fwd_workspace_bytes(code, 256, 8, 2, 64, 4, 2, 128) > 0
        assert handle.msa_attn_bwd_workspace_bytes(code, 256, 8, 2, 64, 4, 2, 128) > 0
    assert (handle.msa_attn_bwd_workspace_bytes(1, 256, 8, 2, 64, 4, 2, 128)
            == handle.msa_attn_bwd_workspace_bytes(2, 256, 8, 2, 64, 4, 2, 128))
    # fp32 and unsupported shapes (D % 8 != 0, blocks above 128) run the VALU kernels: no workspace
    assert handle.msa_attn_fwd_workspace_bytes(0, 256, 8, 2, 64, 4, 2, 128) == 0
    assert handle.msa_attn_bwd_workspace_bytes(0, 256, 8, 2, 64, 4, 2, 128) == 0
    for code in (1, 2):
        assert handle.msa_attn_bwd_workspace_bytes(code, 256, 8, 2, 60, 4, 2, 128) == 0
        assert handle.msa_attn_fwd_workspace_bytes(code, 256, 8, 2, 64, 4, 2, 131) == 0


def _cu(values):
    return torch.tensor(values, dtype=torch.int32)


def test_score_validation_messages():
    q = torch.ones(3, 2, 4)
    k = torch.ones(3, 1, 4)
    with pytest.raises(ValueError, match="nondecreasing"):
        msa.m3_index_score(q, k, _cu([0, 2, 1, 3]), 3)
    with pytest.raises(ValueError, match="max_seqlen"):
        msa.m3_index_score(q, k, _cu([0, 3]), 2)
    with pytest.raises(ValueError, match="rank-3"):
        msa.m3_index_score(q[0], k, _cu([0, 3]), 3)
    with pytest.raises(TypeError, match="BF16, FP16, or FP32"):
        msa.m3_index_score(q.double(), k.double(), _cu([0, 3]), 3)
    with pytest.raises(ValueError, match="scale must be finite"):
        msa.m3_index_score(q, k, _cu([0, 3]), 3, scale=float("nan"))
    with pytest.raises(ValueError, match="block_size"):
        msa.m3_index_score(q, k, _cu([0, 3]), 3, block_size=0)
    with pytest.raises(RuntimeError, match="ROCm device"):
        msa.m3_index_score(q, k, _cu([0, 3]), 3)


def test_topk_validation_messages():
    s = torch.zeros(3, 2, 2)
    with pytest.raises(ValueError, match="FP32"):
        msa.m3_topk(s.double(), _cu([0, 3]))
    with pytest.raises(ValueError, match="nondecreasing"):
        msa.m3_topk(s, _cu([0, 2, 1, 3]), block_size=2)
    with pytest.raises(ValueError, match="local_blocks"):
        msa.m3_topk(s, _cu([0, 3]), block_size=2, topk_blocks=1, local_blocks=2)
    with pytest.raises(ValueError, match="enough block slots"):
        msa.m3_topk(s, _cu([0, 3]), block_size=1)
    with pytest.raises(RuntimeError, match="ROCm device"):
        msa.m3_topk(s, _cu([0, 3]), block_size=2)


def test_k2q_validation_messages_and_capacity_overflow():
    ids = torch.zeros(3, 2, 4, dtype=torch.int32)
    with pytest.raises(ValueError, match="nondecreasing"):
        build_k2q_csr(ids, _cu([0, 2, 1, 3]), block_size=2)
    with pytest.raises(ValueError, match="span T"):
        build_k2q_csr(ids, _cu([0, 2]), block_size=2)
    with pytest.raises(ValueError, match="block_size"):
        build_k2q_csr(ids, _cu([0, 3]), block_size=0)
    oversized = torch.tensor(0, dtype=torch.int32).expand(1, 2, 2**30)
    with pytest.raises(OverflowError, match="edge capacity"):
        build_k2q_csr(oversized, _cu([0, 1]), block_size=1)


def test_attention_validation_messages():
    q = torch.randn(2, 1, 4)
    k = torch.randn(2, 1, 4)
    ids = torch.zeros(2, 1, 1, dtype=torch.int32)
    cu = _cu([0, 2])
    for bad in (float("nan"), float("inf"), -float("inf")):
        with pytest.raises(ValueError, match="scale must be finite"):
            msa.m3_sparse_attention(q, k, k, ids, cu, 2, block_size=2, scale=bad)
    with pytest.raises(ValueError, match="positive integer"):
        msa.m3_sparse_attention(q, k, k, ids, cu, 0, block_size=2)
    with pytest.raises(ValueError, match="smaller"):
        msa.m3_sparse_attention(q, k, k, ids, cu, 1, block_size=2)
    with pytest.raises(ValueError, match="end at total_tokens"):
        msa.m3_sparse_attention(q, k, k, ids, _cu([0, 1]), 2, block_size=2)
    with pytest.raises(TypeError, match="share a BF16"):
        msa.m3_sparse_attention(q.double(), k.double(), k.double(), ids, cu, 2)
    with pytest.raises(ValueError, match="multiple of G"):
        msa.m3_sparse_attention(torch.randn(2, 3, 4), torch.randn(2, 2, 4), torch.randn(2, 2, 4),
                                torch.zeros(2, 2, 1, dtype=torch.int32), cu, 2)
    with pytest.raises(ValueError, match="int32 \\[T,G,K\\]"):
        msa.m3_sparse_attention(q, k, k, ids.long(), cu, 2)
    with pytest.raises(RuntimeError, match="ROCm device"):
        msa.m3_sparse_attention(q, k, k, ids, cu, 2, block_size=2)


def test_fused_score_topk_validation_messages():
    iq = torch.zeros(4, 1, 8, dtype=torch.bfloat16)
    ik = torch.zeros(4, 1, 8, dtype=torch.bfloat16)
    cu = torch.tensor([0, 4], dtype=torch.int32)
    with pytest.raises(ValueError, match="max_seqlen"):
        msa.m3_index_score_topk(iq, ik, cu, 3, block_size=2, topk_blocks=1)
    with pytest.raises(ValueError, match="local_blocks"):
        msa.m3_index_score_topk(iq, ik, cu, 4, block_size=2, topk_blocks=1, local_blocks=2)
    with pytest.raises(ValueError, match="topk_blocks"):
        msa.m3_index_score_topk(iq, ik, cu, 4, block_size=2, topk_blocks=-1)


def test_ratio_magic_division_is_exact_in_its_range():
    """The kernels split a work item's row index x into (edge, head) with
    x / r = umulhi(x, ceil(2^32 / r)) for x * r < 2^32 (attn_kv_common.hpp
    div_by_ratio); exhaustive over the ranges the kernels use (r <= 512, x < 512 r)."""
    import numpy as np

    for r in range(2, 513):
        magic = ((1 << 32) + r - 1) // r
        x = np.arange(512 * r, dtype=np.uint64)
        assert np.array_equal((x * np.uint64(magic)) >> np.uint64(32), x // np.uint64(r)), r


def test_indexer_kl_validation_messages():
    iq = torch.zeros(6, 2, 32, dtype=torch.bfloat16)
    ik = torch.zeros(6, 1, 32, dtype=torch.bfloat16)
    q = torch.zeros(6, 4, 32, dtype=torch.bfloat16)
    k = torch.zeros(6, 2, 32, dtype=torch.bfloat16)
    ids = torch.zeros(6, 2, 1, dtype=torch.int32)
    cu = torch.tensor([0, 6], dtype=torch.int32)
    with pytest.raises(ValueError, match="index_k"):
        msa.m3_indexer_kl(iq, ik[:, :, :16], q, k, ids, cu, 6)
    with pytest.raises(ValueError, match="matching index_q"):
        msa.m3_indexer_kl(iq, ik, q, k[:, :1], ids, cu, 6)
    with pytest.raises(ValueError, match="multiple of G"):
        msa.m3_indexer_kl(iq, ik, q[:, :3], k, ids, cu, 6)
    with pytest.raises(ValueError, match="indices"):
        msa.m3_indexer_kl(iq, ik, q, k, ids.long(), cu, 6)
    with pytest.raises(TypeError, match="dtype"):
        msa.m3_indexer_kl(iq, ik, q.half(), k, ids, cu, 6)
    with pytest.raises(ValueError, match="block_size"):
        msa.m3_indexer_kl(iq, ik, q, k, ids, cu, 6, block_size=0)
    with pytest.raises(ValueError, match="finite"):
        msa.m3_indexer_kl(iq, ik, q, k, ids, cu, 6, scale=float("nan"))
    with pytest.raises(ValueError, match="max_seqlen"):
        msa.m3_indexer_kl(iq, ik, q, k, ids, cu, 5)
    with pytest.raises(RuntimeError):  # valid CPU tensors: no CPU execution path
        msa.m3_indexer_kl(iq, ik, q, k, ids, cu, 6)
