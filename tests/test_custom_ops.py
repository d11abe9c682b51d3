"""torch.library registration (no GPU): the ops exist in the msa_mi355x namespace,
their fake kernels give the eager operators' output shapes and dtypes, and the
compile-path wrappers keep the eager static checks."""

from __future__ import annotations

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

from msa_triton_amd import custom_ops as C


def test_ops_are_registered():
    for name in ("index_score", "index_score_backward", "topk", "sparse_attention", "sparse_attention_backward",
                 "indexer_kl"):
        assert hasattr(torch.ops.msa_mi355x, name)


def test_fake_kernels_shapes_and_dtypes():
    with FakeTensorMode():
        iq = torch.empty(37, 3, 64, dtype=torch.bfloat16, device="cuda")
        ik = torch.empty(37, 1, 64, dtype=torch.bfloat16, device="cuda")
        cu = torch.empty(3, dtype=torch.int32, device="cuda")
        scores, tie = torch.ops.msa_mi355x.index_score(iq, ik, cu, 30, 8, 1.0, True)
        assert scores.shape == (37, 3, 4) and scores.dtype == torch.float32
        assert tie.shape == (37, 3, 4) and tie.dtype == torch.int32
        _, tie0 = torch.ops.msa_mi355x.index_score(iq, ik, cu, 30, 8, 1.0, False)
        assert tie0.shape == (0,)
        dq, dk = torch.ops.msa_mi355x.index_score_backward(iq, ik, cu, tie, scores, 30, 8, 1.0, True, False)
        assert dq.shape == iq.shape and dq.dtype == iq.dtype and dk.shape == (0,)
        ids = torch.ops.msa_mi355x.topk(scores, cu, 8, 5, 1)
        assert ids.shape == (37, 3, 5) and ids.dtype == torch.int32
        q = torch.empty(37, 6, 32, dtype=torch.bfloat16, device="cuda")
        kv = torch.empty(37, 3, 32, dtype=torch.bfloat16, device="cuda")
        out, lse, rs, o32 = torch.ops.msa_mi355x.sparse_attention(q, kv, kv, ids, cu, 30, 8, 0.25, True)
        assert out.shape == q.shape and out.dtype == q.dtype
        assert lse.shape == (37, 6) and lse.dtype == torch.float32 and rs.shape == (37, 6, 4) and rs.dtype == torch.float64
        assert o32.shape == q.shape and o32.dtype == torch.float32
        assert torch.ops.msa_mi355x.sparse_attention(q, kv, kv, ids, cu, 30, 8, 0.25, False)[3].shape == (0,)
        dq, dk, dv = torch.ops.msa_mi355x.sparse_attention_backward(q, kv, kv, ids, cu, out, rs, o32, out, 8, 0.25,
                                                                    False, True, True)
        assert dq.shape == (0,) and dk.shape == kv.shape and dv.shape == kv.shape
        loss, rows, d_iq, d_ik = torch.ops.msa_mi355x.indexer_kl(iq, ik, q, kv, ids, cu, 30, 8, 1.0, 0.25, True,
                                                                 False, None)
        assert loss.shape == () and loss.dtype == torch.float32 and rows.shape == (37, 3)
        assert d_iq.shape == iq.shape and d_iq.dtype == torch.float32 and d_ik.shape == (0,)


def test_wrappers_keep_static_checks():
    q = torch.zeros(4, 2, 8, dtype=torch.bfloat16)
    kv = torch.zeros(4, 1, 8, dtype=torch.bfloat16)
    cu = torch.tensor([0, 4], dtype=torch.int32)
    with pytest.raises(TypeError, match="dtype"):
        C.m3_sparse_attention(q.float(), kv, kv, torch.zeros(4, 1, 1, dtype=torch.int32), cu, 4)
    with pytest.raises(ValueError, match="scale must be finite"):
        C.m3_sparse_attention(q, kv, kv, torch.zeros(4, 1, 1, dtype=torch.int32), cu, 4, scale=float("inf"))
    with pytest.raises(ValueError, match="local_blocks"):
        C.m3_topk(torch.zeros(4, 1, 1), cu, topk_blocks=1, local_blocks=2)
    with pytest.raises(ValueError, match="rank-3"):
        C.m3_index_score(q[0], kv, cu, 4)
