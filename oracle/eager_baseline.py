"""CPU restatement of the reference's eager path -- TEST / BASELINE INFRASTRUCTURE ONLY.

Follows eager/ops.py:153-180 (sparse_attention_bsnd) of the reference for one
packed sequence: bf16 Q.K^T * scale over the dense key range with the block
keep mask (eager/ops.py:132-150), masked_fill(-inf), fp32 softmax cast back to
bf16, bf16 P.V, and torch autograd for the backward. It is used only as the
``cpu_baseline`` leg of bench.py, row-chunked so that a bounded sample of query
rows can be timed (softmax rows are independent, so chunking changes no value
and the work adds up linearly over chunks). ``eager_score_rows`` and ``eager_topk``
restate the eager indexer score (eager/ops.py:45-67) and selection
(eager/ops.py:112-129) for the same purpose. Never imported by the product path.
"""

from __future__ import annotations

import torch


def eager_rows_fwd_bwd(q, k, v, indices, rows, *, block_size, scale, dout, key_limit=None):
    """Forward + backward of the eager formulation for query rows ``rows`` of a
    single sequence starting at token 0. Keys span [0, key_limit) (the dense
    row of the reference's [S,S] weights; default: the whole sequence).
    Returns (out_rows, dq_rows, dk, dv) as bf16 tensors."""
    r0, r1 = rows
    total, heads, dim = q.shape
    groups = k.shape[1]
    ratio = heads // groups
    key_limit = total if key_limit is None else key_limit
    qr = q[r0:r1].detach().clone().requires_grad_()
    kk = k[:key_limit].detach().clone().requires_grad_()
    vv = v[:key_limit].detach().clone().requires_grad_()
    ids = indices[r0:r1].long()  # [n, G, K]
    n = r1 - r0
    blocks = (key_limit + block_size - 1) // block_size
    safe = ids.masked_fill((ids < 0) | (ids >= blocks), blocks)
    keep_blocks = torch.zeros((n, groups, blocks + 1), dtype=torch.bool)
    keep_blocks.scatter_(-1, safe, True)
    keep = keep_blocks[..., :blocks].repeat_interleave(block_size, dim=-1)[..., :key_limit]  # [n, G, S]
    pos = torch.arange(r0, r1)[:, None]
    keep = keep & (torch.arange(key_limit)[None, None, :] <= pos[:, :, None])
    keep = keep.repeat_interleave(ratio, dim=1)  # [n, Hq, S]
    query = qr.transpose(0, 1)  # [Hq, n, D]
    key = kk.transpose(0, 1).repeat_interleave(ratio, dim=0)  # [Hq, S, D]
    value = vv.transpose(0, 1).repeat_interleave(ratio, dim=0)
    weights = torch.matmul(query, key.transpose(-1, -2).contiguous()) * scale  # [Hq, n, S] bf16
    mask = keep.transpose(0, 1)
    weights = weights.masked_fill(~mask, float("-inf"))
    has = mask.any(-1, keepdim=True)
    safe_w = torch.where(has, weights, torch.zeros_like(weights))
    probs = torch.softmax(safe_w, dim=-1, dtype=torch.float32).to(q.dtype).masked_fill(~has, 0)
    out = torch.matmul(probs, value).transpose(0, 1)  # [n, Hq, D]
    out.backward(dout[r0:r1])
    return out.detach(), qr.grad, kk.grad, vv.grad


def eager_score_rows(index_q, index_k, rows, *, block_size, scale=1.0):
    """Scores of query rows ``rows`` of a single sequence starting at token 0, as the
    reference's eager index_score_bsnd computes them (eager/ops.py:45-67): fp32
    Q.K^T over the dense key range of the sequence, causal mask, -inf padding to
    whole blocks and a block amax. Returns fp32 [n, G, blocks]."""
    r0, r1 = rows
    length = index_k.shape[0]
    q = index_q[r0:r1].float().transpose(0, 1)  # [G, n, Di]
    k = index_k.float().transpose(0, 1)  # [1, S, Di]
    scores = torch.matmul(q, k.transpose(-1, -2))  # [G, n, S]
    if scale != 1.0:
        scores = scores * scale
    keep = torch.arange(length)[None, :] <= torch.arange(r0, r1)[:, None]
    scores = scores.masked_fill(~keep[None], float("-inf"))
    blocks = (length + block_size - 1) // block_size
    scores = torch.nn.functional.pad(scores, (0, blocks * block_size - length), value=float("-inf"))
    scores = scores.reshape(scores.shape[0], r1 - r0, blocks, block_size).amax(-1)
    return scores.transpose(0, 1)


@torch.no_grad()
def eager_topk(scores, positions, *, block_size, topk_blocks, local_blocks):
    """The reference's eager m3_topk selection (eager/ops.py:112-129) for rows with
    sequence-local ``positions``: causal mask, +inf local boost, torch.topk, -inf ->
    -1, right padding to topk_blocks. Returns int32 [n, G, topk_blocks]."""
    blocks = torch.arange(scores.shape[-1])
    query_block = positions // block_size
    valid = blocks[None, None, :] <= query_block[:, None, None]
    boosted = scores.masked_fill(~valid, float("-inf"))
    if local_blocks:
        local = (blocks[None, None, :] > query_block[:, None, None] - local_blocks) & valid
        boosted = boosted.masked_fill(local, float("inf"))
    count = min(topk_blocks, scores.shape[-1])
    values, indices = boosted.topk(count, dim=-1)
    indices = indices.masked_fill(values == float("-inf"), -1).to(torch.int32)
    return torch.nn.functional.pad(indices, (0, topk_blocks - count), value=-1)
