"""CPU restatement of the reference's eager sparse attention -- TEST / BASELINE INFRASTRUCTURE ONLY.

Follows eager/ops.py:153-180 (sparse_attention_bsnd) of the reference for one
packed sequence: bf16 Q.K^T * scale over the dense key range with the block
keep mask (eager/ops.py:132-150), masked_fill(-inf), fp32 softmax cast back to
bf16, bf16 P.V, and torch autograd for the backward. It is used only as the
``cpu_baseline`` leg of bench.py, row-chunked so that a bounded sample of query
rows can be timed (softmax rows are independent, so chunking changes no value
and the work adds up linearly over chunks). Never imported by the product path.
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
