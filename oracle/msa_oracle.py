"""CPU oracle for the MiniMax-M3 sparse-attention path -- TEST INFRASTRUCTURE ONLY.

This module restates the reference algorithm in numpy (float64 / int64) so that
the HIP kernels can be checked against it. It is imported only by ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``; the
product path (``msa_triton_amd``) never calls it.

Functions and the reference code they restate:
  index_score          triton/index_score.py:93-136, tests/reference_fp64.py:16-45
  index_score_backward triton/index_score.py:139-232 (amax subgradient,
                       ties split evenly as torch.amax, eager/ops.py:81-82)
  topk                 triton/topk.py:31-46 (eager/ops.py:94-129)
  k2q_csr              triton/k2q.py:94-128
  sparse_attention     tests/reference_fp64.py:48-85 (dense per sequence/group)
  sparse_attention_backward   gradient of the above (softmax backward)
  attention_rows / attention_kv_rows   the same math restricted to sampled
                       query rows / key rows, gathering only selected blocks,
                       for parity at sizes where the dense form does not fit.
  index_score_rows / topk_rows   index_score / topk for a subset of query
                       rows (pinned against the full restatements).
  index_score_backward_rows / _keys   index_score_backward's dq for a subset of
                       query tokens / dk for a subset of key tokens (pinned against
                       the full restatement).
  indexer_kl (+ _rows, _key_rows)   the indexer KL branch, not implemented
                       upstream: restated from docs/msa_training_flow.md:92-138
                       and docs/implementation_plan.md:66-69 (pinned by closed
                       forms, finite differences and torch float64 autograd of an
                       independent dense formulation, tests/test_oracle_kl.py).

Pinning (see tests/test_oracle_*.py): every function is checked against the
reference's known-answer cases (tests/test_eager.py:143-170,
tests/test_topk.py:20-66, tests/test_k2q.py:101-135,
tests/test_triton_score.py:133-182, docs/code_review_response.md:33-41 and
:246-250), against independent brute force (exact rational dots, pure-Python
ranking and inversion loops) and against torch float64 autograd of an
independently written dense formulation.

Order conventions: ``topk`` emits descending values with ties in ascending
block order (the drop-in's documented canonical order; torch.topk leaves tie
order unspecified, so the reference's order among equal values is unpinned).
"""

from __future__ import annotations

import numpy as np


def bounds_of(cu) -> list[int]:
    return [int(x) for x in np.asarray(cu).reshape(-1)]


def _token_positions(bounds):
    """(seq id, sequence start) for every packed token."""
    total = bounds[-1]
    seq = np.zeros(total, dtype=np.int64)
    start = np.zeros(total, dtype=np.int64)
    for s, (a, b) in enumerate(zip(bounds[:-1], bounds[1:])):
        seq[a:b] = s
        start[a:b] = a
    return seq, start


# --------------------------------------------------------------------------- stage 1


def public_score(best, scale):
    """The reference's public fp32 score (triton/index_score.py:121-127, fp32 arithmetic
    with fusion disabled) of directed block maxima ``best`` (float64): the fp32 pair
    hi = fl32(x), lo = fl32(x - hi), each times s = fl32(|scale|), added in fp32.
    Non-finite hi gives hi * s."""
    x = np.asarray(best, dtype=np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        hi = x.astype(np.float32)
        finite = np.isfinite(hi)
        lo = np.where(finite, x - np.where(finite, hi, 0).astype(np.float64), 0.0).astype(np.float32)
        s = np.float32(abs(scale))
        return np.where(finite, hi * s + lo * s, hi * s).astype(np.float32)


def index_score(iq, ik, cu, max_seqlen, *, block_size=128, scale=1.0):
    """Exact block maxima.

    Returns (scores_f64, scores_f32, tie) where scores_f64[t,g,b] is
    max over causal keys j of block b of scale * (iq[t,g] . ik[j]) evaluated in
    float64 (-inf if none), scores_f32 the public score (``public_score`` of the
    directed maximum: its fp32 rounding when |scale| is 1 or 0), and tie the
    winner code: offset+1 for a unique maximum, -count for ties, 0 for blocks
    without causal keys. Winners compare the directed dot sign(scale) * dot, as
    the reference's compensated comparison does.
    """
    q = np.asarray(iq, dtype=np.float64)
    k = np.asarray(ik, dtype=np.float64)[:, 0, :]
    bounds = bounds_of(cu)
    total, groups, _ = q.shape
    nb = (max_seqlen + block_size - 1) // block_size
    out = np.full((total, groups, nb), -np.inf)
    tie = np.zeros((total, groups, nb), dtype=np.int32)
    pub = np.full((total, groups, nb), -np.inf, dtype=np.float32)
    sign = 1.0 if scale > 0 else (-1.0 if scale < 0 else 0.0)
    for a, b in zip(bounds[:-1], bounds[1:]):
        length = b - a
        for blk in range(nb):
            lo, hi = blk * block_size, min((blk + 1) * block_size, length)
            if lo >= hi:
                continue
            dots = np.einsum("tgd,kd->tgk", q[a:b], k[a + lo : a + hi])  # [S,G,n]
            pos = np.arange(length)[:, None]
            allowed = np.arange(lo, hi)[None, :] <= pos  # [S, n]
            directed = np.where(allowed[:, None, :], sign * dots, -np.inf)
            best = directed.max(-1)
            valid = allowed.any(-1)
            winners = (directed == best[..., None]) & allowed[:, None, :]
            count = winners.sum(-1)
            first = winners.argmax(-1)
            code = np.where(count == 1, first + 1, -count).astype(np.int32)
            with np.errstate(invalid="ignore"):
                scores = np.abs(scale) * best
            out[a:b, :, blk] = np.where(valid[:, None], scores, -np.inf)
            pub[a:b, :, blk] = np.where(valid[:, None], public_score(best, scale), np.float32(-np.inf))
            tie[a:b, :, blk] = np.where(valid[:, None], code, 0)
    return out, pub, tie


def index_score_backward(iq, ik, cu, max_seqlen, ds, *, block_size=128, scale=1.0):
    """Exact amax subgradient: returns (dq [T,G,Di], dk [T,1,Di]) in float64."""
    q = np.asarray(iq, dtype=np.float64)
    k = np.asarray(ik, dtype=np.float64)[:, 0, :]
    ds = np.asarray(ds, dtype=np.float64)
    bounds = bounds_of(cu)
    total, groups, dim = q.shape
    nb = (max_seqlen + block_size - 1) // block_size
    dq = np.zeros_like(q)
    dk = np.zeros((total, dim))
    sign = 1.0 if scale > 0 else (-1.0 if scale < 0 else 0.0)
    for a, b in zip(bounds[:-1], bounds[1:]):
        length = b - a
        for blk in range(nb):
            lo, hi = blk * block_size, min((blk + 1) * block_size, length)
            if lo >= hi:
                continue
            dots = np.einsum("tgd,kd->tgk", q[a:b], k[a + lo : a + hi])
            pos = np.arange(length)[:, None]
            allowed = np.arange(lo, hi)[None, :] <= pos
            directed = np.where(allowed[:, None, :], sign * dots, -np.inf)
            best = directed.max(-1, keepdims=True)
            winners = (directed == best) & allowed[:, None, :]
            count = np.maximum(winners.sum(-1, keepdims=True), 1)
            weight = winners * (ds[a:b, :, blk][..., None] * scale / count)  # [S,G,n]
            weight = np.where(allowed.any(-1)[:, None, None], weight, 0.0)
            dq[a:b] += np.einsum("tgk,kd->tgd", weight, k[a + lo : a + hi])
            dk[a + lo : a + hi] += np.einsum("tgk,tgd->kd", weight, q[a:b])
    return dq, dk[:, None, :]


# --------------------------------------------------------------------------- stage 2


def _rank_order(ranked):
    """Block order of a descending selection along the last axis, as torch.topk ranks
    (triton/topk.py:44-45): NaN of either sign above +inf, then larger values first;
    equal values (and NaNs) in ascending block order."""
    nan = np.isnan(ranked)
    value = np.where(nan, 0.0, ranked)
    blocks = np.broadcast_to(np.arange(ranked.shape[-1]), ranked.shape)
    return np.lexsort((blocks, -value, ~nan), axis=-1)


def topk(scores, cu, *, block_size=128, topk_blocks=16, local_blocks=1):
    """Causal mask, +inf local boost, top-min(K, NB) in canonical order, -1 padding."""
    scores = np.asarray(scores, dtype=np.float32)
    bounds = bounds_of(cu)
    total, groups, nb = scores.shape
    result = np.full((total, groups, topk_blocks), -1, dtype=np.int32)
    if total == 0 or topk_blocks == 0:
        return result
    _, start = _token_positions(bounds)
    qb = (np.arange(total) - start) // block_size
    blocks = np.arange(nb)
    valid = blocks[None, :] <= qb[:, None]
    ranked = np.where(valid[:, None, :], scores.astype(np.float64), -np.inf)
    if local_blocks:
        local = valid & (blocks[None, :] > qb[:, None] - local_blocks)
        ranked = np.where(local[:, None, :], np.inf, ranked)
    count = min(topk_blocks, nb)
    order = _rank_order(ranked)[..., :count]
    values = np.take_along_axis(ranked, order, axis=-1)
    result[..., :count] = np.where(values == -np.inf, -1, order).astype(np.int32)
    return result


def topk_rows(score_rows, positions, *, block_size=128, topk_blocks=16, local_blocks=1):
    """``topk`` for a subset of rows: score_rows [n, G, NB] of tokens whose
    sequence-local positions are ``positions`` [n]. Same masking, boost, order."""
    scores = np.asarray(score_rows, dtype=np.float32)
    n, groups, nb = scores.shape
    result = np.full((n, groups, topk_blocks), -1, dtype=np.int32)
    if n == 0 or topk_blocks == 0:
        return result
    qb = np.asarray(positions, dtype=np.int64) // block_size
    blocks = np.arange(nb)
    valid = blocks[None, :] <= qb[:, None]
    ranked = np.where(valid[:, None, :], scores.astype(np.float64), -np.inf)
    if local_blocks:
        local = valid & (blocks[None, :] > qb[:, None] - local_blocks)
        ranked = np.where(local[:, None, :], np.inf, ranked)
    count = min(topk_blocks, nb)
    order = _rank_order(ranked)[..., :count]
    values = np.take_along_axis(ranked, order, axis=-1)
    result[..., :count] = np.where(values == -np.inf, -1, order).astype(np.int32)
    return result


def index_score_rows(iq, ik, cu, tokens, nb, *, block_size=128, scale=1.0):
    """``index_score`` (f64 scores, f32 scores) for the given query tokens only: [n, G, nb]."""
    q = np.asarray(iq, dtype=np.float64)
    k = np.asarray(ik, dtype=np.float64)[:, 0, :]
    bounds = bounds_of(cu)
    _, start = _token_positions(bounds)
    tokens = np.asarray(tokens, dtype=np.int64)
    groups = q.shape[1]
    out = np.full((len(tokens), groups, nb), -np.inf)
    pub = np.full((len(tokens), groups, nb), -np.inf, dtype=np.float32)
    sign = 1.0 if scale > 0 else (-1.0 if scale < 0 else 0.0)
    for i, t in enumerate(tokens):
        a = int(start[t])
        pos = int(t) - a
        dots = q[t] @ k[a : t + 1].T  # [G, pos + 1]
        for blk in range(pos // block_size + 1):
            lo, hi = blk * block_size, min((blk + 1) * block_size, pos + 1)
            with np.errstate(invalid="ignore"):
                best = (sign * dots[:, lo:hi]).max(-1)
                out[i, :, blk] = np.abs(scale) * best
                pub[i, :, blk] = public_score(best, scale)
    return out, pub


def _amax_weights(directed, allowed, ds_col, scale):
    """amax subgradient weights over the last axis: ds * scale split evenly over the exact
    maxima of the directed dots among the allowed keys (0 where none is allowed)."""
    directed = np.where(allowed, directed, -np.inf)
    best = directed.max(-1, keepdims=True)
    winners = (directed == best) & allowed
    count = np.maximum(winners.sum(-1, keepdims=True), 1)
    return winners * (ds_col[..., None] * scale / count)


def index_score_backward_rows(iq, ik, cu, ds, tokens, *, block_size=128, scale=1.0):
    """``index_score_backward``'s dq [n, G, Di] for the given query tokens only.
    ``ds`` is the full [T, G, NB] upstream gradient."""
    q = np.asarray(iq, dtype=np.float64)
    k = np.asarray(ik, dtype=np.float64)[:, 0, :]
    bounds = bounds_of(cu)
    _, start = _token_positions(bounds)
    tokens = np.asarray(tokens, dtype=np.int64)
    groups, dim = q.shape[1], q.shape[2]
    sign = 1.0 if scale > 0 else (-1.0 if scale < 0 else 0.0)
    dq = np.zeros((len(tokens), groups, dim))
    for i, t in enumerate(tokens):
        t = int(t)
        a = int(start[t])
        pos = t - a
        nblk = pos // block_size + 1
        width = nblk * block_size
        keys = a + np.arange(width)
        allowed = (np.arange(width) <= pos).reshape(nblk, block_size)
        kk = k[np.minimum(keys, t)]  # keys past t are masked
        dots = (sign * (q[t] @ kk.T)).reshape(groups, nblk, block_size)
        w = _amax_weights(dots, allowed[None], np.asarray(ds[t, :, :nblk], dtype=np.float64), scale)
        dq[i] = w.reshape(groups, width)[:, : pos + 1] @ k[a : t + 1]
    return dq


def index_score_backward_keys(iq, ik, cu, ds, keys, *, block_size=128, scale=1.0):
    """``index_score_backward``'s dk [n, Di] for the given key tokens only (every query
    token of the key's sequence at or after it, all groups). ``ds`` is the full
    [T, G, NB] upstream gradient."""
    q = np.asarray(iq, dtype=np.float64)
    k = np.asarray(ik, dtype=np.float64)[:, 0, :]
    bounds = bounds_of(cu)
    seq, _ = _token_positions(bounds)
    keys = np.asarray(keys, dtype=np.int64)
    dim = q.shape[2]
    sign = 1.0 if scale > 0 else (-1.0 if scale < 0 else 0.0)
    dk = np.zeros((len(keys), dim))
    blocks = {}
    for i, j in enumerate(keys):
        s = int(seq[int(j)])
        blocks.setdefault((s, (int(j) - bounds[s]) // block_size), []).append(i)
    for (s, blk), members in blocks.items():
        a, b = bounds[s], bounds[s + 1]
        k0 = a + blk * block_size
        k1 = min(k0 + block_size, b)
        kk = k[k0:k1]
        for t0 in range(k0, b, 4096):  # query tokens in slabs (memory)
            t1 = min(t0 + 4096, b)
            qs = q[t0:t1]  # [n, G, Di]
            allowed = (np.arange(k0, k1)[None, :] <= np.arange(t0, t1)[:, None])[:, None, :]
            n, groups = qs.shape[0], qs.shape[1]
            dots = sign * (qs.reshape(n * groups, dim) @ kk.T).reshape(n, groups, k1 - k0)
            w = _amax_weights(dots, allowed, np.asarray(ds[t0:t1, :, blk], dtype=np.float64), scale)
            for i in members:
                dk[i] += w[:, :, int(keys[i]) - k0].reshape(-1) @ qs.reshape(n * groups, dim)
    return dk[:, None, :]


# --------------------------------------------------------------------------- k2q CSR


def k2q_csr(indices, cu, *, block_size):
    """(row_ptr, query_indices, slot_indices, cu_block_lens) as int32 arrays."""
    ids = np.asarray(indices, dtype=np.int64)
    total, groups, slots = ids.shape
    bounds = bounds_of(cu)
    lengths = [b - a for a, b in zip(bounds[:-1], bounds[1:])]
    counts = [(n + block_size - 1) // block_size for n in lengths]
    cu_blocks = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    num_rows = int(cu_blocks[-1]) * groups
    capacity = total * groups * slots
    row_ptr = np.zeros(num_rows + 1, dtype=np.int32)
    query = np.full(capacity, -1, dtype=np.int32)
    slot = np.full(capacity, -1, dtype=np.int32)
    if capacity == 0:
        return row_ptr, query, slot, cu_blocks.astype(np.int32)
    seq, start = _token_positions(bounds)
    seq_blocks = np.asarray(counts, dtype=np.int64)[seq]
    qb = (np.arange(total) - start) // block_size
    valid = (ids >= 0) & (ids < seq_blocks[:, None, None]) & (ids <= qb[:, None, None])
    rows = (cu_blocks[seq][:, None, None] + ids) * groups + np.arange(groups)[None, :, None]
    flat_valid = valid.reshape(-1)
    flat_rows = rows.reshape(-1)[flat_valid]
    edges = np.nonzero(flat_valid)[0]
    order = np.argsort(flat_rows, kind="stable")
    edges = edges[order]
    n = edges.size
    query[:n] = edges // (groups * slots)
    slot[:n] = edges % slots
    row_ptr[1:] = np.cumsum(np.bincount(flat_rows, minlength=num_rows))
    return row_ptr, query, slot, cu_blocks.astype(np.int32)


# --------------------------------------------------------------------------- stage 3


def _selected_mask(ids_seq, length, block_size):
    """[S, S] bool: key j visible to query t (selected block and j <= t)."""
    pos = np.arange(length)
    key_block = pos // block_size
    sel = (key_block[None, :, None] == ids_seq[:, None, :]).any(-1)  # [S(t), S(j)]
    return sel & (pos[None, :] <= pos[:, None])


def sparse_attention(q, k, v, indices, cu, *, block_size=128, scale=None, dout=None):
    """Dense per-(sequence, group) FP64 attention.

    Returns (out, lse) and, when ``dout`` is given, also (dq, dk, dv).
    A key is visible when its block id appears among the query's selected ids
    and it is not after the query; rows without visible keys give out = 0,
    lse = -inf and zero gradients.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    ids = np.asarray(indices, dtype=np.int64)
    total, heads, dim = q.shape
    groups = k.shape[1]
    ratio = heads // groups
    scale = dim ** -0.5 if scale is None else float(scale)
    bounds = bounds_of(cu)
    out = np.zeros_like(q)
    lse = np.full((total, heads), -np.inf)
    grads = dout is not None
    if grads:
        do = np.asarray(dout, dtype=np.float64)
        dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    for a, b in zip(bounds[:-1], bounds[1:]):
        length = b - a
        if length == 0:
            continue
        for g in range(groups):
            hs = slice(g * ratio, (g + 1) * ratio)
            allowed = _selected_mask(ids[a:b, g], length, block_size)  # [S, S]
            has = allowed.any(-1)
            logits = np.einsum("trd,kd->trk", q[a:b, hs], k[a:b, g]) * scale
            masked = np.where(allowed[:, None, :], logits, -np.inf)
            m = np.where(has[:, None], masked.max(-1), 0.0)
            e = np.where(allowed[:, None, :], np.exp(masked - m[..., None]), 0.0)
            denom = e.sum(-1)
            safe = np.where(has[:, None], denom, 1.0)
            p = e / safe[..., None]
            out[a:b, hs] = np.einsum("trk,kd->trd", p, v[a:b, g])
            lse[a:b, hs] = np.where(has[:, None], m + np.log(safe), -np.inf)
            if grads:
                dov = do[a:b, hs]
                dp = np.einsum("trd,kd->trk", dov, v[a:b, g])
                delta = (p * dp).sum(-1, keepdims=True)
                dlogit = p * (dp - delta)
                dq[a:b, hs] = scale * np.einsum("trk,kd->trd", dlogit, k[a:b, g])
                dk[a:b, g] = scale * np.einsum("trk,trd->kd", dlogit, q[a:b, hs])
                dv[a:b, g] = np.einsum("trk,trd->kd", p, dov)
    if grads:
        return out, lse, dq, dk, dv
    return out, lse


def _row_keys(t, g, ids, start, block_size):
    """Sorted visible key tokens for query token t in group g (duplicates removed)."""
    pos = t - start
    qb = pos // block_size
    keys = []
    for blk in sorted(set(int(x) for x in ids[t, g] if 0 <= x <= qb)):
        lo = start + blk * block_size
        hi = min(lo + block_size, t + 1)
        keys.extend(range(lo, hi))
    return np.asarray(keys, dtype=np.int64)


def attention_rows(q, k, v, indices, cu, tokens, *, block_size=128, scale=None, dout=None):
    """Sparse FP64 attention for selected query tokens only.

    Returns dict with out [n,H,D], lse [n,H] and, with ``dout``, dq [n,H,D] and
    the per-row softmax-gradient center delta [n,H] = sum_j p_j dp_j.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    ids = np.asarray(indices)
    total, heads, dim = q.shape
    groups = k.shape[1]
    ratio = heads // groups
    scale = dim ** -0.5 if scale is None else float(scale)
    _, start = _token_positions(bounds_of(cu))
    tokens = np.asarray(tokens, dtype=np.int64)
    res = {"out": np.zeros((len(tokens), heads, dim)), "lse": np.full((len(tokens), heads), -np.inf)}
    if dout is not None:
        do = np.asarray(dout, dtype=np.float64)
        res["dq"] = np.zeros((len(tokens), heads, dim))
        res["delta"] = np.zeros((len(tokens), heads))
    for i, t in enumerate(tokens):
        for g in range(groups):
            keys = _row_keys(int(t), g, ids, int(start[t]), block_size)
            if keys.size == 0:
                continue
            hs = slice(g * ratio, (g + 1) * ratio)
            kk, vv = k[keys, g], v[keys, g]
            logits = q[t, hs] @ kk.T * scale  # [R, n]
            m = logits.max(-1, keepdims=True)
            e = np.exp(logits - m)
            den = e.sum(-1, keepdims=True)
            p = e / den
            res["out"][i, hs] = p @ vv
            res["lse"][i, hs] = (m + np.log(den))[:, 0]
            if dout is not None:
                dp = do[t, hs] @ vv.T
                delta = (p * dp).sum(-1, keepdims=True)
                res["dq"][i, hs] = scale * (p * (dp - delta)) @ kk
                res["delta"][i, hs] = delta[:, 0]
    return res


def _rows_lse_delta(q, k, v, do, ids, bounds, tokens, g, ratio, scale, block_size):
    """Per (token, head) of group g over the given (sorted, distinct) tokens: lse [n, R]
    and the softmax derivative centre delta = sum_j p_j dp_j [n, R], the values
    attention_rows computes. Evaluated block by block (each selected key block is one
    product over all the rows that chose it) with an online FP64 merge of
    (max, sum exp, sum exp * dp) per row."""
    hs = slice(g * ratio, (g + 1) * ratio)
    tokens = np.asarray(tokens, dtype=np.int64)
    n = len(tokens)
    m = np.full((n, ratio), -np.inf)
    l = np.zeros((n, ratio))
    u = np.zeros((n, ratio))
    if n:
        seq, start = _token_positions(bounds)
        ends = np.asarray(bounds[1:], dtype=np.int64)[seq[tokens]]
        sel = np.asarray(ids[tokens, g, :], dtype=np.int64)  # [n, K]
        qb = (tokens - start[tokens]) // block_size
        valid = (sel >= 0) & (sel <= qb[:, None])
        for slot in range(1, sel.shape[1]):  # a block selected twice counts once
            valid[:, slot] &= ~(sel[:, :slot] == sel[:, slot : slot + 1]).any(-1)
        rows, slots = np.nonzero(valid)
        kb = start[tokens[rows]] + sel[rows, slots] * block_size  # first key of the block
        order = np.argsort(kb, kind="stable")
        rows, kb = rows[order], kb[order]
        cuts = np.flatnonzero(np.diff(kb)) + 1
        for seg_rows, seg_kb in zip(np.split(rows, cuts), np.split(kb, cuts)):
            k0 = int(seg_kb[0])
            k1 = min(k0 + block_size, int(ends[seg_rows[0]]))
            t = tokens[seg_rows]
            nr, nk = len(t), k1 - k0
            x = (q[t, hs].reshape(nr * ratio, -1) @ k[k0:k1, g].T).reshape(nr, ratio, nk) * scale
            vis = (np.arange(k0, k1)[None, :] <= t[:, None])[:, None, :]
            x = np.where(vis, x, -np.inf)
            mb = x.max(-1)  # every such row sees key k0
            e = np.where(vis, np.exp(x - mb[..., None]), 0.0)
            dp = (do[t, hs].reshape(nr * ratio, -1) @ v[k0:k1, g].T).reshape(nr, ratio, nk)
            lb, ub = e.sum(-1), (e * dp).sum(-1)
            mo = m[seg_rows]
            mn = np.maximum(mo, mb)
            wo, wb = np.exp(mo - mn), np.exp(mb - mn)
            l[seg_rows] = l[seg_rows] * wo + lb * wb
            u[seg_rows] = u[seg_rows] * wo + ub * wb
            m[seg_rows] = mn
    has = l > 0
    lse = np.where(has, m + np.log(np.where(has, l, 1.0)), -np.inf)
    delta = np.where(has, u / np.where(has, l, 1.0), 0.0)
    return lse, delta


def attention_kv_rows(q, k, v, indices, cu, dout, keys, *, block_size=128, scale=None):
    """Sparse FP64 dK/dV for selected key tokens (all groups): returns (dk, dv) [n,G,D].

    Key j of block b (its sequence's numbering) receives, from every query token t >= j
    of its sequence whose group-g selection holds b, and each head h of that group:
    dv += p dO[t,h], dk += scale p (dp - delta) q[t,h], with p = exp(scale q.k_j - lse),
    dp = dO[t,h].v_j and the row's lse / delta (tests/reference_fp64.py:48-85; the
    gradient of sparse_attention restricted to the sampled keys)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    do = np.asarray(dout, dtype=np.float64)
    ids = np.asarray(indices)
    total, heads, dim = q.shape
    groups = k.shape[1]
    ratio = heads // groups
    scale = dim ** -0.5 if scale is None else float(scale)
    bounds = bounds_of(cu)
    seq, start = _token_positions(bounds)
    keys = np.asarray(keys, dtype=np.int64)
    dk = np.zeros((len(keys), groups, dim))
    dv = np.zeros((len(keys), groups, dim))
    for g in range(groups):
        hs = slice(g * ratio, (g + 1) * ratio)
        hits = []
        for j in keys:
            j = int(j)
            s = int(seq[j])
            a, b = bounds[s], bounds[s + 1]
            blk = (j - a) // block_size
            hits.append(np.nonzero((ids[j:b, g, :] == blk).any(-1))[0] + j)  # tokens that selected j's block
        needed = np.unique(np.concatenate(hits + [np.zeros(0, dtype=np.int64)]))
        lse_n, delta_n = _rows_lse_delta(q, k, v, do, ids, bounds, needed, g, ratio, scale, block_size)
        for i, j in enumerate(keys):
            t = hits[i]
            if t.size == 0:
                continue
            r = np.searchsorted(needed, t)
            qh, dh = q[t, hs], do[t, hs]  # [n, R, D]
            p = np.exp(qh @ k[int(j), g] * scale - lse_n[r])  # [n, R]
            dp = dh @ v[int(j), g]
            dk[i, g] = scale * np.einsum("nr,nrd->d", p * (dp - delta_n[r]), qh)
            dv[i, g] = np.einsum("nr,nrd->d", p, dh)
    return dk, dv


# ---------------------------------------------------------------------------- indexer KL
#
# Not implemented upstream. The definition restated here is the reference's
# training-flow description (docs/msa_training_flow.md:92-138, docs/implementation_plan.md:66-69):
# over the causal tokens of each (token, group)'s selected blocks, the student is
# softmax of the index token logits z_j = index_scale * iq[t,g] . ik[j] (token
# logits, not block maxima, and no local +inf boost), the teacher is the mean over
# the group's query heads of softmax(a_hj), a_hj = scale * q[t,h] . k[j,g] (the
# main attention's probabilities, detached), and the loss is
# KL(teacher || student) = sum_j T_j (log T_j - log S_j), averaged over all
# (token, group) pairs (a pair without visible keys contributes 0). Only index_q
# and index_k receive gradients: dLoss/dz_j = (S_j - T_j) / (T * G).


def _kl_row(iq_row, ik_keys, q_rows, k_keys, index_scale, scale):
    """(KL, dz [n]) of one (token, group) over its visible keys, in float64."""
    z = index_scale * (ik_keys @ iq_row)
    zs = z - z.max()
    log_s = zs - np.log(np.exp(zs).sum())
    a = scale * (q_rows @ k_keys.T)  # [R, n]
    a = a - a.max(-1, keepdims=True)
    p = np.exp(a)
    p /= p.sum(-1, keepdims=True)
    t = p.mean(0)
    with np.errstate(divide="ignore"):
        log_t = np.where(t > 0, np.log(np.where(t > 0, t, 1.0)), 0.0)
    kl = float(np.sum(np.where(t > 0, t * (log_t - log_s), 0.0)))
    return kl, np.exp(log_s) - t


def indexer_kl(iq, ik, q, k, indices, cu, *, block_size=128, index_scale=1.0, scale=None):
    """Loss, per-row KL [T,G] and the loss gradients d_iq [T,G,Di], d_ik [T,1,Di]."""
    iq = np.asarray(iq, dtype=np.float64)
    ik = np.asarray(ik, dtype=np.float64)
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    ids = np.asarray(indices)
    total, groups, _ = iq.shape
    ratio = q.shape[1] // groups
    scale = q.shape[2] ** -0.5 if scale is None else float(scale)
    _, start = _token_positions(bounds_of(cu))
    row_kl = np.zeros((total, groups))
    d_iq = np.zeros_like(iq)
    d_ik = np.zeros_like(ik)
    rows = max(total * groups, 1)
    for t in range(total):
        for g in range(groups):
            keys = _row_keys(t, g, ids, int(start[t]), block_size)
            if keys.size == 0:
                continue
            hs = slice(g * ratio, (g + 1) * ratio)
            kl, dz = _kl_row(iq[t, g], ik[keys, 0], q[t, hs], k[keys, g], index_scale, scale)
            row_kl[t, g] = kl
            dz = dz * (index_scale / rows)
            d_iq[t, g] = dz @ ik[keys, 0]
            d_ik[keys, 0] += dz[:, None] * iq[t, g][None, :]
    return {"loss": float(row_kl.sum() / rows), "row_kl": row_kl, "d_iq": d_iq, "d_ik": d_ik}


def indexer_kl_rows(iq, ik, q, k, indices, cu, tokens, *, block_size=128, index_scale=1.0, scale=None):
    """``indexer_kl``'s row KL [n,G] and d_iq [n,G,Di] for the given query tokens only."""
    iq = np.asarray(iq, dtype=np.float64)
    ik = np.asarray(ik, dtype=np.float64)
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    ids = np.asarray(indices)
    total, groups, dim_i = iq.shape
    ratio = q.shape[1] // groups
    scale = q.shape[2] ** -0.5 if scale is None else float(scale)
    _, start = _token_positions(bounds_of(cu))
    tokens = np.asarray(tokens, dtype=np.int64)
    row_kl = np.zeros((len(tokens), groups))
    d_iq = np.zeros((len(tokens), groups, dim_i))
    rows = max(total * groups, 1)
    for i, t in enumerate(tokens):
        t = int(t)
        for g in range(groups):
            keys = _row_keys(t, g, ids, int(start[t]), block_size)
            if keys.size == 0:
                continue
            hs = slice(g * ratio, (g + 1) * ratio)
            kl, dz = _kl_row(iq[t, g], ik[keys, 0], q[t, hs], k[keys, g], index_scale, scale)
            row_kl[i, g] = kl
            d_iq[i, g] = (dz * (index_scale / rows)) @ ik[keys, 0]
    return {"row_kl": row_kl, "d_iq": d_iq}


def indexer_kl_key_rows(iq, ik, q, k, indices, cu, keys, *, block_size=128, index_scale=1.0, scale=None):
    """``indexer_kl``'s d_ik [n,Di] for the given key tokens only (all rows that see them)."""
    iq = np.asarray(iq, dtype=np.float64)
    ik = np.asarray(ik, dtype=np.float64)
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    ids = np.asarray(indices)
    total, groups, dim_i = iq.shape
    ratio = q.shape[1] // groups
    scale = q.shape[2] ** -0.5 if scale is None else float(scale)
    bounds = bounds_of(cu)
    seq, start = _token_positions(bounds)
    rows = max(total * groups, 1)
    keys = np.asarray(keys, dtype=np.int64)
    out = np.zeros((len(keys), dim_i))
    for i, j in enumerate(keys):
        j = int(j)
        s = int(seq[j])
        b = bounds[s + 1]
        blk = (j - bounds[s]) // block_size
        for g in range(groups):
            hs = slice(g * ratio, (g + 1) * ratio)
            for t in np.nonzero((ids[j:b, g, :] == blk).any(-1))[0] + j:
                t = int(t)
                row_keys = _row_keys(t, g, ids, int(start[t]), block_size)
                _, dz = _kl_row(iq[t, g], ik[row_keys, 0], q[t, hs], k[row_keys, g], index_scale, scale)
                out[i] += dz[np.searchsorted(row_keys, j)] * (index_scale / rows) * iq[t, g]
    return out
