"""MI355X-native MiniMax-M3 three-stage sparse attention (drop-in for ``msa_triton.triton``).

The public operators keep the reference facade (triton/__init__.py:4-29): the
implementation module is imported on first call, so importing the package does
not load the native library.

    m3_index_score(index_q, index_k, cu_seqlens, max_seqlen, *, block_size=128, scale=1.0)
    m3_topk(scores, cu_seqlens, *, block_size=128, topk_blocks=16, local_blocks=1)
    m3_sparse_attention(q, k, v, indices, cu_seqlens, max_seqlen, *, block_size=128,
                        scale=None, return_lse=False)

All three run as hand-written gfx950 HIP kernels behind the C ABI declared in
``include/msa_mi355x.h``; there is no CPU or eager fallback.

    m3_index_score_topk(index_q, index_k, cu_seqlens, max_seqlen, *, block_size=128, scale=1.0,
                        topk_blocks=16, local_blocks=1) -> (scores, indices)

is the first two stages in one call (score and selection kernels back to back);

    m3_indexer_kl(index_q, index_k, q, k, indices, cu_seqlens, max_seqlen, *, block_size=128,
                  index_scale=1.0, scale=None, return_rows=False) -> loss

is the indexer's KL training loss over the selected tokens (teacher: the detached
attention probabilities; student: the index token logits);

    prepare_sequences(cu_seqlens, *, block_size=128) -> PackedSequences

validates ``cu_seqlens`` once and returns immutable metadata with device copies;
passed in place of ``cu_seqlens`` to any operator (and to ``build_k2q_csr``), it
removes the operators' host reads of ``cu_seqlens``, so a layer's forward and
backward run without host synchronisation and can be captured in a HIP graph.
"""

from .layout import PackedSequences


def m3_index_score(index_q, index_k, cu_seqlens, max_seqlen, *, block_size=128, scale=1.0):
    from .index_score import m3_index_score as implementation

    return implementation(index_q, index_k, cu_seqlens, max_seqlen, block_size=block_size, scale=scale)


def m3_topk(scores, cu_seqlens, *, block_size=128, topk_blocks=16, local_blocks=1):
    from .topk import m3_topk as implementation

    return implementation(
        scores, cu_seqlens, block_size=block_size, topk_blocks=topk_blocks, local_blocks=local_blocks
    )


def m3_sparse_attention(
    q, k, v, indices, cu_seqlens, max_seqlen, *, block_size=128, scale=None, return_lse=False
):
    from .sparse_attention import m3_sparse_attention as implementation

    return implementation(
        q, k, v, indices, cu_seqlens, max_seqlen,
        block_size=block_size, scale=scale, return_lse=return_lse,
    )


def m3_index_score_topk(index_q, index_k, cu_seqlens, max_seqlen, *, block_size=128, scale=1.0, topk_blocks=16,
                        local_blocks=1):
    from .index_score import m3_index_score_topk as implementation

    return implementation(index_q, index_k, cu_seqlens, max_seqlen, block_size=block_size, scale=scale,
                          topk_blocks=topk_blocks, local_blocks=local_blocks)


def m3_indexer_kl(index_q, index_k, q, k, indices, cu_seqlens, max_seqlen, *, block_size=128, index_scale=1.0,
                  scale=None, return_rows=False, teacher_lse=None):
    from .indexer_kl import m3_indexer_kl as implementation

    return implementation(index_q, index_k, q, k, indices, cu_seqlens, max_seqlen, block_size=block_size,
                          index_scale=index_scale, scale=scale, return_rows=return_rows, teacher_lse=teacher_lse)


def prepare_sequences(cu_seqlens, *, block_size=128):
    from .layout import prepare_sequences as implementation

    return implementation(cu_seqlens, block_size=block_size)


__all__ = ["m3_index_score", "m3_topk", "m3_sparse_attention", "m3_index_score_topk", "m3_indexer_kl",
           "prepare_sequences", "PackedSequences"]
