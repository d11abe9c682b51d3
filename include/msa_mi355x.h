/*
 * C ABI of the MI355X (gfx950) MiniMax-M3 sparse-attention kernels.
 *
 * Every entry point takes raw device pointers, int64 sizes, scalars and a
 * hipStream_t passed as void*. Kernels are enqueued on that stream and the call
 * returns without synchronising. No entry point allocates device memory: all
 * outputs and workspaces are owned by the caller (sizes from the *_bytes /
 * *_elems queries). Return value: 0 on success, 1 invalid argument,
 * 2 unsupported configuration, 3 HIP launch failure.
 *
 * Layouts are the reference's TND layout: q [T,Hq,D], k/v [T,G,D],
 * index_q [T,G,Di], index_k [T,1,Di], scores [T,G,NB] fp32, indices [T,G,K]
 * int32, cu_seqlens [num_seqs+1] int32, all contiguous. Query heads
 * [g*Hq/G, (g+1)*Hq/G) belong to KV group g. Block ids are sequence-local.
 * dtype codes: 0 = fp32, 1 = fp16, 2 = bf16.
 */
#ifndef MSA_MI355X_H_
#define MSA_MI355X_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Stage 2: causal top-k with forced local blocks.
 * Replaces triton/topk.py:11-47 (m3_topk; eager twin eager/ops.py:94-129).
 * indices [T,G,topk_blocks] int32, left-aligned, -1 padded; ties in
 * descending-value order are emitted by ascending block id; NaN scores (either
 * sign) rank above +inf, as torch.topk ranks them. */
int msa_topk(const float* scores, const int32_t* cu_seqlens, int64_t num_seqs,
             int64_t total_tokens, int64_t groups, int64_t num_blocks, int64_t block_size,
             int64_t topk_blocks, int64_t local_blocks, int32_t* indices, void* stream);

/* k2q CSR workspace: number of int32 tile counters, G * sum_s nb_s (nb_s + 1) / 2,
 * from the host copy of cu_block_lens. Host-only helper (no device access). */
int64_t msa_k2q_counter_elems(int64_t num_seqs, const int32_t* host_cu_block_lens, int64_t groups);

/* Block->query CSR. Replaces triton/k2q.py:39-128 (build_k2q_csr; K2QCSR :20-36).
 * cu_block_lens [num_seqs+1] int32 and tri_prefix [num_seqs+1] int64
 * (tri_prefix[s] = G * sum_{s'<s} nb(nb+1)/2) are device copies of host metadata.
 * workspace: int32 [counter_elems + total_blocks*groups].
 * Outputs: row_ptr [total_blocks*groups+1], query_indices/slot_indices
 * [T*G*K] (tail = -1), edges ordered by (query, slot) inside each row. */
int msa_k2q_build(const int32_t* indices, const int32_t* cu_seqlens, const int32_t* cu_block_lens,
                  const int64_t* tri_prefix, int64_t num_seqs, int64_t total_tokens, int64_t groups,
                  int64_t topk_slots, int64_t block_size, int64_t total_blocks,
                  int64_t counter_elems, int32_t* row_ptr, int32_t* query_indices,
                  int32_t* slot_indices, int32_t* workspace, void* stream);

/* Sub-block form of a selection, for blocks larger than the MFMA kernels' 128-key
 * tiles. With f dividing B, sub-block f b + i (size B / f) holds keys
 * [b B + i B / f, b B + (i + 1) B / f): the f sub-blocks of id b hold exactly the keys
 * the reference's kernels visit for block b (triton/sparse_attention.py:35-84 forward,
 * :87-198 and :223-295 backward), and a sub-block that starts after the query is
 * skipped by the same id <= query-block rule. out [rows, slots * factor]:
 * out[r, s f + i] = f in[r, s] + i, or -1 where in[r, s] < 0 or f in[r, s] + i would
 * pass INT32_MAX. The sub-block selection with its CSR (msa_k2q_build at
 * block_size / factor) and block_size / factor gives the attention of the original
 * selection. No counterpart in the reference (its kernels take any block size). */
int msa_split_block_indices(const int32_t* indices, int64_t rows, int64_t slots, int32_t factor, int32_t* out,
                            void* stream);

/* msa_k2q_build without the workspace argument; allocates nothing. No counterpart in
 * the reference: for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Its workspace is a
 * fixed device array inside the library, one per GPU, held until the process ends:
 * MSA_K2Q_NOALLOC_MAX_ELEMS int32 (16 MiB). Returns 2 (unsupported) without launching
 * anything when counter_elems + total_blocks * groups exceeds that (for one sequence
 * of nb blocks, G * nb (nb + 3) / 2 entries: up to 1022 blocks at G = 8, i.e. 130,816
 * tokens at block 128). All calls on one GPU share the array: calls that overlap in
 * time on one GPU (different streams or threads) race and must be serialised by the
 * caller. The stream must belong to the current device. Outputs and semantics are
 * those of msa_k2q_build. */
#define MSA_K2Q_NOALLOC_MAX_ELEMS (1 << 22)
int msa_k2q_build_noalloc(const int32_t* indices, const int32_t* cu_seqlens, const int32_t* cu_block_lens,
                          const int64_t* tri_prefix, int64_t num_seqs, int64_t total_tokens, int64_t groups,
                          int64_t topk_slots, int64_t block_size, int64_t total_blocks,
                          int64_t counter_elems, int32_t* row_ptr, int32_t* query_indices,
                          int32_t* slot_indices, void* stream);

/* Stage 1 forward workspace in bytes: the squared norm of every index key (fp32 [T])
 * and one bit per (token, group, block) marking the pairs whose winner the bf16 MFMA
 * pass could not certify. 0 for invalid sizes. */
int64_t msa_score_fwd_workspace_bytes(int64_t total_tokens, int64_t groups, int64_t num_blocks);

/* Stage 1 forward: per-group causal block maxima of scale * (index_q . index_k).
 * Replaces triton/index_score.py:93-136 (_index_score_forward) and the launch at
 * :237-265. scores = the reference's FP32 form of the exact winning dot x (:121-127):
 * fl32(fl32(hi s) + fl32(lo s)) with hi = fl32(x), lo = fl32(x - hi), s = fl32(|scale|)
 * (fl32(scale x) for |scale| in {0, 1}); -inf for blocks with no
 * causal key. tie_info (nullable, int32 [T,G,NB]): winner offset + 1 for a
 * unique exact maximum, -count for exact ties, 0 for invalid blocks
 * (same encoding as index_score.py:128-136). workspace: at least
 * msa_score_fwd_workspace_bytes(total_tokens, groups, num_blocks) bytes, 4-byte
 * aligned. */
int msa_score_fwd(const void* index_q, const void* index_k, int32_t dtype,
                  const int32_t* cu_seqlens, int64_t num_seqs, int64_t total_tokens,
                  int64_t groups, int64_t index_dim, int64_t num_blocks, int64_t block_size,
                  double scale, float* scores, int32_t* tie_info, void* workspace, void* stream);

/* Stage 1 forward fused with stage 2: the scores of msa_score_fwd and, from them,
 * the causal top-k selection of msa_topk (int32 [T,G,K], same semantics and tie
 * order). No counterpart entry point in the reference, which runs
 * triton/index_score.py:298-357 and triton/topk.py:11-47 as two operators; this
 * is the score -> top-k fusion the reference's survey lists as follow-on work,
 * as one call: the selection is a second launch on the same stream (selecting
 * inside the score kernel's tiles measured slower). workspace as for msa_score_fwd. */
int msa_index_score_topk(const void* index_q, const void* index_k, int32_t dtype,
                         const int32_t* cu_seqlens, int64_t num_seqs, int64_t total_tokens,
                         int64_t groups, int64_t index_dim, int64_t num_blocks, int64_t block_size,
                         double scale, int64_t topk_blocks, int64_t local_blocks, float* scores,
                         int32_t* tie_info, int32_t* indices, void* workspace, void* stream);

/* Score backward workspace in bytes (block-major tie/grad copies and the FP64
 * per-segment dk sums). */
int64_t msa_score_bwd_workspace_bytes(int64_t total_tokens, int64_t groups, int64_t num_blocks,
                                      int64_t index_dim, int64_t block_size, int64_t total_blocks);

/* Stage 1 backward (amax subgradient: unique winner gets ds*scale, exact ties
 * split it evenly). Replaces index_score.py:139-232 (_index_score_backward_q,
 * _index_score_backward_k_group, _index_score_reduce_k; launches :268-295).
 * grad_q [T,G,Di] / grad_k [T,1,Di] in the input dtype, either nullable.
 * Deterministic: no floating-point atomics. */
int msa_score_bwd(const void* index_q, const void* index_k, int32_t dtype,
                  const int32_t* cu_seqlens, const int32_t* cu_block_lens, const int32_t* tie_info,
                  const float* grad_scores, int64_t num_seqs, int64_t total_tokens, int64_t groups,
                  int64_t index_dim, int64_t num_blocks, int64_t block_size, int64_t total_blocks,
                  double scale, void* grad_q, void* grad_k, void* workspace, void* stream);

/* Stage 3 forward workspace in bytes; 0 means this configuration runs the VALU
 * kernels, which need neither the CSR nor a workspace. Non-zero (the KV-major MFMA
 * kernels) for bf16 and fp16 inputs with head ratio <= 512, head dim 8..256 a
 * multiple of 8 and blocks of at most 128 keys. */
int64_t msa_attn_fwd_workspace_bytes(int32_t dtype, int64_t total_tokens, int64_t q_heads,
                                     int64_t kv_groups, int64_t head_dim, int64_t topk_slots,
                                     int64_t total_blocks, int64_t block_size);

/* Stage 3 forward: sparse GQA attention over the selected blocks.
 * Replaces triton/sparse_attention.py:35-84 (_forward_kernel; launch :336-359).
 * out [T,Hq,D] in the input dtype; lse [T,Hq] fp32 (natural log, -inf for rows
 * without keys, whose output is 0). Slots with id < 0 or id > qb(t) are ignored;
 * keys after the query inside its own block are masked.
 * The bf16 path is KV-major: it consumes the k2q CSR of `indices`
 * (msa_k2q_build: cu_block_lens, row_ptr, query_indices, slot_indices) and a
 * workspace of msa_attn_fwd_workspace_bytes(...) bytes; these may be NULL / 0
 * when that query returns 0.
 * row_state (nullable): private fp64 [T,Hq,4] consumed by msa_attn_bwd; slots 0
 * and 1 receive the full-precision lse in the path's own convention and its
 * normalisation (the reference keeps (max, denominator), sparse_attention.py:83-84);
 * treat it as opaque. out_f32 (nullable): fp32 [T,Hq,D], the output before its
 * rounding to the input dtype; handed to msa_attn_bwd it replaces the backward's
 * per-slot statistics pass (no reference counterpart: the reference recomputes). */
int msa_attn_fwd(const void* q, const void* k, const void* v, int32_t dtype, const int32_t* indices,
                 const int32_t* cu_seqlens, int64_t num_seqs, int64_t total_tokens,
                 int64_t q_heads, int64_t kv_groups, int64_t head_dim, int64_t topk_slots,
                 int64_t block_size, double scale, const int32_t* cu_block_lens,
                 int64_t total_blocks, const int32_t* row_ptr, const int32_t* query_indices,
                 const int32_t* slot_indices, void* workspace, int64_t workspace_bytes, void* out,
                 float* lse, double* row_state, float* out_f32, void* stream);

/* Stage 3 backward workspace in bytes; 0 means this configuration runs the VALU
 * kernels, which need no workspace. */
int64_t msa_attn_bwd_workspace_bytes(int32_t dtype, int64_t total_tokens, int64_t q_heads,
                                     int64_t kv_groups, int64_t head_dim, int64_t topk_slots,
                                     int64_t total_blocks, int64_t block_size);

/* Stage 3 backward: dQ, dK, dV (each nullable; all NULL is a no-op) of the
 * attention computed by msa_attn_fwd with the same row_state. Replaces the
 * autograd backward of triton/sparse_attention.py:361-394 (_backward_kernel,
 * :87-198, with the dK/dV pass _backward_kv_kernel, :223-295, over
 * build_k2q_csr). Without out_f32 the softmax derivative is centred as in the
 * reference (:119-158): delta = sum p (dp - c) / mass from the same p and dp as
 * dS, one extra pass over every (row, slot). With out_f32 (the forward's, for the
 * same row_state) the bf16 path takes delta = out_f32 . dO in fp64 and the
 * forward's exact mass instead, and skips that pass; other paths ignore it.
 * The bf16 path is KV-major and needs the k2q CSR (cu_block_lens, row_ptr,
 * query_indices, slot_indices) and msa_attn_bwd_workspace_bytes(...) bytes of
 * workspace for every gradient set; the VALU path needs the CSR only when
 * grad_k or grad_v is requested. row_state slots 1..3 are (re)written.
 * Deterministic: no floating-point atomics. */
int msa_attn_bwd(const void* q, const void* k, const void* v, int32_t dtype, const void* out,
                 const void* grad_out, double* row_state, const float* out_f32, const int32_t* indices,
                 const int32_t* cu_seqlens, int64_t num_seqs, int64_t total_tokens,
                 int64_t q_heads, int64_t kv_groups, int64_t head_dim, int64_t topk_slots,
                 int64_t block_size, double scale, const int32_t* cu_block_lens,
                 int64_t total_blocks, const int32_t* row_ptr, const int32_t* query_indices,
                 const int32_t* slot_indices, void* grad_q, void* grad_k, void* grad_v,
                 void* workspace, int64_t workspace_bytes, void* stream);

/* Indexer KL (bf16 or fp16; index_q, index_k, q and k all of `dtype`): workspace
 * bytes; 0 means the configuration is not supported (other dtypes, head or index dim
 * not 32 / 64 / 128, more than 8 query heads per group, block above 128). */
int64_t msa_indexer_kl_workspace_bytes(int32_t dtype, int64_t total_tokens, int64_t q_heads,
                                       int64_t kv_groups, int64_t head_dim, int64_t index_dim,
                                       int64_t topk_slots, int64_t total_blocks, int64_t block_size);

/* Indexer KL: the training branch that consumes the selection. No reference
 * kernel: the reference describes it (docs/msa_training_flow.md:92-138) and leaves
 * it unimplemented (docs/implementation_plan.md:66-69). Over the causal tokens of
 * each (token, group)'s selected blocks, KL(teacher || student) with student =
 * softmax of index_scale * index_q . index_k and teacher = the mean over the
 * group's query heads of softmax(scale * q . k); loss [1] = mean over the T x G
 * (token, group) pairs (pairs without visible keys count as 0). row_kl [T,G]
 * (nullable) receives the per-pair KL; grad_index_q [T,G,Di] and grad_index_k
 * [T,1,Di] (fp32, each nullable) the gradients of loss. teacher_lse (nullable):
 * msa_attn_fwd's lse [T,Hq] for the same q, k, indices and scale; when given, the
 * teacher's normalisers are taken from it instead of being recomputed. Uses the
 * k2q CSR of `indices` (msa_k2q_build) and msa_indexer_kl_workspace_bytes(...)
 * bytes. Deterministic: no floating-point atomics. */
int msa_indexer_kl(const void* index_q, const void* index_k, const void* q, const void* k, int32_t dtype,
                   const int32_t* indices, const int32_t* cu_seqlens, int64_t num_seqs,
                   int64_t total_tokens, int64_t q_heads, int64_t kv_groups, int64_t head_dim,
                   int64_t index_dim, int64_t topk_slots, int64_t block_size, double index_scale,
                   double scale, const int32_t* cu_block_lens, int64_t total_blocks,
                   const int32_t* row_ptr, const int32_t* query_indices, const int32_t* slot_indices,
                   const float* teacher_lse, float* loss, float* row_kl, float* grad_index_q,
                   float* grad_index_k, void* workspace, int64_t workspace_bytes, void* stream);

/* Testing hook; no counterpart in the reference. Overrides the byte budgets that size
 * the query-token chunks of the KV-major bf16 passes: msa_attn_fwd (default 2 GiB of
 * per-(token, head, slot) partial records per chunk), msa_attn_bwd (3 GiB) and
 * msa_indexer_kl (1 GiB); a value <= 0 restores that default. A chunk holds at least
 * 64 tokens. Chunking changes only how sums are split into per-chunk partial sums,
 * not what is computed; tests use it to drive small cases through many chunks.
 * Process-wide: set it only while no other thread queries workspace sizes or calls
 * those entry points, and query the workspace sizes again after a change. Returns 0. */
int msa_set_chunk_budgets(int64_t fwd_bytes, int64_t bwd_bytes, int64_t kl_bytes);

/* Testing hook; no counterpart in the reference. The KV-major bf16 passes of
 * msa_attn_fwd, msa_attn_bwd and msa_indexer_kl launch their work items largest first
 * (enabled != 0, the default); enabled == 0 launches them in row order instead. Every
 * work item writes only its own outputs, so results are bitwise the same either way;
 * tests use it to check exactly that. Process-wide, like msa_set_chunk_budgets.
 * Returns 0. */
int msa_set_item_order(int enabled);

/* Profiling hook; no counterpart in the reference (bench.py reports its figures).
 * msa_profile_begin arms per-launch timing: until msa_profile_end, every kernel launch
 * of msa_attn_fwd and msa_attn_bwd is bracketed by two HIP events recorded on the
 * call's stream (at most 16384 launches). msa_profile_end waits for those events and
 * writes, for each kernel kind k < kinds, the summed duration in ms (ms[k]) and the
 * number of launches (launches[k]); either array may be NULL. Kinds, in order:
 * 0 forward work plan (kv_chunk_bounds + kv_item_scan), 1 attn_fwd_partial_kernel,
 * 2 attn_fwd_combine, 3 backward work plans, 4 kv_bwd_center, 5 kv_bwd_stats_kernel,
 * 6 kv_bwd_stats_combine, 7 kv_bwd_main_kernel, 8 kv_bwd_accumulate,
 * 9 kv_bwd_dq_combine. Returns the number of kinds the library defines (10), or -1
 * if an event could not be read. Armed, the event records add a short gap between
 * kernels. Process-wide; not for concurrent use from several threads. */
int msa_profile_begin(void);
int64_t msa_profile_end(double* ms, int64_t* launches, int64_t kinds);

#ifdef __cplusplus
}
#endif

#endif /* MSA_MI355X_H_ */
