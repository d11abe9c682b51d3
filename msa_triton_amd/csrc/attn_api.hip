// C ABI for stage 3 (sparse GQA attention forward / backward).
// bf16 and fp16 inputs whose shape fits the MFMA templates run the KV-major MFMA kernels
// (attn_kv_fwd.hip, attn_kv_bwd.hip); fp32 inputs and other shapes run the VALU kernels
// (attn_scalar.hip).
#include "attn_mfma.hpp"
#include "common.hpp"

namespace msa {

template <int DT>
int attn_fwd_valu_dispatch(const void*, const void*, const void*, const int32_t*, const int32_t*, int, int64_t, int,
                           int, int, int, int, double, void*, float*, double*, float*, hipStream_t);
template <int DT>
int attn_dq_valu_dispatch(const void*, const void*, const void*, const void*, const void*, double*, const int32_t*,
                          const int32_t*, int, int64_t, int, int, int, int, int, double, void*, hipStream_t);
template <int DT>
int attn_dkdv_valu_dispatch(const void*, const void*, const void*, const void*, const double*, const int32_t*,
                            const int32_t*, const int32_t*, const int32_t*, int, int64_t, int, int, int, int, double,
                            void*, void*, hipStream_t);

// Input types the MFMA kernels take (exact products in fp32 for both).
static bool mfma_dtype(int32_t dtype) { return dtype == kBF16 || dtype == kF16; }

static bool valid_common(int64_t num_seqs, int64_t T, int64_t Hq, int64_t G, int64_t D, int64_t B) {
  return num_seqs > 0 && T >= 0 && Hq > 0 && G > 0 && Hq % G == 0 && D > 0 && B > 0;
}

}  // namespace msa

using namespace msa;

extern "C" int64_t msa_attn_fwd_workspace_bytes(int32_t dtype, int64_t total_tokens, int64_t q_heads,
                                                int64_t kv_groups, int64_t head_dim, int64_t topk_slots,
                                                int64_t total_blocks, int64_t block_size) {
  if (q_heads <= 0 || kv_groups <= 0 || q_heads % kv_groups || total_tokens <= 0) return 0;
  if (!mfma_dtype(dtype) || !attn_mfma_supported(q_heads / kv_groups, head_dim, block_size)) return 0;
  return attn_fwd_kv_workspace_bytes(total_tokens, q_heads, kv_groups, head_dim, topk_slots, total_blocks);
}

extern "C" int msa_attn_fwd(const void* q, const void* k, const void* v, int32_t dtype, const int32_t* indices,
                            const int32_t* cu_seqlens, int64_t num_seqs, int64_t total_tokens, int64_t q_heads,
                            int64_t kv_groups, int64_t head_dim, int64_t topk_slots, int64_t block_size,
                            double scale, const int32_t* cu_block_lens, int64_t total_blocks, const int32_t* row_ptr,
                            const int32_t* query_indices, const int32_t* slot_indices, void* workspace,
                            int64_t workspace_bytes, void* out, float* lse, double* row_state, float* out_f32,
                            void* stream) {
  if (!valid_common(num_seqs, total_tokens, q_heads, kv_groups, head_dim, block_size) || topk_slots < 0)
    return kErrInvalidArgument;
  if (total_tokens == 0) return kOk;
  if (head_dim > 2048) return kErrUnsupported;  // VALU path: the q (and dO) rows of a workgroup in LDS
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int nseq = static_cast<int>(num_seqs), Hq = static_cast<int>(q_heads), G = static_cast<int>(kv_groups);
  const int D = static_cast<int>(head_dim), K = static_cast<int>(topk_slots), B = static_cast<int>(block_size);
  if (mfma_dtype(dtype) && attn_mfma_supported(Hq / G, D, B)) {
    // the edge arrays are empty (and may be NULL) when there are no slots
    if (!cu_block_lens || !row_ptr || !workspace || (K > 0 && (!query_indices || !slot_indices)))
      return kErrInvalidArgument;
    return attn_fwd_kv(dtype, q, k, v, indices, cu_seqlens, nseq, total_tokens, Hq, G, D, K, B, static_cast<float>(scale),
                       cu_block_lens, total_blocks, row_ptr, query_indices, slot_indices, workspace, workspace_bytes,
                       out, lse, row_state, out_f32, st);
  }
  switch (dtype) {
    case kF32: return attn_fwd_valu_dispatch<kF32>(q, k, v, indices, cu_seqlens, nseq, total_tokens, Hq, G, D, K, B, scale, out, lse, row_state, out_f32, st);
    case kF16: return attn_fwd_valu_dispatch<kF16>(q, k, v, indices, cu_seqlens, nseq, total_tokens, Hq, G, D, K, B, scale, out, lse, row_state, out_f32, st);
    case kBF16: return attn_fwd_valu_dispatch<kBF16>(q, k, v, indices, cu_seqlens, nseq, total_tokens, Hq, G, D, K, B, scale, out, lse, row_state, out_f32, st);
    default: return kErrInvalidArgument;
  }
}

extern "C" int64_t msa_attn_bwd_workspace_bytes(int32_t dtype, int64_t total_tokens, int64_t q_heads,
                                                int64_t kv_groups, int64_t head_dim, int64_t topk_slots,
                                                int64_t total_blocks, int64_t block_size) {
  if (q_heads <= 0 || kv_groups <= 0 || q_heads % kv_groups || total_tokens <= 0) return 0;
  if (!mfma_dtype(dtype) || !attn_mfma_supported(q_heads / kv_groups, head_dim, block_size)) return 0;
  return attn_bwd_kv_workspace_bytes(total_tokens, q_heads, kv_groups, head_dim, topk_slots, total_blocks);
}

extern "C" int msa_attn_bwd(const void* q, const void* k, const void* v, int32_t dtype, const void* out,
                            const void* grad_out, double* row_state, const float* out_f32, const int32_t* indices,
                            const int32_t* cu_seqlens, int64_t num_seqs, int64_t total_tokens, int64_t q_heads,
                            int64_t kv_groups, int64_t head_dim, int64_t topk_slots, int64_t block_size,
                            double scale, const int32_t* cu_block_lens, int64_t total_blocks, const int32_t* row_ptr,
                            const int32_t* query_indices, const int32_t* slot_indices, void* grad_q, void* grad_k,
                            void* grad_v, void* workspace, int64_t workspace_bytes, void* stream) {
  if (!valid_common(num_seqs, total_tokens, q_heads, kv_groups, head_dim, block_size) || topk_slots < 0 ||
      total_blocks < 0 || row_state == nullptr)
    return kErrInvalidArgument;
  if (total_tokens == 0 || (!grad_q && !grad_k && !grad_v)) return kOk;
  if (head_dim > 2048) return kErrUnsupported;  // VALU path: the q (and dO) rows of a workgroup in LDS
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int nseq = static_cast<int>(num_seqs), Hq = static_cast<int>(q_heads), G = static_cast<int>(kv_groups);
  const int D = static_cast<int>(head_dim), K = static_cast<int>(topk_slots), B = static_cast<int>(block_size);
  const bool need_kv = grad_k != nullptr || grad_v != nullptr;
  if (mfma_dtype(dtype) && attn_mfma_supported(Hq / G, D, B)) {
    if (!cu_block_lens || !row_ptr || !workspace || (K > 0 && (!query_indices || !slot_indices)))
      return kErrInvalidArgument;
    return attn_bwd_kv(dtype, q, k, v, out, grad_out, row_state, indices, cu_seqlens, nseq, total_tokens, Hq, G, D, K, B,
                       static_cast<float>(scale), cu_block_lens, total_blocks, row_ptr, query_indices, slot_indices,
                       grad_q, grad_k, grad_v, workspace, workspace_bytes, out_f32, st);
  }
  if (need_kv && (!cu_block_lens || !row_ptr || (K > 0 && !query_indices))) return kErrInvalidArgument;
  // VALU path: the query pass (dQ and the row statistics), then the KV pass.
  int rc = kErrInvalidArgument;
  switch (dtype) {
    case kF32: rc = attn_dq_valu_dispatch<kF32>(q, k, v, out, grad_out, row_state, indices, cu_seqlens, nseq, total_tokens, Hq, G, D, K, B, scale, grad_q, st); break;
    case kF16: rc = attn_dq_valu_dispatch<kF16>(q, k, v, out, grad_out, row_state, indices, cu_seqlens, nseq, total_tokens, Hq, G, D, K, B, scale, grad_q, st); break;
    case kBF16: rc = attn_dq_valu_dispatch<kBF16>(q, k, v, out, grad_out, row_state, indices, cu_seqlens, nseq, total_tokens, Hq, G, D, K, B, scale, grad_q, st); break;
    default: return kErrInvalidArgument;
  }
  if (rc != kOk || !need_kv) return rc;
  switch (dtype) {
    case kF32: return attn_dkdv_valu_dispatch<kF32>(q, k, v, grad_out, row_state, cu_seqlens, cu_block_lens, row_ptr, query_indices, nseq, total_tokens, Hq, G, D, B, scale, grad_k, grad_v, st);
    case kF16: return attn_dkdv_valu_dispatch<kF16>(q, k, v, grad_out, row_state, cu_seqlens, cu_block_lens, row_ptr, query_indices, nseq, total_tokens, Hq, G, D, B, scale, grad_k, grad_v, st);
    default: return attn_dkdv_valu_dispatch<kBF16>(q, k, v, grad_out, row_state, cu_seqlens, cu_block_lens, row_ptr, query_indices, nseq, total_tokens, Hq, G, D, B, scale, grad_k, grad_v, st);
  }
}
