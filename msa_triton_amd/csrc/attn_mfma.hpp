// MFMA kernels of stage 3 (bf16 and fp16 inputs, dt = kBF16 / kF16): KV-major forward
// (attn_kv_fwd.hip) and backward (attn_kv_bwd.hip).
#pragma once
#include "common.hpp"

namespace msa {

// Shapes the MFMA kernels cover: head ratio <= 512 (a work item holds whole edges of
// at most 512 rows), 8 <= D <= 256 with D % 8 == 0, block <= 128.
bool attn_mfma_supported(int64_t ratio, int64_t head_dim, int64_t block_size);

int64_t attn_fwd_kv_workspace_bytes(int64_t T, int64_t Hq, int64_t G, int64_t D, int64_t K, int64_t total_blocks);

int64_t attn_bwd_kv_workspace_bytes(int64_t T, int64_t Hq, int64_t G, int64_t D, int64_t K, int64_t total_blocks);

int attn_bwd_kv(int dt, const void* q, const void* k, const void* v, const void* out, const void* dout, double* rs,
                const int32_t* indices, const int32_t* cu, int nseq, int64_t T, int Hq, int G, int D, int K, int B,
                float scale, const int32_t* cu_blocks, int64_t total_blocks, const int32_t* row_ptr,
                const int32_t* qidx, const int32_t* sidx, void* dq, void* dk, void* dv, void* ws, int64_t ws_bytes,
                const float* o32, hipStream_t st);

int attn_fwd_kv(int dt, const void* q, const void* k, const void* v, const int32_t* indices, const int32_t* cu, int nseq,
                int64_t T, int Hq, int G, int D, int K, int B, float scale, const int32_t* cu_blocks,
                int64_t total_blocks, const int32_t* row_ptr, const int32_t* qidx, const int32_t* sidx, void* ws,
                int64_t ws_bytes, void* out, float* lse, double* rs, float* o32, hipStream_t st);

}  // namespace msa
