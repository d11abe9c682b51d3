// Causal top-k block selection with forced local blocks.
//
// Semantics follow triton/topk.py:31-46 (eager twin eager/ops.py:94-129):
//   * blocks b > qb(t) are masked to -inf,
//   * blocks in (qb-L, qb] are forced to +inf,
//   * the min(K, NB) largest are returned in descending order, -inf picks
//     become -1, and the row is right-padded with -1 up to K slots.
// Ties (equal values, e.g. several +inf local blocks) are emitted in
// ascending block order; this is the canonical order documented for the
// drop-in (torch.topk leaves it unspecified).
//
// Sixteen lanes own one (token, group) row and hold the row's causal prefix in
// registers (VPL values per lane). Selection is an iterated argmax on a 64-bit
// key (ordered float bits << 32 | ~block) so that the comparison itself
// implements "larger value, then smaller block id".
#include "topk_row.hpp"

namespace msa {

// Sixteen lanes per row, four rows per wavefront (topk_row16). In these kernels the
// workgroups take the rows from the last one back: a row's work grows with its
// position in the sequence, so the heaviest rows start first.
template <int VPL>
__global__ __launch_bounds__(256) void topk_kernel(const float* __restrict__ scores,
                                                   const int32_t* __restrict__ cu, int nseq,
                                                   int64_t rows, int G, int NB, int B, int K, int L,
                                                   int32_t* __restrict__ out) {
  topk_row16<VPL>(scores, cu, nseq, rows, G, NB, B, K, L, out,
                  static_cast<int64_t>(gridDim.x - 1 - blockIdx.x) * 16 + (threadIdx.x >> 4), threadIdx.x & 15);
}

// One wavefront per row for long rows (more than 1024 blocks): topk_row64.
template <int VPL>
__global__ __launch_bounds__(256) void topk_wave_kernel(const float* __restrict__ scores,
                                                        const int32_t* __restrict__ cu, int nseq,
                                                        int64_t rows, int G, int NB, int B, int K, int L,
                                                        int32_t* __restrict__ out) {
  const int64_t row = static_cast<int64_t>(gridDim.x - 1 - blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  topk_row64<VPL>(scores, cu, nseq, G, NB, B, K, L, out, row, threadIdx.x & 63);
}

// One wavefront per row, row streamed from memory (more than 4096 blocks): topk_row_stream.
__global__ __launch_bounds__(256) void topk_stream_kernel(const float* __restrict__ scores,
                                                          const int32_t* __restrict__ cu, int nseq, int64_t rows,
                                                          int G, int NB, int B, int K, int L,
                                                          int32_t* __restrict__ out) {
  const int64_t row = static_cast<int64_t>(gridDim.x - 1 - blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  topk_row_stream(scores, cu, nseq, G, NB, B, K, L, out, row, threadIdx.x & 63);
}

}  // namespace msa

using namespace msa;

namespace msa {

int topk_launch(const float* scores, const int32_t* cu_seqlens, int nseq, int64_t rows, int G, int NB, int B, int K,
                int L, int32_t* indices, hipStream_t st) {
  if (rows == 0 || K == 0) return kOk;
  dim3 grid(grid_1d(rows, 16)), block(256);
#define MSA_TOPK_LAUNCH(V) \
  hipLaunchKernelGGL(topk_kernel<V>, grid, block, 0, st, scores, cu_seqlens, nseq, rows, G, NB, B, K, L, indices)
#define MSA_TOPK_WAVE(V) \
  hipLaunchKernelGGL(topk_wave_kernel<V>, dim3(grid_1d(rows, 4)), block, 0, st, scores, cu_seqlens, nseq, rows, G, NB, B, K, L, indices)
  if (NB <= 16) MSA_TOPK_LAUNCH(1);
  else if (NB <= 32) MSA_TOPK_LAUNCH(2);
  else if (NB <= 64) MSA_TOPK_LAUNCH(4);
  else if (NB <= 128) MSA_TOPK_LAUNCH(8);
  else if (NB <= 256) MSA_TOPK_LAUNCH(16);
  else if (NB <= 512) MSA_TOPK_LAUNCH(32);
  else if (NB <= 1024) MSA_TOPK_LAUNCH(64);
  else if (NB <= 2048) MSA_TOPK_WAVE(32);
  else if (NB <= 4096) MSA_TOPK_WAVE(64);
  else hipLaunchKernelGGL(topk_stream_kernel, dim3(grid_1d(rows, 4)), block, 0, st, scores, cu_seqlens, nseq, rows, G, NB, B, K, L, indices);
#undef MSA_TOPK_LAUNCH
#undef MSA_TOPK_WAVE
  return status_from(hipGetLastError());
}

}  // namespace msa

extern "C" int msa_topk(const float* scores, const int32_t* cu_seqlens, int64_t num_seqs,
                        int64_t total_tokens, int64_t groups, int64_t num_blocks, int64_t block_size,
                        int64_t topk_blocks, int64_t local_blocks, int32_t* indices, void* stream) {
  if (total_tokens < 0 || groups <= 0 || num_blocks <= 0 || block_size <= 0 || topk_blocks < 0 ||
      local_blocks < 0 || local_blocks > topk_blocks || num_seqs <= 0)
    return kErrInvalidArgument;
  return topk_launch(scores, cu_seqlens, static_cast<int>(num_seqs), total_tokens * groups, static_cast<int>(groups),
                     static_cast<int>(num_blocks), static_cast<int>(block_size), static_cast<int>(topk_blocks),
                     static_cast<int>(local_blocks), indices, static_cast<hipStream_t>(stream));
}
