// Stage 1: indexer block scores and their amax backward.
//
// Forward semantics (triton/index_score.py:93-136, FP64 oracle
// tests/reference_fp64.py:16-45): for row (t, g) and sequence-local block b,
//   score[t,g,b] = max_{j in block b, j <= t} scale * (index_q[t,g] . index_k[j])
// or -inf when the block holds no causal key. The reference compares winners
// with a compensated (hi, lo) FP32 dot and publishes fl32(hi*|s| + lo*|s|); for
// finite bf16/fp16/fp32 inputs that is the correctly rounded exact block max.
// Here the winning dot is evaluated in FP64 (bf16/fp16/fp32 products are exact
// in FP64; the accumulation order is fixed, see exact_dot) and rounded once to
// FP32. Winners are compared on the exact
// (directed) dot, ties are exact equality: tie_info = offset+1 for a unique
// winner, -count for ties (index_score.py:128-136).
//
// Backward (index_score.py:139-232): ds*scale goes to the unique winner or is
// split evenly across exact ties. dq is a per-row gather; dk inverts the winner
// map per key block. Both accumulate in FP64 in a fixed order (no float
// atomics), then round to the input dtype.
#include "common.hpp"
#include "score_mfma.hpp"

namespace msa {

// ---- forward, exact FP64 path (all dtypes) -----------------------------------

// One wavefront per (row, block): lanes evaluate keys in FP64 and reduce.
template <int DT>
__global__ __launch_bounds__(256) void score_fwd_exact(const void* __restrict__ iq,
                                                       const void* __restrict__ ik,
                                                       const int32_t* __restrict__ cu, int nseq,
                                                       int64_t rows, int G, int Di, int NB, int B,
                                                       double scale, float* __restrict__ scores,
                                                       int32_t* __restrict__ tie_info) {
  const int64_t w = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (w >= rows * NB) return;
  const int lane = threadIdx.x & 63;
  const int64_t row = w / NB;
  const int b = static_cast<int>(w % NB);
  const int64_t t = row / G;
  const int s = find_seq(cu, nseq, t);
  const int64_t start = cu[s];
  const int64_t pos = t - start;
  const int64_t out = row * NB + b;
  if (static_cast<int64_t>(b) * B > pos) {
    if (lane == 0) {
      scores[out] = -__builtin_inff();
      if (tie_info) tie_info[out] = 0;
    }
    return;
  }
  const int64_t k0 = start + static_cast<int64_t>(b) * B;
  const int64_t k1 = (k0 + B < t + 1) ? k0 + B : t + 1;
  const BlockMax bm = block_max_exact<DT>(iq, row * Di, ik, k0, k1, Di, scale, lane);
  if (lane == 0) {
    scores[out] = static_cast<float>(fabs(scale) * bm.best);
    if (tie_info) tie_info[out] = bm.count == 1 ? bm.first + 1 : -bm.count;
  }
}

// ---- backward -----------------------------------------------------------------

// Transpose (tie, ds) from [rows, NB] to block-major [NB, rows] so the key-block
// pass reads them contiguously. 64x64 tiles through LDS.
__global__ __launch_bounds__(256) void score_bwd_transpose(const int32_t* __restrict__ tie,
                                                           const float* __restrict__ ds, int64_t rows,
                                                           int NB, int32_t* __restrict__ tie_t,
                                                           float* __restrict__ ds_t) {
  __shared__ int32_t tt[64][65];
  __shared__ float dt[64][65];
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * 64;
  const int b0 = blockIdx.y * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int i = ty; i < 64; i += 4) {
    const int64_t r = r0 + i;
    const int b = b0 + tx;
    if (r < rows && b < NB) {
      tt[i][tx] = tie[r * NB + b];
      dt[i][tx] = ds[r * NB + b];
    }
  }
  __syncthreads();
  for (int i = ty; i < 64; i += 4) {
    const int b = b0 + i;
    const int64_t r = r0 + tx;
    if (r < rows && b < NB) {
      tie_t[static_cast<int64_t>(b) * rows + r] = tt[tx][i];
      ds_t[static_cast<int64_t>(b) * rows + r] = dt[tx][i];
    }
  }
}

// dq[t,g] = sum over valid blocks of w * k[winner] (ties: w/count per tied key).
// One wavefront per row, lanes over index dims, FP64 accumulation in block order.
template <int DT, int DPL>
__global__ __launch_bounds__(256) void score_bwd_dq(const void* __restrict__ iq,
                                                    const void* __restrict__ ik,
                                                    const int32_t* __restrict__ cu, int nseq,
                                                    const int32_t* __restrict__ tie,
                                                    const float* __restrict__ ds, int64_t rows, int G,
                                                    int Di, int NB, int B, double scale,
                                                    void* __restrict__ dq) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const int64_t t = row / G;
  const int s = find_seq(cu, nseq, t);
  const int64_t start = cu[s];
  const int64_t pos = t - start;
  const int nvalid = static_cast<int>(pos / B + 1 < NB ? pos / B + 1 : NB);
  double acc[DPL];
#pragma unroll
  for (int i = 0; i < DPL; ++i) acc[i] = 0.0;
  for (int b0 = 0; b0 < nvalid; b0 += 64) {
    const int bl = b0 + lane;
    const int32_t my_tie = bl < nvalid ? tie[row * NB + bl] : 0;
    const float my_ds = bl < nvalid ? ds[row * NB + bl] : 0.f;
    const int n = nvalid - b0 < 64 ? nvalid - b0 : 64;
    for (int i = 0; i < n; ++i) {
      const int32_t ti = __shfl(my_tie, i, kWave);
      const float di = __shfl(my_ds, i, kWave);
      const int64_t k0 = start + static_cast<int64_t>(b0 + i) * B;
      if (ti > 0) {
        const double wgt = static_cast<double>(di) * scale;
        const int64_t key = k0 + ti - 1;
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          const int d = lane + j * kWave;
          if (d < Di) acc[j] = fma(wgt, static_cast<double>(load_as_f32<DT>(ik, key * Di + d)), acc[j]);
        }
      } else if (ti < 0) {
        const int64_t k1 = (k0 + B < t + 1) ? k0 + B : t + 1;
        const BlockMax bm = block_max_exact<DT>(iq, row * Di, ik, k0, k1, Di, scale, lane);
        const double wgt = static_cast<double>(di) * scale / static_cast<double>(bm.count);
        for_each_winner<DT>(iq, row * Di, ik, k0, k1, Di, scale, bm.best, lane, [&](int64_t kk) {
#pragma unroll
          for (int j = 0; j < DPL; ++j) {
            const int d = lane + j * kWave;
            if (d < Di) acc[j] = fma(wgt, static_cast<double>(load_as_f32<DT>(ik, kk * Di + d)), acc[j]);
          }
        });
      }
    }
  }
#pragma unroll
  for (int j = 0; j < DPL; ++j) {
    const int d = lane + j * kWave;
    if (d < Di) store_from_f32<DT>(dq, row * Di + d, static_cast<float>(acc[j]));
  }
}

// dk for one (key block, 128-key chunk, 64-dim chunk): one wavefront scans the
// block's rows (t, g) with t in the block's sequence and t >= block start, in
// row order, and adds w * q[row] into the winner's FP64 accumulator in LDS.
// Lanes own index dims, so every row update is a whole-wave, conflict-free
// read-modify-write; the fixed row order makes the sum deterministic.
template <int DT>
__global__ __launch_bounds__(64) void score_bwd_dk(const void* __restrict__ iq,
                                                   const void* __restrict__ ik,
                                                   const int32_t* __restrict__ cu,
                                                   const int32_t* __restrict__ cu_blocks, int nseq,
                                                   const int32_t* __restrict__ tie_t,
                                                   const float* __restrict__ ds_t, int64_t rows, int G,
                                                   int Di, int B, double scale, void* __restrict__ dk) {
  __shared__ double acc[128][64];
  const int lane = threadIdx.x;
  const int64_t gb = blockIdx.x;
  const int kc = blockIdx.y;  // key chunk of 128
  const int d = blockIdx.z * 64 + lane;
  int s = upper_index(cu_blocks, nseq + 1, gb);
  while (s < nseq && cu_blocks[s + 1] <= gb) ++s;
  const int b = static_cast<int>(gb - cu_blocks[s]);
  const int64_t start = cu[s], end = cu[s + 1];
  const int64_t k0 = start + static_cast<int64_t>(b) * B;
  const int64_t kend = k0 + B < end ? k0 + B : end;
  const int64_t c0 = k0 + static_cast<int64_t>(kc) * 128;
  if (c0 >= kend) return;
  const int nk = static_cast<int>(kend - c0 < 128 ? kend - c0 : 128);
  for (int i = 0; i < nk; ++i) acc[i][lane] = 0.0;
  const int64_t r_begin = k0 * G, r_end = end * G;
  const int32_t* tcol = tie_t + static_cast<int64_t>(b) * rows;
  const float* dcol = ds_t + static_cast<int64_t>(b) * rows;
  const int64_t qoff = static_cast<int64_t>(kc) * 128 + 1;  // tie value of this chunk's first key
  for (int64_t r0 = r_begin; r0 < r_end; r0 += 64) {
    const int64_t r = r0 + lane;
    const int32_t my_tie = r < r_end ? tcol[r] : 0;
    const float my_ds = r < r_end ? dcol[r] : 0.f;
    const bool mine = my_tie < 0 || (my_tie >= qoff && my_tie < qoff + nk);
    uint64_t mask = __ballot(mine);
    while (mask) {
      const int i = __builtin_ctzll(mask);
      mask &= mask - 1;
      const int32_t ti = __shfl(my_tie, i, kWave);
      const float di = __shfl(my_ds, i, kWave);
      const int64_t row = r0 + i;
      const float qv = d < Di ? load_as_f32<DT>(iq, row * Di + d) : 0.f;
      if (ti > 0) {
        const int o = static_cast<int>(ti - qoff);
        acc[o][lane] = fma(static_cast<double>(di) * scale, static_cast<double>(qv), acc[o][lane]);
      } else {
        const int64_t t = row / G;
        const int64_t k1 = (k0 + B < t + 1) ? k0 + B : t + 1;
        const BlockMax bm = block_max_exact<DT>(iq, row * Di, ik, k0, k1, Di, scale, lane);
        const double wgt = static_cast<double>(di) * scale / static_cast<double>(bm.count);
        const int64_t hi = k1 < c0 + nk ? k1 : c0 + nk;
        if (hi > c0) {
          for_each_winner<DT>(iq, row * Di, ik, c0, hi, Di, scale, bm.best, lane, [&](int64_t kk) {
            const int o = static_cast<int>(kk - c0);
            acc[o][lane] = fma(wgt, static_cast<double>(qv), acc[o][lane]);
          });
        }
      }
    }
  }
  if (d < Di) {
    for (int i = 0; i < nk; ++i) store_from_f32<DT>(dk, (c0 + i) * Di + d, static_cast<float>(acc[i][lane]));
  }
}

template <int DT>
int score_fwd_launch(const void* iq, const void* ik, const int32_t* cu, int nseq, int64_t rows, int G,
                     int Di, int NB, int B, double scale, float* scores, int32_t* tie, hipStream_t st) {
  if (DT == kBF16 && score_mfma_supported(Di, B, scale)) {
    return score_fwd_mfma_launch(iq, ik, cu, nseq, rows, G, Di, NB, B, scale, scores, tie, st);
  }
  const int64_t waves = rows * NB;
  hipLaunchKernelGGL(score_fwd_exact<DT>, dim3(grid_1d(waves, 4)), dim3(256), 0, st, iq, ik, cu, nseq, rows,
                     G, Di, NB, B, scale, scores, tie);
  return status_from(hipGetLastError());
}

template <int DT>
int score_bwd_launch(const void* iq, const void* ik, const int32_t* cu, const int32_t* cu_blocks, int nseq,
                     const int32_t* tie, const float* ds, int64_t rows, int G, int Di, int NB, int B,
                     int64_t total_blocks, double scale, void* dq, void* dk, void* ws, hipStream_t st) {
  if (dq) {
    const dim3 grid(grid_1d(rows, 4)), block(256);
    if (Di <= 64) hipLaunchKernelGGL((score_bwd_dq<DT, 1>), grid, block, 0, st, iq, ik, cu, nseq, tie, ds, rows, G, Di, NB, B, scale, dq);
    else if (Di <= 128) hipLaunchKernelGGL((score_bwd_dq<DT, 2>), grid, block, 0, st, iq, ik, cu, nseq, tie, ds, rows, G, Di, NB, B, scale, dq);
    else if (Di <= 256) hipLaunchKernelGGL((score_bwd_dq<DT, 4>), grid, block, 0, st, iq, ik, cu, nseq, tie, ds, rows, G, Di, NB, B, scale, dq);
    else hipLaunchKernelGGL((score_bwd_dq<DT, 8>), grid, block, 0, st, iq, ik, cu, nseq, tie, ds, rows, G, Di, NB, B, scale, dq);
  }
  if (dk && total_blocks > 0) {
    int32_t* tie_t = static_cast<int32_t*>(ws);
    float* ds_t = reinterpret_cast<float*>(tie_t + rows * NB);
    const dim3 tgrid(grid_1d(rows, 64), static_cast<unsigned>((NB + 63) / 64));
    hipLaunchKernelGGL(score_bwd_transpose, tgrid, dim3(256), 0, st, tie, ds, rows, NB, tie_t, ds_t);
    const dim3 grid(static_cast<unsigned>(total_blocks), static_cast<unsigned>((B + 127) / 128),
                    static_cast<unsigned>((Di + 63) / 64));
    hipLaunchKernelGGL(score_bwd_dk<DT>, grid, dim3(64), 0, st, iq, ik, cu, cu_blocks, nseq, tie_t, ds_t, rows,
                       G, Di, B, scale, dk);
  }
  return status_from(hipGetLastError());
}

}  // namespace msa

using namespace msa;

extern "C" int msa_score_fwd(const void* index_q, const void* index_k, int32_t dtype,
                             const int32_t* cu_seqlens, int64_t num_seqs, int64_t total_tokens,
                             int64_t groups, int64_t index_dim, int64_t num_blocks, int64_t block_size,
                             double scale, float* scores, int32_t* tie_info, void* stream) {
  if (num_seqs <= 0 || total_tokens < 0 || groups <= 0 || index_dim <= 0 || num_blocks <= 0 ||
      block_size <= 0)
    return kErrInvalidArgument;
  const int64_t rows = total_tokens * groups;
  if (rows == 0) return kOk;
  if (index_dim > 512) return kErrUnsupported;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int nseq = static_cast<int>(num_seqs), G = static_cast<int>(groups);
  const int Di = static_cast<int>(index_dim), NB = static_cast<int>(num_blocks);
  const int B = static_cast<int>(block_size);
  switch (dtype) {
    case kF32: return score_fwd_launch<kF32>(index_q, index_k, cu_seqlens, nseq, rows, G, Di, NB, B, scale, scores, tie_info, st);
    case kF16: return score_fwd_launch<kF16>(index_q, index_k, cu_seqlens, nseq, rows, G, Di, NB, B, scale, scores, tie_info, st);
    case kBF16: return score_fwd_launch<kBF16>(index_q, index_k, cu_seqlens, nseq, rows, G, Di, NB, B, scale, scores, tie_info, st);
    default: return kErrInvalidArgument;
  }
}

extern "C" int64_t msa_score_bwd_workspace_bytes(int64_t total_tokens, int64_t groups, int64_t num_blocks,
                                                 int64_t index_dim) {
  (void)index_dim;
  return total_tokens * groups * num_blocks * 8 + 256;
}

extern "C" int msa_score_bwd(const void* index_q, const void* index_k, int32_t dtype,
                             const int32_t* cu_seqlens, const int32_t* cu_block_lens, const int32_t* tie_info,
                             const float* grad_scores, int64_t num_seqs, int64_t total_tokens, int64_t groups,
                             int64_t index_dim, int64_t num_blocks, int64_t block_size, int64_t total_blocks,
                             double scale, void* grad_q, void* grad_k, void* workspace, void* stream) {
  if (num_seqs <= 0 || total_tokens < 0 || groups <= 0 || index_dim <= 0 || num_blocks <= 0 ||
      block_size <= 0 || total_blocks < 0)
    return kErrInvalidArgument;
  const int64_t rows = total_tokens * groups;
  if (rows == 0) return kOk;
  if (index_dim > 512) return kErrUnsupported;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int nseq = static_cast<int>(num_seqs), G = static_cast<int>(groups);
  const int Di = static_cast<int>(index_dim), NB = static_cast<int>(num_blocks);
  const int B = static_cast<int>(block_size);
  switch (dtype) {
    case kF32: return score_bwd_launch<kF32>(index_q, index_k, cu_seqlens, cu_block_lens, nseq, tie_info, grad_scores, rows, G, Di, NB, B, total_blocks, scale, grad_q, grad_k, workspace, st);
    case kF16: return score_bwd_launch<kF16>(index_q, index_k, cu_seqlens, cu_block_lens, nseq, tie_info, grad_scores, rows, G, Di, NB, B, total_blocks, scale, grad_q, grad_k, workspace, st);
    case kBF16: return score_bwd_launch<kBF16>(index_q, index_k, cu_seqlens, cu_block_lens, nseq, tie_info, grad_scores, rows, G, Di, NB, B, total_blocks, scale, grad_q, grad_k, workspace, st);
    default: return kErrInvalidArgument;
  }
}
