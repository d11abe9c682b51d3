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
// split evenly across exact ties. dq is a per-row gather; dk scans each key
// block's rows for the winners it owns (row segments, summed in order). Both accumulate in FP64 in a fixed order (no float
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
    // blocks in order; unique winners' key rows are loaded four at a time
    int i = 0;
    while (i < n) {
      int bi[4];
      int cnt = 0;
      while (cnt < 4 && i < n) {
        if (__shfl(my_tie, i, kWave) <= 0) break;  // a tie (or an empty block) is handled alone, in order
        bi[cnt++] = i++;
      }
      if (cnt > 0) {
        float kv[4][DPL];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          if (u < cnt) {
            const int32_t ti = __shfl(my_tie, bi[u], kWave);
            const int64_t key = start + static_cast<int64_t>(b0 + bi[u]) * B + ti - 1;
#pragma unroll
            for (int j = 0; j < DPL; ++j) {
              const int d = lane + j * kWave;
              kv[u][j] = d < Di ? load_as_f32<DT>(ik, key * Di + d) : 0.f;
            }
          }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          if (u < cnt) {
            const double wgt = static_cast<double>(__shfl(my_ds, bi[u], kWave)) * scale;
#pragma unroll
            for (int j = 0; j < DPL; ++j) acc[j] = fma(wgt, static_cast<double>(kv[u][j]), acc[j]);
          }
        }
        continue;
      }
      const int32_t ti = __shfl(my_tie, i, kWave);
      const float di = __shfl(my_ds, i, kWave);
      const int64_t k0 = start + static_cast<int64_t>(b0 + i) * B;
      ++i;
      if (ti < 0) {
        const int64_t k1 = (k0 + B < t + 1) ? k0 + B : t + 1;
        const BlockMax bm = block_max_exact<DT>(iq, row * Di, ik, k0, k1, Di, scale, lane);
        const double wgt = static_cast<double>(di) * scale / static_cast<double>(bm.count);
        for (int64_t base = k0; base < k1; base += kWave) {
          const int64_t kk = base + lane;
          const bool win = kk < k1 && directed(exact_dot<DT>(iq, row * Di, ik, kk * Di, Di), scale) == bm.best;
          uint64_t mask = __ballot(win);
          while (mask) {
            const int wl = __builtin_ctzll(mask);
            mask &= mask - 1;
#pragma unroll
            for (int j = 0; j < DPL; ++j) {
              const int d = lane + j * kWave;
              if (d < Di) acc[j] = fma(wgt, static_cast<double>(load_as_f32<DT>(ik, (base + wl) * Di + d)), acc[j]);
            }
          }
        }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < DPL; ++j) {
    const int d = lane + j * kWave;
    if (d < Di) store_from_f32<DT>(dq, row * Di + d, static_cast<float>(acc[j]));
  }
}

// dk, partial sums. One wavefront per (key block gb, 8 keys, row segment, 128-dim
// chunk): it scans the segment's rows (t, g) of gb's sequence with t >= block
// start, 64 per step (lanes = rows, block-major tie/ds), and adds w * q[row] for
// rows whose unique winner is one of its keys (lanes = dims, FP64, row order;
// q rows are loaded four at a time). Exact ties add w / count to every tied key
// among its keys (exact recomputation). The per-segment sums go to
// part[((wave * dchunks + dc) * 8 + key) * 128 + dim]; score_bwd_dk_reduce adds
// the segments in order.
constexpr int kDkKeys = 8;

template <int DT>
__global__ __launch_bounds__(256) void score_bwd_dk_part(
    const void* __restrict__ iq, const void* __restrict__ ik, const int32_t* __restrict__ cu,
    const int32_t* __restrict__ cu_blocks, int nseq, const int32_t* __restrict__ tie_t,
    const float* __restrict__ ds_t, int64_t rows, int G, int Di, int B, int kgroups, int nseg, int64_t seg_rows,
    int64_t total_blocks, double scale, double* __restrict__ part) {
  const int lane = threadIdx.x & 63;
  const int64_t w = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (w >= total_blocks * kgroups * nseg) return;
  const int sg = static_cast<int>(w % nseg);
  const int kg = static_cast<int>((w / nseg) % kgroups);
  const int64_t gb = w / nseg / kgroups;
  const int dc = blockIdx.y, dchunks = gridDim.y;
  int s = upper_index(cu_blocks, nseq + 1, gb);
  while (s < nseq && cu_blocks[s + 1] <= gb) ++s;
  const int b = static_cast<int>(gb - cu_blocks[s]);
  const int64_t start = cu[s], end = cu[s + 1];
  const int64_t k0 = start + static_cast<int64_t>(b) * B;
  const int64_t kend = k0 + B < end ? k0 + B : end;
  const int o0 = kg * kDkKeys;
  const int64_t kA = k0 + o0;
  const int nk = static_cast<int>(kend - kA < kDkKeys ? kend - kA : kDkKeys);
  const int64_t r_begin = k0 * G + sg * seg_rows;
  const int64_t r_stop = (k0 * G + (sg + 1) * seg_rows) < end * G ? k0 * G + (sg + 1) * seg_rows : end * G;
  double acc[kDkKeys][2];
#pragma unroll
  for (int kk = 0; kk < kDkKeys; ++kk) acc[kk][0] = acc[kk][1] = 0.0;
  const int d0 = dc * 128 + lane, d1 = d0 + 64;
  if (nk > 0) {
    const int32_t* tcol = tie_t + static_cast<int64_t>(b) * rows;
    const float* dcol = ds_t + static_cast<int64_t>(b) * rows;
    int32_t tie_n = 0;
    float ds_n = 0.f;
    if (r_begin + lane < r_stop) {
      tie_n = tcol[r_begin + lane];
      ds_n = dcol[r_begin + lane];
    }
    for (int64_t r0 = r_begin; r0 < r_stop; r0 += 64) {
      const int32_t tie = tie_n;
      const float dsv = ds_n;
      if (r0 + 64 + lane < r_stop) {  // prefetch the next step; lanes past the segment end carry no row
        tie_n = tcol[r0 + 64 + lane];
        ds_n = dcol[r0 + 64 + lane];
      } else {
        tie_n = 0;
        ds_n = 0.f;
      }
      const int rel = tie - 1 - o0;  // winner offset relative to this wave's first key
      uint64_t m = __ballot(tie > 0 && rel >= 0 && rel < nk);
      while (m) {
        int idx[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          idx[u] = -1;
          if (m) {
            idx[u] = __builtin_ctzll(m);
            m &= m - 1;
          }
        }
        float qv[4][2];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          qv[u][0] = qv[u][1] = 0.f;
          if (idx[u] >= 0) {
            const int64_t row = r0 + idx[u];
            if (d0 < Di) qv[u][0] = load_as_f32<DT>(iq, row * Di + d0);
            if (d1 < Di) qv[u][1] = load_as_f32<DT>(iq, row * Di + d1);
          }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          if (idx[u] < 0) continue;
          const int ru = __shfl(rel, idx[u], kWave);
          const double wgt = static_cast<double>(__shfl(dsv, idx[u], kWave)) * scale;
#pragma unroll
          for (int kk = 0; kk < kDkKeys; ++kk) {
            if (kk == ru) {
              acc[kk][0] = fma(wgt, static_cast<double>(qv[u][0]), acc[kk][0]);
              acc[kk][1] = fma(wgt, static_cast<double>(qv[u][1]), acc[kk][1]);
            }
          }
        }
      }
      // exact ties (rare): recompute the block maximum and test this wave's keys
      uint64_t tm = __ballot(tie < 0);
      while (tm) {
        const int i = __builtin_ctzll(tm);
        tm &= tm - 1;
        const int64_t row = r0 + i;
        const int64_t t = row / G;
        const int64_t k1 = (k0 + B < t + 1) ? k0 + B : t + 1;
        const int64_t hi = k1 < kA + nk ? k1 : kA + nk;
        if (hi <= kA) continue;
        const BlockMax bm = block_max_exact<DT>(iq, row * Di, ik, k0, k1, Di, scale, lane);
        const double wgt = static_cast<double>(__shfl(dsv, i, kWave)) * scale / static_cast<double>(bm.count);
        // lanes 0 .. hi - kA - 1 test this wave's visible keys against the exact maximum
        const bool win = lane < hi - kA &&
                         directed(exact_dot<DT>(iq, row * Di, ik, (kA + lane) * Di, Di), scale) == bm.best;
        const uint32_t wmask = static_cast<uint32_t>(__ballot(win));
        const float q0 = d0 < Di ? load_as_f32<DT>(iq, row * Di + d0) : 0.f;
        const float q1 = d1 < Di ? load_as_f32<DT>(iq, row * Di + d1) : 0.f;
#pragma unroll
        for (int kk = 0; kk < kDkKeys; ++kk) {
          if ((wmask >> kk) & 1u) {
            acc[kk][0] = fma(wgt, static_cast<double>(q0), acc[kk][0]);
            acc[kk][1] = fma(wgt, static_cast<double>(q1), acc[kk][1]);
          }
        }
      }
    }
  }
  double* dst = part + (w * dchunks + dc) * kDkKeys * 128;
#pragma unroll
  for (int kk = 0; kk < kDkKeys; ++kk) {
    dst[kk * 128 + lane] = acc[kk][0];
    dst[kk * 128 + 64 + lane] = acc[kk][1];
  }
}

// dk[key][d] = sum over the key block's row segments (in order) of the partial sums.
template <int DT>
__global__ __launch_bounds__(256) void score_bwd_dk_reduce(const int32_t* __restrict__ cu,
                                                           const int32_t* __restrict__ cu_blocks, int nseq,
                                                           int64_t T, int G, int Di, int B, int kgroups, int nseg,
                                                           int64_t seg_rows, const double* __restrict__ part,
                                                           void* __restrict__ dk) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= T * Di) return;
  const int64_t key = i / Di;
  const int d = static_cast<int>(i % Di);
  const int s = find_seq(cu, nseq, key);
  const int64_t start = cu[s], end = cu[s + 1];
  const int b = static_cast<int>((key - start) / B);
  const int o = static_cast<int>((key - start) % B);
  const int64_t gb = cu_blocks[s] + b;
  const int64_t k0 = start + static_cast<int64_t>(b) * B;
  const int kg = o / kDkKeys, kk = o % kDkKeys;
  const int dc = d / 128, dl = d % 128, dchunks = (Di + 127) / 128;
  double sum = 0.0;
  for (int sg = 0; sg < nseg; ++sg) {
    if (k0 * G + sg * seg_rows >= end * G) break;  // empty segment (no partial written work)
    const int64_t w = (gb * kgroups + kg) * nseg + sg;
    sum += part[((w * dchunks + dc) * kDkKeys + kk) * 128 + dl];
  }
  store_from_f32<DT>(dk, i, static_cast<float>(sum));
}

static int64_t dk_seg_rows(int64_t rows) {
  const int64_t s = (rows + 7) / 8;
  return s > 16384 ? s : 16384;
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
    double* part = reinterpret_cast<double*>(ds_t + rows * NB);  // 8 * rows * NB bytes in: 8-byte aligned
    const dim3 tgrid(grid_1d(rows, 64), static_cast<unsigned>((NB + 63) / 64));
    hipLaunchKernelGGL(score_bwd_transpose, tgrid, dim3(256), 0, st, tie, ds, rows, NB, tie_t, ds_t);
    const int kgroups = (B + kDkKeys - 1) / kDkKeys;
    const int64_t seg_rows = dk_seg_rows(rows);
    const int nseg = static_cast<int>((rows + seg_rows - 1) / seg_rows);
    const int dchunks = (Di + 127) / 128;
    const int64_t waves = total_blocks * kgroups * nseg;
    const dim3 grid(grid_1d(waves, 4), static_cast<unsigned>(dchunks));
    hipLaunchKernelGGL(score_bwd_dk_part<DT>, grid, dim3(256), 0, st, iq, ik, cu, cu_blocks, nseq, tie_t, ds_t, rows,
                       G, Di, B, kgroups, nseg, seg_rows, total_blocks, scale, part);
    const int64_t T = rows / G;
    hipLaunchKernelGGL(score_bwd_dk_reduce<DT>, dim3(grid_1d(T * Di, 256)), dim3(256), 0, st, cu, cu_blocks, nseq, T,
                       G, Di, B, kgroups, nseg, seg_rows, part, dk);
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
                                                 int64_t index_dim, int64_t block_size, int64_t total_blocks) {
  if (total_tokens <= 0 || groups <= 0 || num_blocks <= 0 || index_dim <= 0 || block_size <= 0) return 256;
  const int64_t rows = total_tokens * groups;
  // block-major tie / ds copies, then the dk partial sums (FP64)
  const int64_t tr = rows * num_blocks * 8 + 8;
  const int64_t seg_rows = dk_seg_rows(rows);
  const int64_t nseg = (rows + seg_rows - 1) / seg_rows;
  const int64_t kgroups = (block_size + kDkKeys - 1) / kDkKeys;
  const int64_t dchunks = (index_dim + 127) / 128;
  const int64_t part = total_blocks * kgroups * nseg * dchunks * kDkKeys * 128 * 8;
  return tr + part + 256;
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
