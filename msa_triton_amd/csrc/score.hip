// Stage 1: indexer block scores and their amax backward.
//
// Forward semantics (triton/index_score.py:93-136, FP64 oracle
// tests/reference_fp64.py:16-45): for row (t, g) and sequence-local block b,
//   score[t,g,b] = max_{j in block b, j <= t} scale * (index_q[t,g] . index_k[j])
// or -inf when the block holds no causal key. The reference compares winners
// with a compensated (hi, lo) FP32 dot and publishes fl32(fl32(hi*|s|) + fl32(lo*|s|))
// with |s| in FP32. Here the winning dot is evaluated in FP64 (bf16/fp16/fp32 products
// are exact in FP64; the accumulation order is fixed, see exact_dot), split into the
// same FP32 pair (hi = fl32(dot), lo = fl32(dot - hi)) and published by the same
// FP32 formula (public_score). Winners are compared on the exact
// (directed) dot, ties are exact equality: tie_info = offset+1 for a unique
// winner, -count for ties (index_score.py:128-136).
//
// Backward (index_score.py:139-232): ds*scale goes to the unique winner or is
// split evenly across exact ties. dq is a per-row gather; dk scans each key
// block's rows once per row segment and adds each row into its winner's FP64 LDS
// row (rows in order; segments summed in order). Both accumulate in FP64 in a fixed
// order (no float atomics), then round to the input dtype.
#include "common.hpp"
#include "score_mfma.hpp"
#include "topk_row.hpp"

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
    scores[out] = public_score(bm.best, static_cast<float>(fabs(scale)));
    if (tie_info) tie_info[out] = bm.count == 1 ? bm.first + 1 : -bm.count;
  }
}

// ---- backward -----------------------------------------------------------------

// Transpose (tie, ds) from [rows, NB] to block-major [NB, rows] so the key-block
// pass reads them contiguously. 64x64 tiles through LDS. The key-block pass reads block
// b's column only from the rows that see it (position >= b B), so a tile whose rows lie in
// one sequence and see none of its blocks is skipped (about half the tiles of a long
// sequence).
__global__ __launch_bounds__(256) void score_bwd_transpose(const int32_t* __restrict__ tie,
                                                           const float* __restrict__ ds, int64_t rows,
                                                           int NB, const int32_t* __restrict__ cu, int nseq,
                                                           int G, int B, int32_t* __restrict__ tie_t,
                                                           float* __restrict__ ds_t) {
  __shared__ int32_t tt[64][65];
  __shared__ float dt[64][65];
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * 64;
  const int b0 = blockIdx.y * 64;
  {
    const int64_t t0 = r0 / G, t1 = (r0 + 63 < rows ? r0 + 63 : rows - 1) / G;
    const int s1 = find_seq(cu, nseq, t1);
    if (find_seq(cu, nseq, t0) == s1 && static_cast<int64_t>(b0) * B > t1 - cu[s1]) return;  // whole workgroup
  }
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

__device__ __forceinline__ int lane_i32(int v, int l) { return __builtin_amdgcn_readlane(v, l); }

// Element `hi` (0: low half, 1: high half) of a word holding two 2-byte values, as fp32.
template <int DT>
__device__ __forceinline__ float half_of(uint32_t w, int hi) {
  if constexpr (DT == kBF16) {
    return __uint_as_float(hi ? (w & 0xffff0000u) : (w << 16));
  } else {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(hi ? (w >> 16) : (w & 0xffffu))));
  }
}

// Two FP64 values in the 2-byte output dtype (rounded as store_from_f64 does), packed.
template <int DT>
__device__ __forceinline__ uint32_t pack2(double lo, double hi) {
  if constexpr (DT == kBF16) {
    return static_cast<uint32_t>(f32_to_bf16_bits(static_cast<float>(lo))) |
           (static_cast<uint32_t>(f32_to_bf16_bits(static_cast<float>(hi))) << 16);
  } else {
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(f64_to_f32_odd(lo)))) |
           (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(f64_to_f32_odd(hi)))) << 16);
  }
}
__device__ __forceinline__ float lane_f32(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// dq[t,g] = sum over valid blocks of w * k[winner] (ties: w/count per tied key).
// One wavefront per row, lane j of the wave owns dims dc0 + DPL j .. + DPL - 1 (one
// launch per 64 DPL dims: each dim's sum is independent of the others). The
// row's blocks are taken 64 at a time (lane = block); unique winners are added in
// block order with kDqBatch key rows in flight (block / key broadcast by readlane),
// then the chunk's exact ties (rare) in block order. FP64 accumulation.
constexpr int kDqBatch = 16;
template <int DT, int DPL>
__global__ __launch_bounds__(256) void score_bwd_dq(const void* __restrict__ iq,
                                                    const void* __restrict__ ik,
                                                    const int32_t* __restrict__ cu, int nseq,
                                                    const int32_t* __restrict__ tie,
                                                    const float* __restrict__ ds, int64_t rows, int G,
                                                    int Di, int NB, int B, double scale,
                                                    void* __restrict__ dq, int dc0) {
  // heaviest rows first: a row's work grows with its position in the sequence
  const int64_t row = static_cast<int64_t>(gridDim.x - 1 - blockIdx.x) * 4 + (threadIdx.x >> 6);
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
  const int dbase = dc0 + DPL * lane;  // this pass's dims (index dims above 64 x DPL take several passes)
  for (int b0 = 0; b0 < nvalid; b0 += 64) {
    const int bl = b0 + lane;
    const int32_t my_tie = bl < nvalid ? tie[row * NB + bl] : 0;
    const float my_ds = bl < nvalid ? ds[row * NB + bl] : 0.f;
    // winner key relative to the sequence start (< 2^31: it is a token of the sequence)
    const int my_key = my_tie > 0 ? bl * B + my_tie - 1 : 0;
    uint64_t um = __ballot(my_tie > 0);
    while (um) {
      int bi[kDqBatch];
      int cnt = 0;
#pragma unroll
      for (int u = 0; u < kDqBatch; ++u) {
        bi[u] = 0;
        if (um) {
          bi[u] = __builtin_ctzll(um);
          um &= um - 1;
          cnt = u + 1;
        }
      }
      float kv[kDqBatch][DPL];
#pragma unroll
      for (int u = 0; u < kDqBatch; ++u) {
        const int64_t key = start + lane_i32(my_key, bi[u]);
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          const int d = dbase + j;
          kv[u][j] = (u < cnt && d < Di) ? load_as_f32<DT>(ik, key * Di + d) : 0.f;
        }
      }
#pragma unroll
      for (int u = 0; u < kDqBatch; ++u) {
        if (u < cnt) {
          const double wgt = static_cast<double>(lane_f32(my_ds, bi[u])) * scale;
#pragma unroll
          for (int j = 0; j < DPL; ++j) acc[j] = fma(wgt, static_cast<double>(kv[u][j]), acc[j]);
        }
      }
    }
    // exact ties of this chunk, in block order (rare)
    uint64_t tm = __ballot(my_tie < 0);
    while (tm) {
      const int i = __builtin_ctzll(tm);
      tm &= tm - 1;
      const float di = lane_f32(my_ds, i);
      const int64_t k0 = start + static_cast<int64_t>(b0 + i) * B;
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
            const int d = dbase + j;
            if (d < Di) acc[j] = fma(wgt, static_cast<double>(load_as_f32<DT>(ik, (base + wl) * Di + d)), acc[j]);
          }
        }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < DPL; ++j) {
    const int d = dbase + j;
    if (d < Di) store_from_f64<DT>(dq, row * Di + d, acc[j]);
  }
}

// Wide-gather dq for 2-byte dtypes with Di = 32, 64 or 128: a row of Di
// elements is LPR = Di / 8 lanes x 16 bytes, so one load instruction fetches RPI =
// 64 / LPR winner rows. Per 64-block chunk the unique winners are compacted (in
// block order) into the wave's LDS list; lane (slot, chunk) adds entries slot,
// slot + RPI, ... of the list into FP64 sums of its 8 dims, and the RPI slot sums
// are added in slot order at the end (a fixed order). Exact ties (rare) are added
// by every slot-0 lane after the chunk's unique winners, in block order.
constexpr int kDqWideUnroll = 4;  // key-row gather instructions in flight per wave (80 VGPRs: 6 waves per SIMD)

template <int DT, int LPR>
__global__ __launch_bounds__(256) void score_bwd_dq_wide(const void* __restrict__ iq,
                                                         const void* __restrict__ ik,
                                                         const int32_t* __restrict__ cu, int nseq,
                                                         const int32_t* __restrict__ tie,
                                                         const float* __restrict__ ds, int64_t rows, int G,
                                                         int Di, int NB, int B, double scale,
                                                         void* __restrict__ dq) {
  constexpr int RPI = 64 / LPR;
  __shared__ int32_t lkey[4][64];
  __shared__ float lw[4][64];
  const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(gridDim.x - 1 - blockIdx.x) * 4 + wid;  // heaviest rows first
  if (row >= rows) return;  // whole wave
  const int slot = lane / LPR, dch = lane % LPR;
  const int64_t t = row / G;
  const int sq = find_seq(cu, nseq, t);
  const int64_t start = cu[sq];
  const int64_t pos = t - start;
  const int nvalid = static_cast<int>(pos / B + 1 < NB ? pos / B + 1 : NB);
  const uint16_t* kb16 = static_cast<const uint16_t*>(ik);
  double acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.0;
  const uint64_t lt = (uint64_t(1) << lane) - 1;
  for (int b0 = 0; b0 < nvalid; b0 += 64) {
    const int bl = b0 + lane;
    const int32_t my_tie = bl < nvalid ? tie[row * NB + bl] : 0;
    const float my_ds = bl < nvalid ? ds[row * NB + bl] : 0.f;
    const uint64_t um = __ballot(my_tie > 0);
    if (my_tie > 0) {
      const int p = __popcll(um & lt);
      lkey[wid][p] = bl * B + my_tie - 1;  // winner key relative to the sequence start
      lw[wid][p] = my_ds;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int n = __popcll(um);
    for (int e0 = 0; e0 < n; e0 += kDqWideUnroll * RPI) {
      // all list reads, then all key-row loads (clamped entries, in bounds), then the sums
      uint4 kv[kDqWideUnroll];
      double wv[kDqWideUnroll];
      int kk[kDqWideUnroll];
      float wf[kDqWideUnroll];
      bool ok[kDqWideUnroll];
#pragma unroll
      for (int u = 0; u < kDqWideUnroll; ++u) {
        const int e = e0 + u * RPI + slot;
        ok[u] = e < n;
        kk[u] = lkey[wid][ok[u] ? e : 0];
        wf[u] = lw[wid][ok[u] ? e : 0];
      }
#pragma unroll
      for (int u = 0; u < kDqWideUnroll; ++u)
        kv[u] = *reinterpret_cast<const uint4*>(kb16 + (start + kk[u]) * Di + 8 * dch);
#pragma unroll
      for (int u = 0; u < kDqWideUnroll; ++u) {
        if (!ok[u]) kv[u] = make_uint4(0u, 0u, 0u, 0u);
        wv[u] = ok[u] ? static_cast<double>(wf[u]) * scale : 0.0;
      }
#pragma unroll
      for (int u = 0; u < kDqWideUnroll; ++u) {
        const uint32_t x[4] = {kv[u].x, kv[u].y, kv[u].z, kv[u].w};
#pragma unroll
        for (int q2 = 0; q2 < 4; ++q2) {
          acc[2 * q2] = fma(wv[u], static_cast<double>(half_of<DT>(x[q2], 0)), acc[2 * q2]);
          acc[2 * q2 + 1] = fma(wv[u], static_cast<double>(half_of<DT>(x[q2], 1)), acc[2 * q2 + 1]);
        }
      }
    }
    __builtin_amdgcn_wave_barrier();  // list reused by the next chunk
    // exact ties of this chunk (rare), in block order: slot-0 lanes hold the sums they add to
    uint64_t tm = __ballot(my_tie < 0);
    while (tm) {
      const int i = __builtin_ctzll(tm);
      tm &= tm - 1;
      const float di = lane_f32(my_ds, i);
      const int64_t k0 = start + static_cast<int64_t>(b0 + i) * B;
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
          if (slot == 0) {
            const uint4 kw = *reinterpret_cast<const uint4*>(kb16 + (base + wl) * Di + 8 * dch);
            const uint32_t x[4] = {kw.x, kw.y, kw.z, kw.w};
#pragma unroll
            for (int q2 = 0; q2 < 4; ++q2) {
              acc[2 * q2] = fma(wgt, static_cast<double>(half_of<DT>(x[q2], 0)), acc[2 * q2]);
              acc[2 * q2 + 1] = fma(wgt, static_cast<double>(half_of<DT>(x[q2], 1)), acc[2 * q2 + 1]);
            }
          }
        }
      }
    }
  }
  // slot sums in slot order
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    double tot = 0.0;
#pragma unroll
    for (int sl = 0; sl < RPI; ++sl) tot += __shfl(acc[i], sl * LPR + dch, kWave);
    acc[i] = tot;
  }
  if (slot == 0) {
    uint32_t o[4];
#pragma unroll
    for (int q2 = 0; q2 < 4; ++q2)
      o[q2] = pack2<DT>(acc[2 * q2], acc[2 * q2 + 1]);
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(dq) + row * Di + 8 * dch) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// dk, partial sums. One workgroup per (key block gb, segment of kDkSeg rows, chunk of
// 128 keys). The segment's rows (t, g) of gb's sequence with t >= block start are
// read once (block-major tie / ds) and bucketed by their unique winner with a stable
// counting sort in LDS (per 64-row wave step the rank among equal winners comes from
// seven ballots on the winner's bits; waves are merged in order), so each key's rows
// stay in row order. Wave w then sums the keys w, w + 4, ...: lanes over dims, query
// rows streamed kDkBatch at a time, FP64 accumulation in row order; the segment's
// exact ties (rare) follow in row order. The sums go to
// part[((gb * nseg + sg) * kchunks + kc) * 128 + key][Di]; score_bwd_dk_reduce adds
// the segments in order.
// acc += w * q[row] over this lane's dims dbase .. dbase + DPL - 1.
template <int DT, int DPL>
__device__ __forceinline__ void dk_add_row(double (&acc)[8], double wgt, const void* __restrict__ iq, int64_t row,
                                           int Di, int dbase) {
#pragma unroll
  for (int j = 0; j < DPL; ++j) {
    const int d = dbase + j;
    if (d < Di) acc[j] = fma(wgt, static_cast<double>(load_as_f32<DT>(iq, row * Di + d)), acc[j]);
  }
}

constexpr int kDkSeg = 8192;
constexpr int kDkBatch = 16;
constexpr int kDkWideUnroll = 4;  // row-gather instructions per batch (4 rows each; two batches in flight)
// Listed exact ties per segment (a segment with more rescans its rows per key). With 4-instruction
// batches (131 VGPRs) and this list the pass fits three workgroups per CU (53 KB of LDS each):
// at c4 1.13-1.17 vs 1.21-1.24 ms for the score backward with two (8-instruction batches).
constexpr int kDkTieCap = 64;

template <int DT, int DPL>
__global__ __launch_bounds__(256, DPL >= 8 ? 2 : 3) void score_bwd_dk_part(
    const void* __restrict__ iq, const void* __restrict__ ik, const int32_t* __restrict__ cu,
    const int32_t* __restrict__ cu_blocks, int nseq, const int32_t* __restrict__ tie_t,
    const float* __restrict__ ds_t, int64_t rows, int G, int Di, int B, int64_t nblk, int nseg, double scale,
    double* __restrict__ part, int dc0) {
  __shared__ uint16_t lrow[kDkSeg];   // bucketed row offsets (within the segment)
  __shared__ float lds_w[kDkSeg];     // their ds
  __shared__ int32_t cnt[128], bstart[128];
  __shared__ int32_t wcnt[4][128];
  __shared__ int32_t tie_row[kDkTieCap];
  __shared__ double tie_best[kDkTieCap];
  __shared__ int32_t tie_count[kDkTieCap];
  __shared__ int32_t ntie_s;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  // Segments are aligned to multiples of kDkSeg in the row space: key block gb takes segment
  // S0 + sg, S0 = (its first row) / kDkSeg, clipped to its rows. Work L = workgroup index,
  // S-major over (S, key block): the workgroups running together gather from the same one or
  // two 2 MiB segments of index_q. Workgroups go to the 8 XCDs round-robin, so consecutive
  // pairs run on different XCDs (contiguous runs of L per XCD would load them unevenly: the
  // nonempty pairs are concentrated in the low segments at one long sequence).
  const int64_t nwork = nblk * nseg;
  const int64_t lw = blockIdx.x;
  if (lw >= nwork) return;  // whole workgroup (padding)
  const int64_t S = lw / nblk;
  const int64_t gb = lw % nblk;
  const int kc = blockIdx.y, kchunks = gridDim.y;
  int s = upper_index(cu_blocks, nseq + 1, gb);
  while (s < nseq && cu_blocks[s + 1] <= gb) ++s;
  const int b = static_cast<int>(gb - cu_blocks[s]);
  const int64_t start = cu[s], end = cu[s + 1];
  const int64_t k0 = start + static_cast<int64_t>(b) * B;
  const int64_t S0 = k0 * G / kDkSeg;
  if (S < S0) return;  // whole workgroup: the block starts after this segment
  const int sg = static_cast<int>(S - S0);
  const int64_t w = gb * nseg + sg;  // (gb, sg): index of this pair's partial sums
  const int64_t r_begin = S == S0 ? k0 * G : S * kDkSeg;
  const int64_t r_stop = (S + 1) * kDkSeg < end * G ? (S + 1) * kDkSeg : end * G;
  if (r_begin >= r_stop) return;  // whole workgroup: empty segment (the reduce skips it)
  const int o_lo = 128 * kc;      // this chunk's first key offset in the block
  const int nseg_rows = static_cast<int>(r_stop - r_begin);
  const int32_t* tcol = tie_t + static_cast<int64_t>(b) * rows + r_begin;
  const float* dcol = ds_t + static_cast<int64_t>(b) * rows + r_begin;
  // Stable counting sort by winner, one quarter of the segment per wave: wave w takes rows
  // kWaveRows w .. kWaveRows (w + 1) - 1 (row kWaveRows w + 64 r + lane in round r) and owns
  // the slice of every key's bucket after the slices of waves 0 .. w - 1. Each wave ranks its
  // rounds with ballots and advances its own counters, so the rounds need no workgroup
  // barrier, and every bucket still lists its rows in row order.
  constexpr int kWaveRows = kDkSeg / 4;
  constexpr int kRounds = kWaveRows / 64;
  if (tid < 128) wcnt[0][tid] = wcnt[1][tid] = wcnt[2][tid] = wcnt[3][tid] = 0;
  if (tid == 0) ntie_s = 0;
  // the wave's tie codes and ds, round r in register r: all loads in flight at once
  int32_t tcs[kRounds];
  float dvs[kRounds];
  const int wrow0 = kWaveRows * wid;
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int i = wrow0 + 64 * r + lane;
    tcs[r] = i < nseg_rows ? tcol[i] : 0;
    dvs[r] = i < nseg_rows ? dcol[i] : 0.f;
  }
  __syncthreads();
  // ---- per-wave histograms of winners in this key chunk; list the exact ties
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int32_t tc = tcs[r];
    const int o = tc - 1 - o_lo;
    if (tc > 0 && o >= 0 && o < 128) atomicAdd(&wcnt[wid][o], 1);
    if (tc < 0) {
      const int slot = atomicAdd(&ntie_s, 1);
      if (slot < kDkTieCap) tie_row[slot] = wrow0 + 64 * r + lane;
    }
  }
  __syncthreads();
  if (tid < 128) cnt[tid] = wcnt[0][tid] + wcnt[1][tid] + wcnt[2][tid] + wcnt[3][tid];
  __syncthreads();
  if (tid < 64) {  // exclusive scan of the 128 bucket counts (two per lane)
    const int a0 = cnt[2 * tid], a1 = cnt[2 * tid + 1];
    int x = a0 + a1;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x, o, kWave);
      if (lane >= o) x += y;
    }
    bstart[2 * tid] = x - a0 - a1;
    bstart[2 * tid + 1] = x - a1;
  }
  __syncthreads();
  if (tid < 128) {  // each wave's next free position in each bucket
    int p = bstart[tid];
#pragma unroll
    for (int w2 = 0; w2 < 4; ++w2) {
      const int n = wcnt[w2][tid];
      wcnt[w2][tid] = p;
      p += n;
    }
  }
  __syncthreads();
  // ---- stable scatter, 64 rows per round and wave (the wave's own counters only)
  const uint64_t lt = (uint64_t(1) << lane) - 1;
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    if (wrow0 + 64 * r >= nseg_rows) break;  // wave-uniform
    const int i = wrow0 + 64 * r + lane;
    const int32_t tc = tcs[r];  // 0 past the segment end
    const int o = tc - 1 - o_lo;
    const bool on = tc > 0 && o >= 0 && o < 128;
    uint64_t match = __ballot(on);
#pragma unroll
    for (int bit = 0; bit < 7; ++bit) {
      const uint64_t m = __ballot(on && ((o >> bit) & 1));
      match &= ((o >> bit) & 1) ? m : ~m;
    }
    const int rank = __popcll(match & lt);
    const int total = __popcll(match);
    if (on) {
      const int p = wcnt[wid][o] + rank;
      lrow[p] = static_cast<uint16_t>(i);
      lds_w[p] = dvs[r];
    }
    // all of the round's counter reads precede the advance (LDS operations of a wave run in order)
    __builtin_amdgcn_wave_barrier();
    if (on && rank == total - 1) wcnt[wid][o] += total;  // last lane of its group
    __builtin_amdgcn_wave_barrier();
  }
  __syncthreads();
  // ---- exact ties of the segment (rare): sort the listed rows, block maximum per row
  const int ntie = ntie_s < kDkTieCap ? ntie_s : kDkTieCap;
  const bool tie_overflow = ntie_s > kDkTieCap;
  if (ntie > 1 && tid == 0) {  // insertion sort: row order
    for (int x = 1; x < ntie; ++x) {
      const int v = tie_row[x];
      int y = x - 1;
      while (y >= 0 && tie_row[y] > v) {
        tie_row[y + 1] = tie_row[y];
        --y;
      }
      tie_row[y + 1] = v;
    }
  }
  __syncthreads();
  for (int x = wid; x < ntie; x += 4) {
    const int64_t row = r_begin + tie_row[x];
    const int64_t t = row / G;
    const int64_t k1 = (k0 + B < t + 1) ? k0 + B : t + 1;
    const BlockMax bm = block_max_exact<DT>(iq, row * Di, ik, k0, k1, Di, scale, lane);
    if (lane == 0) {
      tie_best[x] = bm.best;
      tie_count[x] = bm.count;
    }
  }
  __syncthreads();
  // ---- per-key sums: wave w takes keys w, w + 4, ... of this chunk
  const int64_t kchunk_end = k0 + B < end ? k0 + B : end;
  const int nkeys_c = static_cast<int>(kchunk_end - k0 - o_lo < 128 ? kchunk_end - k0 - o_lo : 128);
  if (wid >= nkeys_c) return;  // whole wave: no keys (no barrier follows)
  // exact ties: the key takes w / count of each tied row (row order) whose exact dot attains the maximum
  auto add_ties = [&](double (&acc)[8], int64_t key, int dbase, auto dpl) {
    constexpr int kDpl = decltype(dpl)::value;
    if (!tie_overflow) {
      for (int x = 0; x < ntie; ++x) {
        const int64_t row = r_begin + tie_row[x];
        if (key > row / G) continue;  // not visible from this row
        if (directed(exact_dot<DT>(iq, row * Di, ik, key * Di, Di), scale) != tie_best[x]) continue;
        const double wgt = static_cast<double>(dcol[tie_row[x]]) * scale / static_cast<double>(tie_count[x]);
        dk_add_row<DT, kDpl>(acc, wgt, iq, row, Di, dbase);
      }
    } else {
      // more ties than the list holds: rescan the segment in row order
      for (int i = 0; i < nseg_rows; ++i) {
        if (tcol[i] >= 0) continue;
        const int64_t row = r_begin + i;
        const int64_t t = row / G;
        if (key > t) continue;
        const int64_t k1 = (k0 + B < t + 1) ? k0 + B : t + 1;
        const BlockMax bm = block_max_exact<DT>(iq, row * Di, ik, k0, k1, Di, scale, lane);
        if (directed(exact_dot<DT>(iq, row * Di, ik, key * Di, Di), scale) != bm.best) continue;
        const double wgt = static_cast<double>(dcol[i]) * scale / static_cast<double>(bm.count);
        dk_add_row<DT, kDpl>(acc, wgt, iq, row, Di, dbase);
      }
    }
  };
  if ((DT != kF32) && Di == 128) {
    // 128-dim 2-byte rows: lane (slot, dch) reads 16 bytes (dims 8 dch .. +7) of entry slot of
    // every 4, i.e. 4 rows per load instruction. A key's entries go in batches of kDkWideUnroll
    // load instructions; the next batch (of the same key or of the wave's next key) is loaded
    // while one is summed. Each batch issues all of its loads (entries past the key's end read
    // the segment's first row and are not added), so the wait for a batch leaves the next
    // batch's loads in flight.
    constexpr int kLpr = 16, kRpi = 4, kSpan = kDkWideUnroll * kRpi;
    const int slot = lane / kLpr, dch = lane % kLpr;
    const uint16_t* q16 = static_cast<const uint16_t*>(iq);
    struct Batch {
      int o, e, kend;
    };
    auto first_of = [&](int o) {  // wave-uniform: kept in scalar registers
      const int e = __builtin_amdgcn_readfirstlane(bstart[o]);
      return Batch{o, e, e + __builtin_amdgcn_readfirstlane(cnt[o])};
    };
    auto next_of = [&](const Batch& x) {
      Batch y{x.o, x.e + kSpan, x.kend};
      if (y.e >= y.kend) {
        y.o = x.o + 4;
        y = y.o < nkeys_c ? first_of(y.o) : Batch{y.o, 0, 0};
      }
      return Batch{__builtin_amdgcn_readfirstlane(y.o), __builtin_amdgcn_readfirstlane(y.e),
                   __builtin_amdgcn_readfirstlane(y.kend)};
    };
    auto issue = [&](const Batch& x, uint4 (&qw)[kDkWideUnroll], float (&wf)[kDkWideUnroll]) {
      int ro[kDkWideUnroll];
#pragma unroll
      for (int u = 0; u < kDkWideUnroll; ++u) {
        const int ee = x.e + u * kRpi + slot;
        const int ec = ee < kDkSeg ? ee : kDkSeg - 1;  // always inside the list (value unused past the key)
        const int r = lrow[ec];
        const float wv = lds_w[ec];
        const bool ok = ee < x.kend;
        ro[u] = ok ? r : 0;
        wf[u] = ok ? wv : 0.f;
      }
#pragma unroll
      for (int u = 0; u < kDkWideUnroll; ++u)
        qw[u] = *reinterpret_cast<const uint4*>(q16 + (r_begin + ro[u]) * 128 + 8 * dch);
    };
    double acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.0;
    auto consume = [&](const Batch& x, const uint4 (&qw)[kDkWideUnroll], const float (&wf)[kDkWideUnroll]) {
#pragma unroll
      for (int u = 0; u < kDkWideUnroll; ++u) {
        if (x.e + u * kRpi >= x.kend) break;  // wave-uniform
        const double wv = x.e + u * kRpi + slot < x.kend ? static_cast<double>(wf[u]) * scale : 0.0;
        const uint32_t w4[4] = {qw[u].x, qw[u].y, qw[u].z, qw[u].w};
#pragma unroll
        for (int q2 = 0; q2 < 4; ++q2) {
          acc[2 * q2] = fma(wv, static_cast<double>(half_of<DT>(w4[q2], 0)), acc[2 * q2]);
          acc[2 * q2 + 1] = fma(wv, static_cast<double>(half_of<DT>(w4[q2], 1)), acc[2 * q2 + 1]);
        }
      }
      if (x.e + kSpan >= x.kend) {  // the key's last batch: slot sums in slot order, ties, store
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          double tot = 0.0;
#pragma unroll
          for (int sl = 0; sl < kRpi; ++sl) tot += __shfl(acc[j], sl * kLpr + dch, kWave);
          acc[j] = tot;
        }
        if (ntie > 0 || tie_overflow) add_ties(acc, k0 + o_lo + x.o, 8 * dch, std::integral_constant<int, 8>{});
        if (slot == 0) {
          double* dst = part + ((w * kchunks + kc) * 128 + x.o) * static_cast<int64_t>(Di) + 8 * dch;
#pragma unroll
          for (int j = 0; j < 8; ++j) dst[j] = acc[j];
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = 0.0;
      }
    };
    uint4 qa[kDkWideUnroll], qb[kDkWideUnroll];
    float wa[kDkWideUnroll], wb[kDkWideUnroll];
    Batch x0 = first_of(wid);
    issue(x0, qa, wa);
    for (;;) {
      const Batch x1 = next_of(x0);
      issue(x1, qb, wb);
      consume(x0, qa, wa);
      if (x1.o >= nkeys_c) break;
      const Batch x2 = next_of(x1);
      issue(x2, qa, wa);
      consume(x1, qb, wb);
      if (x2.o >= nkeys_c) break;
      x0 = x2;
    }
    return;
  }
  // other dtypes / dims: lanes over dims dc0 + DPL lane .. + DPL - 1 (index dims above 64 x DPL
  // take one launch per 64 DPL dims), query rows streamed kDkBatch at a time
  const int dbase = dc0 + DPL * lane;
  for (int o = wid; o < nkeys_c; o += 4) {
    const int64_t key = k0 + o_lo + o;
    double acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.0;
    const int e0 = bstart[o], e1 = e0 + cnt[o];
    for (int e = e0; e < e1; e += kDkBatch) {
      float qv[kDkBatch][DPL];
#pragma unroll
      for (int u = 0; u < kDkBatch; ++u) {
        const int64_t row = r_begin + lrow[e + u < e1 ? e + u : e0];
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          const int d = dbase + j;
          qv[u][j] = (e + u < e1 && d < Di) ? load_as_f32<DT>(iq, row * Di + d) : 0.f;
        }
      }
#pragma unroll
      for (int u = 0; u < kDkBatch; ++u) {
        if (e + u < e1) {
          const double wgt = static_cast<double>(lds_w[e + u]) * scale;
#pragma unroll
          for (int j = 0; j < DPL; ++j) acc[j] = fma(wgt, static_cast<double>(qv[u][j]), acc[j]);
        }
      }
    }
    add_ties(acc, key, dbase, std::integral_constant<int, DPL>{});
    double* dst = part + ((w * kchunks + kc) * 128 + o) * static_cast<int64_t>(Di);
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      const int d = dbase + j;
      if (d < Di) dst[d] = acc[j];
    }
  }
}

// dk[key][d] = sum over the key block's row segments (in order) of the partial sums.
template <int DT>
__global__ __launch_bounds__(256) void score_bwd_dk_reduce(const int32_t* __restrict__ cu,
                                                           const int32_t* __restrict__ cu_blocks, int nseq,
                                                           int64_t T, int G, int Di, int B, int nseg,
                                                           const double* __restrict__ part,
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
  const int kc = o / 128, kchunks = (B + 127) / 128;
  const int64_t S0 = k0 * G / kDkSeg;  // the block's first segment (aligned to kDkSeg rows)
  double sum = 0.0;
  for (int sg = 0; sg < nseg; ++sg) {
    if ((S0 + sg) * kDkSeg >= end * G) break;  // empty segment (nothing written)
    const int64_t w = gb * nseg + sg;
    sum += part[((w * kchunks + kc) * 128 + o % 128) * static_cast<int64_t>(Di) + d];
  }
  store_from_f64<DT>(dk, i, sum);
}

static int64_t dk_nseg(int64_t rows) { return (rows + kDkSeg - 1) / kDkSeg; }

template <int DT>
int score_fwd_launch(const void* iq, const void* ik, const int32_t* cu, int nseq, int64_t rows, int G,
                     int Di, int NB, int B, double scale, float* scores, int32_t* tie, int K, int L, int32_t* sel,
                     void* ws, hipStream_t st) {
  // sel != null: the top-k selection follows on the same stream (topk.hip). Selecting
  // inside the MFMA kernel's tiles, from the scores just written, was measured slower
  // at c4 (2.43-2.81 ms vs 2.27 ms for the two launches): the score kernel runs two
  // workgroups per CU and the selection's registers cost its main loop.
  if (DT == kBF16 && score_mfma_supported(Di, B, scale)) {
    const int rc = score_fwd_mfma_launch(iq, ik, cu, nseq, rows, G, Di, NB, B, scale, scores, tie, ws, st);
    if (rc != kOk || !sel) return rc;
    return topk_launch(scores, cu, nseq, rows, G, NB, B, K, L, sel, st);
  }
  const int64_t waves = rows * NB;
  hipLaunchKernelGGL(score_fwd_exact<DT>, dim3(grid_1d(waves, 4)), dim3(256), 0, st, iq, ik, cu, nseq, rows,
                     G, Di, NB, B, scale, scores, tie);
  const int rc = status_from(hipGetLastError());
  if (rc != kOk || !sel) return rc;
  return topk_launch(scores, cu, nseq, rows, G, NB, B, K, L, sel, st);
}

template <int DT>
int score_bwd_launch(const void* iq, const void* ik, const int32_t* cu, const int32_t* cu_blocks, int nseq,
                     const int32_t* tie, const float* ds, int64_t rows, int G, int Di, int NB, int B,
                     int64_t total_blocks, double scale, void* dq, void* dk, void* ws, hipStream_t st) {
  if (dq && DT != kF32 && (Di == 32 || Di == 64 || Di == 128)) {
    const dim3 grid(grid_1d(rows, 4)), block(256);
    switch (Di / 8) {
      case 4: hipLaunchKernelGGL((score_bwd_dq_wide<DT, 4>), grid, block, 0, st, iq, ik, cu, nseq, tie, ds, rows, G, Di, NB, B, scale, dq); break;
      case 8: hipLaunchKernelGGL((score_bwd_dq_wide<DT, 8>), grid, block, 0, st, iq, ik, cu, nseq, tie, ds, rows, G, Di, NB, B, scale, dq); break;
      default: hipLaunchKernelGGL((score_bwd_dq_wide<DT, 16>), grid, block, 0, st, iq, ik, cu, nseq, tie, ds, rows, G, Di, NB, B, scale, dq); break;
    }
  } else if (dq) {
    const dim3 grid(grid_1d(rows, 4)), block(256);
    if (Di <= 64) hipLaunchKernelGGL((score_bwd_dq<DT, 1>), grid, block, 0, st, iq, ik, cu, nseq, tie, ds, rows, G, Di, NB, B, scale, dq, 0);
    else if (Di <= 128) hipLaunchKernelGGL((score_bwd_dq<DT, 2>), grid, block, 0, st, iq, ik, cu, nseq, tie, ds, rows, G, Di, NB, B, scale, dq, 0);
    else if (Di <= 256) hipLaunchKernelGGL((score_bwd_dq<DT, 4>), grid, block, 0, st, iq, ik, cu, nseq, tie, ds, rows, G, Di, NB, B, scale, dq, 0);
    else
      for (int dc0 = 0; dc0 < Di; dc0 += 512)
        hipLaunchKernelGGL((score_bwd_dq<DT, 8>), grid, block, 0, st, iq, ik, cu, nseq, tie, ds, rows, G, Di, NB, B, scale, dq, dc0);
  }
  if (dk && total_blocks > 0) {
    int32_t* tie_t = static_cast<int32_t*>(ws);
    float* ds_t = reinterpret_cast<float*>(tie_t + rows * NB);
    double* part = reinterpret_cast<double*>(ds_t + rows * NB);  // 8 * rows * NB bytes in: 8-byte aligned
    const dim3 tgrid(grid_1d(rows, 64), static_cast<unsigned>((NB + 63) / 64));
    hipLaunchKernelGGL(score_bwd_transpose, tgrid, dim3(256), 0, st, tie, ds, rows, NB, cu, nseq, G, B, tie_t, ds_t);
    const int nseg = static_cast<int>(dk_nseg(rows));
    const int kchunks = (B + 127) / 128;
    const dim3 grid(static_cast<unsigned>(total_blocks * nseg), static_cast<unsigned>(kchunks));
#define MSA_DK_PART(DPLV, DC0) hipLaunchKernelGGL((score_bwd_dk_part<DT, DPLV>), grid, dim3(256), 0, st, iq, ik, cu, cu_blocks, nseq, tie_t, ds_t, rows, G, Di, B, total_blocks, nseg, scale, part, DC0)
    if (Di <= 64) MSA_DK_PART(1, 0);
    else if (Di <= 128) MSA_DK_PART(2, 0);
    else if (Di <= 256) MSA_DK_PART(4, 0);
    else
      for (int dc0 = 0; dc0 < Di; dc0 += 512) MSA_DK_PART(8, dc0);
#undef MSA_DK_PART
    const int64_t T = rows / G;
    hipLaunchKernelGGL(score_bwd_dk_reduce<DT>, dim3(grid_1d(T * Di, 256)), dim3(256), 0, st, cu, cu_blocks, nseq, T,
                       G, Di, B, nseg, part, dk);
  }
  return status_from(hipGetLastError());
}

}  // namespace msa

using namespace msa;

extern "C" int64_t msa_score_fwd_workspace_bytes(int64_t total_tokens, int64_t groups, int64_t num_blocks) {
  if (total_tokens < 0 || groups <= 0 || num_blocks <= 0) return 0;
  return score_fwd_mfma_workspace_bytes(total_tokens, total_tokens * groups, num_blocks);
}

extern "C" int msa_score_fwd(const void* index_q, const void* index_k, int32_t dtype,
                             const int32_t* cu_seqlens, int64_t num_seqs, int64_t total_tokens,
                             int64_t groups, int64_t index_dim, int64_t num_blocks, int64_t block_size,
                             double scale, float* scores, int32_t* tie_info, void* workspace, void* stream) {
  if (num_seqs <= 0 || total_tokens < 0 || groups <= 0 || index_dim <= 0 || num_blocks <= 0 ||
      block_size <= 0)
    return kErrInvalidArgument;
  const int64_t rows = total_tokens * groups;
  if (rows == 0) return kOk;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int nseq = static_cast<int>(num_seqs), G = static_cast<int>(groups);
  const int Di = static_cast<int>(index_dim), NB = static_cast<int>(num_blocks);
  const int B = static_cast<int>(block_size);
  switch (dtype) {
    case kF32: return score_fwd_launch<kF32>(index_q, index_k, cu_seqlens, nseq, rows, G, Di, NB, B, scale, scores, tie_info, 0, 0, nullptr, workspace, st);
    case kF16: return score_fwd_launch<kF16>(index_q, index_k, cu_seqlens, nseq, rows, G, Di, NB, B, scale, scores, tie_info, 0, 0, nullptr, workspace, st);
    case kBF16: return score_fwd_launch<kBF16>(index_q, index_k, cu_seqlens, nseq, rows, G, Di, NB, B, scale, scores, tie_info, 0, 0, nullptr, workspace, st);
    default: return kErrInvalidArgument;
  }
}

extern "C" int msa_index_score_topk(const void* index_q, const void* index_k, int32_t dtype,
                                    const int32_t* cu_seqlens, int64_t num_seqs, int64_t total_tokens,
                                    int64_t groups, int64_t index_dim, int64_t num_blocks, int64_t block_size,
                                    double scale, int64_t topk_blocks, int64_t local_blocks, float* scores,
                                    int32_t* tie_info, int32_t* indices, void* workspace, void* stream) {
  if (num_seqs <= 0 || total_tokens < 0 || groups <= 0 || index_dim <= 0 || num_blocks <= 0 ||
      block_size <= 0 || topk_blocks < 0 || local_blocks < 0 || local_blocks > topk_blocks ||
      (topk_blocks > 0 && !indices))
    return kErrInvalidArgument;
  const int64_t rows = total_tokens * groups;
  if (rows == 0) return kOk;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int nseq = static_cast<int>(num_seqs), G = static_cast<int>(groups);
  const int Di = static_cast<int>(index_dim), NB = static_cast<int>(num_blocks);
  const int B = static_cast<int>(block_size), K = static_cast<int>(topk_blocks);
  const int L = static_cast<int>(local_blocks);
  int32_t* sel = K > 0 ? indices : nullptr;
  switch (dtype) {
    case kF32: return score_fwd_launch<kF32>(index_q, index_k, cu_seqlens, nseq, rows, G, Di, NB, B, scale, scores, tie_info, K, L, sel, workspace, st);
    case kF16: return score_fwd_launch<kF16>(index_q, index_k, cu_seqlens, nseq, rows, G, Di, NB, B, scale, scores, tie_info, K, L, sel, workspace, st);
    case kBF16: return score_fwd_launch<kBF16>(index_q, index_k, cu_seqlens, nseq, rows, G, Di, NB, B, scale, scores, tie_info, K, L, sel, workspace, st);
    default: return kErrInvalidArgument;
  }
}

extern "C" int64_t msa_score_bwd_workspace_bytes(int64_t total_tokens, int64_t groups, int64_t num_blocks,
                                                 int64_t index_dim, int64_t block_size, int64_t total_blocks) {
  if (total_tokens <= 0 || groups <= 0 || num_blocks <= 0 || index_dim <= 0 || block_size <= 0) return 256;
  const int64_t rows = total_tokens * groups;
  // block-major tie / ds copies, then the dk partial sums (FP64)
  const int64_t tr = rows * num_blocks * 8 + 8;
  const int64_t nseg = dk_nseg(rows);
  const int64_t kchunks = (block_size + 127) / 128;
  const int64_t part = total_blocks * nseg * kchunks * 128 * index_dim * 8;
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
