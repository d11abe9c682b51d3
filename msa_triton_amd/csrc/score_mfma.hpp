// Exact FP64 evaluation helpers for the indexer score, shared by the exact
// kernel, the MFMA kernel's certification step and the backward tie paths.
//
// All exact dots use ONE summation order -- two sequential FMA chains over the
// halves [0, h) and [h, n) of the index dim (h = n/2), added at the end -- so
// every kernel that re-evaluates a (query, key) dot reproduces the same FP64
// bits and tie membership is consistent between forward and backward. (For
// bf16/fp16 inputs the FP64 sum is exact in practice, so the order only matters
// in pathological exponent ranges.)
#pragma once
#include "common.hpp"

namespace msa {

struct BlockMax {
  double best;  // directed exact max (sign(scale) * dot), 0 when scale == 0
  int count;    // number of keys attaining it
  int first;    // smallest key offset (from the block start) attaining it
};

__device__ __forceinline__ double directed(double dot, double scale) {
  return scale > 0.0 ? dot : (scale < 0.0 ? -dot : 0.0);
}

// The public score of a block whose directed exact maximum is x, as the reference
// publishes it (triton/index_score.py:121-127, FP32 arithmetic without fused
// multiply-add): the FP32 pair hi = fl32(x), lo = fl32(x - hi) of the winning dot, each
// times s = fl32(|scale|), added in FP32. For |scale| = 1 (and 0) that is fl32(x); for
// other scales it can differ from fl32(|scale| x) by one ulp (two roundings). x = -inf
// (no finite visible dot) or an x beyond the FP32 range gives fl32(x) s.
__device__ __forceinline__ float public_score(double x, float s) {
#pragma clang fp contract(off)  // two products and a sum, each rounded (HIP contracts by default)
  const float hi = static_cast<float>(x);
  if (!__builtin_isfinite(hi)) return __fmul_rn(hi, s);
  const float lo = static_cast<float>(x - static_cast<double>(hi));  // x - hi is exact in FP64
  return hi * s + lo * s;
}

template <int DT>
__device__ __forceinline__ double exact_half_dot(const void* __restrict__ a, int64_t ia,
                                                 const void* __restrict__ b, int64_t ib, int d0, int d1) {
  double acc = 0.0;
  for (int d = d0; d < d1; ++d)
    acc = fma(static_cast<double>(load_as_f32<DT>(a, ia + d)), static_cast<double>(load_as_f32<DT>(b, ib + d)), acc);
  return acc;
}

template <int DT>
__device__ __forceinline__ double exact_dot(const void* __restrict__ a, int64_t ia,
                                            const void* __restrict__ b, int64_t ib, int n) {
  const int h = n / 2;
  return exact_half_dot<DT>(a, ia, b, ib, 0, h) + exact_half_dot<DT>(a, ia, b, ib, h, n);
}

// Wave-cooperative exact block max over keys [k0, k1) for query row offset qoff.
template <int DT>
__device__ BlockMax block_max_exact(const void* __restrict__ iq, int64_t qoff, const void* __restrict__ ik,
                                    int64_t k0, int64_t k1, int Di, double scale, int lane) {
  double best = -__builtin_inf();
  int count = 0, first = 0x7fffffff;
  for (int64_t kk = k0 + lane; kk < k1; kk += kWave) {
    const double v = directed(exact_dot<DT>(iq, qoff, ik, kk * Di, Di), scale);
    if (v > best) {
      best = v;
      count = 1;
      first = static_cast<int>(kk - k0);
    } else if (v == best) {  // also a first key whose dot is -inf (NaN dots are skipped)
      if (count == 0) first = static_cast<int>(kk - k0);
      ++count;
    }
  }
  const double wbest = wave_max_f64(best);
  const bool on = (best == wbest) && count > 0;
  BlockMax r;
  r.best = wbest;
  r.count = wave_sum_i32(on ? count : 0);
  int f = on ? first : 0x7fffffff;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) f = min(f, __shfl_xor(f, o, kWave));
  r.first = f;
  return r;
}

// Calls fn(key) for each key in [k0, k1) whose directed exact dot equals best,
// in ascending key order (uniform control flow across the wave).
template <int DT, typename Fn>
__device__ void for_each_winner(const void* __restrict__ iq, int64_t qoff, const void* __restrict__ ik,
                                int64_t k0, int64_t k1, int Di, double scale, double best, int lane, Fn fn) {
  for (int64_t base = k0; base < k1; base += kWave) {
    const int64_t kk = base + lane;
    bool win = false;
    if (kk < k1) win = directed(exact_dot<DT>(iq, qoff, ik, kk * Di, Di), scale) == best;
    uint64_t mask = __ballot(win);
    while (mask) {
      const int i = __builtin_ctzll(mask);
      mask &= mask - 1;
      fn(base + i);
    }
  }
}

// MFMA score path (bf16). Declared here, defined in score_mfma.hip.
bool score_mfma_supported(int Di, int B, double scale);
int64_t score_fwd_mfma_workspace_bytes(int64_t total_tokens, int64_t rows, int64_t NB);
int score_fwd_mfma_launch(const void* iq, const void* ik, const int32_t* cu, int nseq, int64_t rows, int G,
                          int Di, int NB, int B, double scale, float* scores, int32_t* tie, void* ws,
                          hipStream_t st);

}  // namespace msa
