// Stage 1 on MFMA (bf16 inputs): block maxima of the indexer logits with a
// certified exact winner.
//
// Work unit: a tile of 128 consecutive (t, g) rows of the flattened [T*G] row
// space; the tile's query fragments stay in registers for its whole lifetime.
// For every key block reachable by the tile's rows, the 4 waves each take 32 of
// the block's (<= 128) keys and evaluate the 128 x 32 logits on
// v_mfma_f32_16x16x32_bf16 (exact bf16 products, fp32 accumulation).
//
// Exactness (the public score must equal fl32(scale * exact winning dot) and
// the winner set must be the exact one, index_score.py:121-136): with
//   E = (Di_pad + 8) * 2^-22 * ||q|| * max_k ||k||  >=  |s_mfma - s_exact|,
// every key whose approximate directed logit is below (max_approx - 2E) is
// certainly beaten by the approximate winner. If exactly one key survives,
// it is the unique exact winner and only its dot is evaluated in FP64 (from LDS
// copies of the tile rows and the key block, in the fixed summation order of
// exact_dot). Otherwise the row takes the slow path: every key of the block is
// re-evaluated in FP64 and max / tie count / first winner are taken exactly.
#include "mfma_util.hpp"
#include "score_mfma.hpp"

namespace msa {

namespace {

constexpr int kTileRows = 128;

template <int NK>
struct ScoreSmem {
  static constexpr int DP = 32 * NK;
  static constexpr int RS = DP + 8;
  uint16_t q[kTileRows * RS];  // tile rows, raw bf16 (not sign-flipped)
  uint16_t k[kTileRows * RS];  // current key block, raw bf16
  float wmax[4][kTileRows];    // per-wave approximate row maximum
  int widx[4][kTileRows];      // per-wave approximate argmax (key offset in block)
  int wcnt[4][kTileRows];      // per-wave number of candidates
  float kmax2[4];              // per-wave max key norm^2
  float qnorm[kTileRows];
  int qb[kTileRows];           // query block of each row (-1 if no row)
  int seq_of[kTileRows];       // sequence of each row
  double half[kTileRows];      // second-half partial dots
  int slow[kTileRows];
  int nslow;
  double red_v[4];
  int red_c[4];
  int red_f[4];
};

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Half-dot over dims [d0, d1) of two LDS rows, sequential FMA (exact_dot order).
__device__ __forceinline__ double lds_half_dot(const uint16_t* a, const uint16_t* b, int d0, int d1) {
  double acc = 0.0;
  for (int d = d0; d < d1; ++d)
    acc = fma(static_cast<double>(bf16_bits_to_f32(a[d])), static_cast<double>(bf16_bits_to_f32(b[d])), acc);
  return acc;
}

}  // namespace

template <int NK>
__global__ __launch_bounds__(256) void score_fwd_mfma_kernel(const uint16_t* __restrict__ iq,
                                                             const uint16_t* __restrict__ ik,
                                                             const int32_t* __restrict__ cu, int nseq, int64_t rows,
                                                             int G, int Di, int NB, int B, double scale,
                                                             float* __restrict__ scores, int32_t* __restrict__ tie) {
  constexpr int DP = 32 * NK, RS = ScoreSmem<NK>::RS;
  __shared__ ScoreSmem<NK> sm;
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63, c = lane & 15, q4 = lane >> 4;
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * kTileRows;
  const int nr = static_cast<int>(rows - r0 < kTileRows ? rows - r0 : kTileRows);
  const bool neg = scale < 0.0;
  const double ascale = fabs(scale);
  const float cerr = static_cast<float>(DP + 8) * 0x1p-22f;

  // ---- stage the tile rows (raw) and per-row metadata
  for (int e = tid; e < kTileRows * (DP / 8); e += 256) {
    const int rr = e / (DP / 8), d0 = 8 * (e % (DP / 8));
    uint4 val = make_uint4(0u, 0u, 0u, 0u);
    if (rr < nr && d0 < Di) val = *reinterpret_cast<const uint4*>(iq + (r0 + rr) * Di + d0);
    *reinterpret_cast<uint4*>(sm.q + rr * RS + d0) = val;
  }
  if (tid < kTileRows) {
    if (tid < nr) {
      const int64_t t = (r0 + tid) / G;
      const int s = find_seq(cu, nseq, t);
      sm.seq_of[tid] = s;
      sm.qb[tid] = static_cast<int>((t - cu[s]) / B);
    } else {
      sm.seq_of[tid] = -1;
      sm.qb[tid] = -1;
    }
  }
  if (tid == 0) sm.nslow = 0;
  __syncthreads();
  if (tid < kTileRows) {
    float s2 = 0.f;
    for (int d = 0; d < Di; ++d) {
      const float x = bf16_bits_to_f32(sm.q[tid * RS + d]);
      s2 = fmaf(x, x, s2);
    }
    sm.qnorm[tid] = sqrtf(s2) * 1.0001f;
  }
  // B-operand fragments of the tile rows: row 16*rt + c, dims 32*kk + 8*q4 (sign-flipped if scale < 0).
  bf16x8 qf[8][NK];
#pragma unroll
  for (int rt = 0; rt < 8; ++rt)
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) {
      uint4 w = *reinterpret_cast<const uint4*>(sm.q + (16 * rt + c) * RS + 32 * kk + 8 * q4);
      if (neg) {
        w.x ^= 0x80008000u;
        w.y ^= 0x80008000u;
        w.z ^= 0x80008000u;
        w.w ^= 0x80008000u;
      }
      qf[rt][kk] = __builtin_bit_cast(bf16x8, w);
    }

  const int64_t t_first = r0 / G, t_last = (r0 + nr - 1) / G;
  for (int s = find_seq(cu, nseq, t_first); s < nseq && cu[s] <= t_last; ++s) {
    const int64_t start = cu[s], end = cu[s + 1];
    const int64_t ra = start * G > r0 ? start * G : r0;
    const int64_t rb = end * G < r0 + nr ? end * G : r0 + nr;
    if (ra >= rb) continue;
    const int qb_last = static_cast<int>(((rb - 1) / G - start) / B);
    for (int b = 0; b <= qb_last; ++b) {
      const int64_t kb = start + static_cast<int64_t>(b) * B;
      const int nk = static_cast<int>(end - kb < B ? end - kb : B);
      __syncthreads();  // previous block's LDS consumers are done
      // ---- this wave's 32 keys: offsets 32*wid + 16*kt + c
      bf16x8 kf[2][NK];
      float kn2 = 0.f;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const int kl = 32 * wid + 16 * kt + c;
        float part = 0.f;
#pragma unroll
        for (int kk = 0; kk < NK; ++kk) {
          const int d0 = 32 * kk + 8 * q4;
          uint4 w = make_uint4(0u, 0u, 0u, 0u);
          if (kl < nk && d0 < Di) w = *reinterpret_cast<const uint4*>(ik + (kb + kl) * Di + d0);
          *reinterpret_cast<uint4*>(sm.k + kl * RS + d0) = w;
          kf[kt][kk] = __builtin_bit_cast(bf16x8, w);
          const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            part = fmaf(bf16_lo(ws[j]), bf16_lo(ws[j]), part);
            part = fmaf(bf16_hi(ws[j]), bf16_hi(ws[j]), part);
          }
        }
        part += __shfl_xor(part, 16, kWave);
        part += __shfl_xor(part, 32, kWave);
        kn2 = fmaxf(kn2, part);
      }
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) kn2 = fmaxf(kn2, __shfl_xor(kn2, o, kWave));
      if (lane == 0) sm.kmax2[wid] = kn2 * 1.0001f;
      // ---- logits: C[key 16*kt + 4*q4 + i][row 16*rt + c]
      f32x4 acc[8][2];
#pragma unroll
      for (int rt = 0; rt < 8; ++rt)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
          f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kk = 0; kk < NK; ++kk) a = mfma(kf[kt][kk], qf[rt][kk], a);
          acc[rt][kt] = a;
        }
      // ---- per-row approximate max / argmax over this wave's keys
      bool rowok[8];
      int64_t trow[8];
#pragma unroll
      for (int rt = 0; rt < 8; ++rt) {
        const int rr = 16 * rt + c;
        const int64_t r = r0 + rr;
        rowok[rt] = r >= ra && r < rb && sm.qb[rr] >= b;
        trow[rt] = r / G;
        float m = -__builtin_inff();
        int idx = 0x7fffffff;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int kl = 32 * wid + 16 * kt + 4 * q4 + i;
            const bool ok = rowok[rt] && kl < nk && kb + kl <= trow[rt];
            const float v = ok ? acc[rt][kt][i] : -__builtin_inff();
            if (v > m) {
              m = v;
              idx = kl;
            }
          }
#pragma unroll
        for (int o = 16; o <= 32; o <<= 1) {
          const float om = __shfl_xor(m, o, kWave);
          const int oi = __shfl_xor(idx, o, kWave);
          if (om > m || (om == m && oi < idx)) {
            m = om;
            idx = oi;
          }
        }
        if (q4 == 0) {
          sm.wmax[wid][rr] = m;
          sm.widx[wid][rr] = idx;
        }
      }
      __syncthreads();
      // ---- candidates within 2E of the row maximum
      const float kmax = sqrtf(fmaxf(fmaxf(sm.kmax2[0], sm.kmax2[1]), fmaxf(sm.kmax2[2], sm.kmax2[3])));
#pragma unroll
      for (int rt = 0; rt < 8; ++rt) {
        const int rr = 16 * rt + c;
        const float gm = fmaxf(fmaxf(sm.wmax[0][rr], sm.wmax[1][rr]), fmaxf(sm.wmax[2][rr], sm.wmax[3][rr]));
        const float thr = gm - 2.f * cerr * sm.qnorm[rr] * kmax;
        int cnt = 0;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int kl = 32 * wid + 16 * kt + 4 * q4 + i;
            const bool ok = rowok[rt] && kl < nk && kb + kl <= trow[rt];
            cnt += (ok && acc[rt][kt][i] >= thr) ? 1 : 0;
          }
        cnt += __shfl_xor(cnt, 16, kWave);
        cnt += __shfl_xor(cnt, 32, kWave);
        if (q4 == 0) sm.wcnt[wid][rr] = cnt;
      }
      __syncthreads();
      // ---- resolve rows: 2 threads per row evaluate the two halves of the winner's exact dot
      const int rr = tid & (kTileRows - 1);
      const int half = tid >> 7;
      const int64_t r = r0 + rr;
      const bool valid = r >= ra && r < rb && sm.qb[rr] >= b;
      const int h = Di / 2;
      int winner = -1;
      bool unique = false;
      if (valid) {
        float gm = sm.wmax[0][rr];
        int gw = 0;
#pragma unroll
        for (int w = 1; w < 4; ++w)
          if (sm.wmax[w][rr] > gm) {
            gm = sm.wmax[w][rr];
            gw = w;
          }
        const int total = sm.wcnt[0][rr] + sm.wcnt[1][rr] + sm.wcnt[2][rr] + sm.wcnt[3][rr];
        unique = total == 1;
        winner = sm.widx[gw][rr];
        if (unique && half == 1) sm.half[rr] = lds_half_dot(sm.q + rr * RS, sm.k + winner * RS, h, Di);
      }
      __syncthreads();
      if (half == 0 && valid) {
        if (unique) {
          const double dot = lds_half_dot(sm.q + rr * RS, sm.k + winner * RS, 0, h) + sm.half[rr];
          const double dv = neg ? -dot : dot;
          scores[r * NB + b] = static_cast<float>(ascale * dv);
          if (tie) tie[r * NB + b] = winner + 1;
        } else {
          sm.slow[atomicAdd(&sm.nslow, 1)] = rr;
        }
      }
      __syncthreads();
      // ---- slow path: exact evaluation of every key of the block for the listed rows
      const int nslow = sm.nslow;
      for (int si = 0; si < nslow; ++si) {
        const int sr = sm.slow[si];
        const int64_t srow = r0 + sr;
        const int64_t st = srow / G;
        double v = -__builtin_inf();
        int idx = 0x7fffffff;
        if (tid < nk && kb + tid <= st) {
          const double dot = lds_half_dot(sm.q + sr * RS, sm.k + tid * RS, 0, h) +
                             lds_half_dot(sm.q + sr * RS, sm.k + tid * RS, h, Di);
          v = neg ? -dot : dot;
          idx = tid;
        }
        const double wbest = wave_max_f64(v);
        int wc = wave_sum_i32((v == wbest && idx != 0x7fffffff) ? 1 : 0);
        int wf = (v == wbest) ? idx : 0x7fffffff;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) wf = min(wf, __shfl_xor(wf, o, kWave));
        if (lane == 0) {
          sm.red_v[wid] = wbest;
          sm.red_c[wid] = wc;
          sm.red_f[wid] = wf;
        }
        __syncthreads();
        if (tid == 0) {
          double best = sm.red_v[0];
          for (int w = 1; w < 4; ++w) best = fmax(best, sm.red_v[w]);
          int count = 0, first = 0x7fffffff;
          for (int w = 0; w < 4; ++w)
            if (sm.red_v[w] == best) {
              count += sm.red_c[w];
              first = min(first, sm.red_f[w]);
            }
          scores[srow * NB + b] = static_cast<float>(ascale * best);
          if (tie) tie[srow * NB + b] = count == 1 ? first + 1 : -count;
        }
        __syncthreads();
      }
      if (tid == 0) sm.nslow = 0;
    }
  }
  // ---- blocks without a causal key: -inf, tie code 0
  for (int e = tid; e < kTileRows * NB; e += 256) {
    const int rr2 = e / NB, b = e % NB;
    if (rr2 < nr && b > sm.qb[rr2]) {
      scores[(r0 + rr2) * NB + b] = -__builtin_inff();
      if (tie) tie[(r0 + rr2) * NB + b] = 0;
    }
  }
}

bool score_mfma_supported(int Di, int B, double scale) {
  return scale != 0.0 && Di >= 8 && Di <= 128 && Di % 8 == 0 && B >= 1 && B <= 128;
}

int score_fwd_mfma_launch(const void* iq, const void* ik, const int32_t* cu, int nseq, int64_t rows, int G, int Di,
                          int NB, int B, double scale, float* scores, int32_t* tie, hipStream_t st) {
  const dim3 grid(grid_1d(rows, kTileRows)), block(256);
  const auto* q = static_cast<const uint16_t*>(iq);
  const auto* k = static_cast<const uint16_t*>(ik);
  if (Di <= 32)
    hipLaunchKernelGGL(score_fwd_mfma_kernel<1>, grid, block, 0, st, q, k, cu, nseq, rows, G, Di, NB, B, scale, scores, tie);
  else if (Di <= 64)
    hipLaunchKernelGGL(score_fwd_mfma_kernel<2>, grid, block, 0, st, q, k, cu, nseq, rows, G, Di, NB, B, scale, scores, tie);
  else
    hipLaunchKernelGGL(score_fwd_mfma_kernel<4>, grid, block, 0, st, q, k, cu, nseq, rows, G, Di, NB, B, scale, scores, tie);
  return status_from(hipGetLastError());
}

}  // namespace msa
