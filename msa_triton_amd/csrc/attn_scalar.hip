// Stage 3, VALU path: sparse GQA attention forward, query-pass backward and
// CSR-driven KV-pass backward for every input dtype. Logits, dP and the
// softmax are evaluated in FP64: bf16/fp16/fp32 products are exact in FP64, so
// the query pass and the KV pass see identical logits/dP values and the
// softmax-gradient cancellation (dp - delta) is consistent between them. bf16 inputs
// with head dims up to 128 and up to 512 heads per group take the KV-major MFMA kernels
// (attn_kv_fwd.hip, attn_kv_bwd.hip; blocks above 128 keys as sub-blocks); this file
// serves fp16 / fp32 inputs and the shapes outside those templates. fp16 stays here on
// purpose: an fp16 output has three more significant bits than bf16, so fp32 sums put
// about eight times as many fp16 outputs near a rounding midpoint (an fp32-accumulating
// emulation leaves one outside the reference's gate at one of its small test shapes,
// which allow none), and the MFMA kernels' exact three-term splits of P and dS have no
// fp16 counterpart (fp16's five exponent bits: P's residuals underflow, dS can overflow).
//
// Semantics (triton/sparse_attention.py):
//   forward  :35-84  slots with 0 <= id <= qb(t) are visited in slot order,
//                    keys after the query in its own block are masked, online
//                    softmax, out = 0 and lse = -inf for rows without keys;
//   query bwd:87-198 p = exp(s - lse), mass = sum p, center c = O . dO,
//                    delta = sum p (dp - c) / mass,
//                    dS = p/mass * ((dp - c) - delta) * scale, dQ = sum dS k;
//   KV bwd   :223-295 per key, walk its (block, group) CSR row and accumulate
//                    dK += dS q, dV += p/mass dO over the R heads of each edge.
// The query pass forms dQ = scale/mass * (sum p (dp-c) k - delta * sum p k),
// which needs one pass over the keys instead of two.
#include "common.hpp"

namespace msa {

struct RowCtx {
  int64_t start;  // sequence start token
  int64_t qb;     // query block of t
};

__device__ __forceinline__ RowCtx row_ctx(const int32_t* __restrict__ cu, int nseq, int64_t t, int B) {
  const int s = find_seq(cu, nseq, t);
  RowCtx c;
  c.start = cu[s];
  c.qb = (t - c.start) / B;
  return c;
}

// Eight consecutive elements kept as loaded (16 bytes for 2-byte types, 32 for fp32),
// and their fp32 values.
template <int DT>
struct Raw8 {
  uint4 w[DT == kF32 ? 2 : 1];
};

template <int DT>
__device__ __forceinline__ Raw8<DT> load8_raw(const void* __restrict__ base, int64_t i) {
  Raw8<DT> r;
  if constexpr (DT == kF32) {
    r.w[0] = *reinterpret_cast<const uint4*>(static_cast<const float*>(base) + i);
    r.w[1] = *reinterpret_cast<const uint4*>(static_cast<const float*>(base) + i + 4);
  } else {
    r.w[0] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + i);
  }
  return r;
}

template <int DT>
__device__ __forceinline__ void unpack8(const Raw8<DT>& r, float (&x)[8]) {
  if constexpr (DT == kF32) {
    const uint32_t ws[8] = {r.w[0].x, r.w[0].y, r.w[0].z, r.w[0].w, r.w[1].x, r.w[1].y, r.w[1].z, r.w[1].w};
#pragma unroll
    for (int u = 0; u < 8; ++u) x[u] = __uint_as_float(ws[u]);
  } else {
    const uint32_t ws[4] = {r.w[0].x, r.w[0].y, r.w[0].z, r.w[0].w};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if constexpr (DT == kBF16) {
        x[2 * u] = __uint_as_float(ws[u] << 16);
        x[2 * u + 1] = __uint_as_float(ws[u] & 0xffff0000u);
      } else {
        x[2 * u] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(ws[u] & 0xffffu)));
        x[2 * u + 1] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(ws[u] >> 16)));
      }
    }
  }
}

// Elements [i, i + 8) of a row as fp32, from one 16-byte load (2-byte dtypes) or two
// (fp32); i a multiple of 8 (16-byte aligned). A lane walking its own key row this way
// issues one load instruction per 8 elements instead of one per element: with 64 lanes
// on 64 different rows, the address unit, not the FP64 arithmetic, limits these kernels.
template <int DT>
__device__ __forceinline__ void load8_as_f32(const void* __restrict__ base, int64_t i, float (&x)[8]) {
  unpack8<DT>(load8_raw<DT>(base, i), x);
}

// sum_d a[d] * row[off + d] in FP64, d = 0 .. D - 1 in order (a in LDS as fp32, 16-byte
// aligned when D % 8 == 0).
template <int DT>
__device__ __forceinline__ double row_dot(const float* a, const void* __restrict__ row, int64_t off, int D) {
  double acc = 0.0;
  if (D % 8 == 0 && (reinterpret_cast<uintptr_t>(row) & 15) == 0) {  // 16-byte aligned rows
    for (int d = 0; d < D; d += 8) {
      float x[8];
      load8_as_f32<DT>(row, off + d, x);
      const float4 a0 = *reinterpret_cast<const float4*>(a + d), a1 = *reinterpret_cast<const float4*>(a + d + 4);
      const float av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
      for (int u = 0; u < 8; ++u) acc = fma(static_cast<double>(av[u]), static_cast<double>(x[u]), acc);
    }
  } else {
    for (int d = 0; d < D; ++d) acc = fma(static_cast<double>(a[d]), static_cast<double>(load_as_f32<DT>(row, off + d)), acc);
  }
  return acc;
}

// Forward: one wavefront per (t, h). Keys are processed 64 at a time: each lane
// evaluates one key's logit, lanes then own head dims for the P.V update.
template <int DT, int DPL>
__global__ __launch_bounds__(256) void attn_fwd_valu(const void* __restrict__ q, const void* __restrict__ k,
                                                     const void* __restrict__ v,
                                                     const int32_t* __restrict__ indices,
                                                     const int32_t* __restrict__ cu, int nseq, int64_t T,
                                                     int Hq, int G, int D, int K, int B, double scale,
                                                     void* __restrict__ out, float* __restrict__ lse,
                                                     double* __restrict__ row_state, float* __restrict__ o32,
                                                     int dc0) {
  extern __shared__ float smem[];
  const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t th = static_cast<int64_t>(blockIdx.x) * 4 + wid;
  const bool active = th < T * Hq;
  float* qs = smem + wid * D;
  if (active)
    for (int d = lane; d < D; d += kWave) qs[d] = load_as_f32<DT>(q, th * D + d);
  __syncthreads();
  if (!active) return;
  const int64_t t = th / Hq;
  const int h = static_cast<int>(th % Hq);
  const int g = h / (Hq / G);
  const RowCtx rc = row_ctx(cu, nseq, t, B);
  double m = -__builtin_inf(), l = 0.0;
  double o[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j) o[j] = 0.0;
  const int32_t* sel = indices + (t * G + g) * K;
  for (int slot = 0; slot < K; ++slot) {
    const int blk = sel[slot];
    if (blk < 0 || blk > rc.qb) continue;
    const int64_t kb0 = rc.start + static_cast<int64_t>(blk) * B;
    const int64_t kend = (kb0 + B < t + 1) ? kb0 + B : t + 1;
    for (int64_t base = kb0; base < kend; base += kWave) {
      const int64_t key = base + lane;
      double sv = -__builtin_inf();
      if (key < kend) {
        sv = row_dot<DT>(qs, k, (key * G + g) * D, D) * scale;
      }
      const double mt = wave_max_f64(sv);
      const double mn = fmax(m, mt);
      const double alpha = (m == -__builtin_inf()) ? 0.0 : exp(m - mn);
      const double p = (key < kend) ? exp(sv - mn) : 0.0;
      l = l * alpha + wave_sum_f64(p);
#pragma unroll
      for (int j = 0; j < DPL; ++j) o[j] *= alpha;
      const int n = kend - base < kWave ? static_cast<int>(kend - base) : kWave;
      for (int i = 0; i < n; ++i) {
        const double pi = __shfl(p, i, kWave);
        const int64_t off = ((base + i) * G + g) * D;
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          const int d = dc0 + lane + j * kWave;
          if (d < D) o[j] = fma(pi, static_cast<double>(load_as_f32<DT>(v, off + d)), o[j]);
        }
      }
      m = mn;
    }
  }
#pragma unroll
  for (int j = 0; j < DPL; ++j) {
    const int d = dc0 + lane + j * kWave;
    if (d < D) {
      const double r = l > 0.0 ? o[j] / l : 0.0;
      store_from_f64<DT>(out, th * D + d, r);
      if (o32) o32[th * D + d] = static_cast<float>(r);
    }
  }
  if (lane == 0) {
    const double full = l > 0.0 ? m + log(l) : -__builtin_inf();
    lse[th] = static_cast<float>(full);
    if (row_state) {
      row_state[th * 4] = full;
      row_state[th * 4 + 1] = 1.0;  // FP64 lse: p = exp(x - lse) needs no mass correction
    }
  }
}

// Query-pass backward: one wavefront per (t, h).
template <int DT, int DPL>
__global__ __launch_bounds__(256) void attn_bwd_dq_valu(
    const void* __restrict__ q, const void* __restrict__ k, const void* __restrict__ v,
    const void* __restrict__ out, const void* __restrict__ dout, double* __restrict__ row_state,
    const int32_t* __restrict__ indices, const int32_t* __restrict__ cu, int nseq, int64_t T, int Hq, int G,
    int D, int K, int B, double scale, void* __restrict__ dq, int dc0) {
  extern __shared__ float smem[];
  const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t th = static_cast<int64_t>(blockIdx.x) * 4 + wid;
  const bool active = th < T * Hq;
  float* qs = smem + wid * 2 * D;
  float* gs = qs + D;
  double cpart = 0.0;
  if (active) {
    for (int d = lane; d < D; d += kWave) {
      qs[d] = load_as_f32<DT>(q, th * D + d);
      const float gd = load_as_f32<DT>(dout, th * D + d);
      gs[d] = gd;
      cpart = fma(static_cast<double>(load_as_f32<DT>(out, th * D + d)), static_cast<double>(gd), cpart);
    }
  }
  __syncthreads();
  if (!active) return;
  const int64_t t = th / Hq;
  const int h = static_cast<int>(th % Hq);
  const int g = h / (Hq / G);
  const RowCtx rc = row_ctx(cu, nseq, t, B);
  const double c = wave_sum_f64(cpart);
  const double row_lse = row_state[th * 4];
  double mass = 0.0, delta = 0.0;
  double a[DPL], bsum[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j) a[j] = bsum[j] = 0.0;
  const int32_t* sel = indices + (t * G + g) * K;
  if (row_lse != -__builtin_inf()) {
    for (int slot = 0; slot < K; ++slot) {
      const int blk = sel[slot];
      if (blk < 0 || blk > rc.qb) continue;
      const int64_t kb0 = rc.start + static_cast<int64_t>(blk) * B;
      const int64_t kend = (kb0 + B < t + 1) ? kb0 + B : t + 1;
      for (int64_t base = kb0; base < kend; base += kWave) {
        const int64_t key = base + lane;
        double p = 0.0, u = 0.0;
        if (key < kend) {
          const int64_t off = (key * G + g) * D;
          const double sacc = row_dot<DT>(qs, k, off, D), dacc = row_dot<DT>(gs, v, off, D);
          p = exp(sacc * scale - row_lse);
          u = p * (dacc - c);
          mass += p;
          delta += u;
        }
        const int n = kend - base < kWave ? static_cast<int>(kend - base) : kWave;
        for (int i = 0; i < n; ++i) {
          const double pi = __shfl(p, i, kWave);
          const double ui = __shfl(u, i, kWave);
          const int64_t off = ((base + i) * G + g) * D;
#pragma unroll
          for (int j = 0; j < DPL; ++j) {
            const int d = dc0 + lane + j * kWave;
            if (d < D) {
              const double kv = load_as_f32<DT>(k, off + d);
              a[j] = fma(ui, kv, a[j]);
              bsum[j] = fma(pi, kv, bsum[j]);
            }
          }
        }
      }
    }
  }
  const double msum = wave_sum_f64(mass);
  const double dsum = wave_sum_f64(delta);
  const bool has = msum > 0.0;
  const double dhat = has ? dsum / msum : 0.0;
  if (dq) {
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      const int d = dc0 + lane + j * kWave;
      if (d < D) {
        const double val = has ? static_cast<double>(scale) * (a[j] - dhat * bsum[j]) / msum : 0.0;
        store_from_f64<DT>(dq, th * D + d, val);
      }
    }
  }
  if (lane == 0) {
    row_state[th * 4 + 1] = has ? msum : 1.0;
    row_state[th * 4 + 2] = c;
    row_state[th * 4 + 3] = dhat;
  }
}

// Row-parallel form of the two query-pass kernels above for D = 8 LPR, LPR in
// {1, 2, 4, 8, 16}, 16-byte aligned rows: the logits stay one lane per key, but the
// key-weighted row sums (P.V in the forward, the two K sums of dQ) take LPR lanes per
// key row (8 dims each, one 16-byte load), RPW = 64 / LPR keys a step instead of one
// key per step with 2-byte loads. Each key slot (lane / LPR) keeps its own FP64 partial
// sums, added pairwise over the slots at the end (a fixed butterfly).
template <int DT, int LPR>
__global__ __launch_bounds__(256) void attn_fwd_rows(const void* __restrict__ q, const void* __restrict__ k,
                                                     const void* __restrict__ v,
                                                     const int32_t* __restrict__ indices,
                                                     const int32_t* __restrict__ cu, int nseq, int64_t T,
                                                     int Hq, int G, int D, int K, int B, double scale,
                                                     void* __restrict__ out, float* __restrict__ lse,
                                                     double* __restrict__ row_state, float* __restrict__ o32) {
  constexpr int RPW = kWave / LPR;
  extern __shared__ float smem[];
  const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t th = static_cast<int64_t>(blockIdx.x) * 4 + wid;
  const bool active = th < T * Hq;
  float* qs = smem + wid * D;
  if (active)
    for (int d = lane; d < D; d += kWave) qs[d] = load_as_f32<DT>(q, th * D + d);
  __syncthreads();
  if (!active) return;
  const int slot = lane / LPR, dch = lane % LPR;
  const int64_t t = th / Hq;
  const int h = static_cast<int>(th % Hq);
  const int g = h / (Hq / G);
  const RowCtx rc = row_ctx(cu, nseq, t, B);
  double m = -__builtin_inf(), l = 0.0;
  double o[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) o[u] = 0.0;
  const int32_t* sel = indices + (t * G + g) * K;
  for (int sk = 0; sk < K; ++sk) {
    const int blk = sel[sk];
    if (blk < 0 || blk > rc.qb) continue;
    const int64_t kb0 = rc.start + static_cast<int64_t>(blk) * B;
    const int64_t kend = (kb0 + B < t + 1) ? kb0 + B : t + 1;
    for (int64_t base = kb0; base < kend; base += kWave) {
      const int64_t key = base + lane;
      double sv = -__builtin_inf();
      if (key < kend) sv = row_dot<DT>(qs, k, (key * G + g) * D, D) * scale;
      const double mt = wave_max_f64(sv);
      const double mn = fmax(m, mt);
      const double alpha = (m == -__builtin_inf()) ? 0.0 : exp(m - mn);
      const double p = (key < kend) ? exp(sv - mn) : 0.0;
      l = l * alpha + wave_sum_f64(p);
#pragma unroll
      for (int u = 0; u < 8; ++u) o[u] *= alpha;
      const int n = kend - base < kWave ? static_cast<int>(kend - base) : kWave;
      for (int i0 = 0; i0 < n; i0 += RPW) {
        const int i = i0 + slot;  // <= 63: i0 < n <= 64 and RPW divides 64
        const double pi = __shfl(p, i, kWave);
        const Raw8<DT> w = load8_raw<DT>(v, ((base + (i < n ? i : 0)) * G + g) * D + 8 * dch);
        if (i < n) {
          float x[8];
          unpack8<DT>(w, x);
#pragma unroll
          for (int u = 0; u < 8; ++u) o[u] = fma(pi, static_cast<double>(x[u]), o[u]);
        }
      }
      m = mn;
    }
  }
#pragma unroll
  for (int off = LPR; off < kWave; off <<= 1) {
#pragma unroll
    for (int u = 0; u < 8; ++u) o[u] += __shfl_xor(o[u], off, kWave);
  }
  if (slot == 0) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t d = th * D + 8 * dch + u;
      const double r = l > 0.0 ? o[u] / l : 0.0;
      store_from_f64<DT>(out, d, r);
      if (o32) o32[d] = static_cast<float>(r);
    }
  }
  if (lane == 0) {
    const double full = l > 0.0 ? m + log(l) : -__builtin_inf();
    lse[th] = static_cast<float>(full);
    if (row_state) {
      row_state[th * 4] = full;
      row_state[th * 4 + 1] = 1.0;  // FP64 lse: p = exp(x - lse) needs no mass correction
    }
  }
}

template <int DT, int LPR>
__global__ __launch_bounds__(256) void attn_bwd_dq_rows(
    const void* __restrict__ q, const void* __restrict__ k, const void* __restrict__ v,
    const void* __restrict__ out, const void* __restrict__ dout, double* __restrict__ row_state,
    const int32_t* __restrict__ indices, const int32_t* __restrict__ cu, int nseq, int64_t T, int Hq, int G,
    int D, int K, int B, double scale, void* __restrict__ dq) {
  constexpr int RPW = kWave / LPR;
  extern __shared__ float smem[];
  const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t th = static_cast<int64_t>(blockIdx.x) * 4 + wid;
  const bool active = th < T * Hq;
  float* qs = smem + wid * 2 * D;
  float* gs = qs + D;
  double cpart = 0.0;
  if (active) {
    for (int d = lane; d < D; d += kWave) {
      qs[d] = load_as_f32<DT>(q, th * D + d);
      const float gd = load_as_f32<DT>(dout, th * D + d);
      gs[d] = gd;
      cpart = fma(static_cast<double>(load_as_f32<DT>(out, th * D + d)), static_cast<double>(gd), cpart);
    }
  }
  __syncthreads();
  if (!active) return;
  const int slot = lane / LPR, dch = lane % LPR;
  const int64_t t = th / Hq;
  const int h = static_cast<int>(th % Hq);
  const int g = h / (Hq / G);
  const RowCtx rc = row_ctx(cu, nseq, t, B);
  const double c = wave_sum_f64(cpart);
  const double row_lse = row_state[th * 4];
  double mass = 0.0, delta = 0.0;
  double a[8], bsum[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) a[u] = bsum[u] = 0.0;
  const int32_t* sel = indices + (t * G + g) * K;
  if (row_lse != -__builtin_inf()) {
    for (int sk = 0; sk < K; ++sk) {
      const int blk = sel[sk];
      if (blk < 0 || blk > rc.qb) continue;
      const int64_t kb0 = rc.start + static_cast<int64_t>(blk) * B;
      const int64_t kend = (kb0 + B < t + 1) ? kb0 + B : t + 1;
      for (int64_t base = kb0; base < kend; base += kWave) {
        const int64_t key = base + lane;
        double p = 0.0, uu = 0.0;
        if (key < kend) {
          const int64_t off = (key * G + g) * D;
          const double sacc = row_dot<DT>(qs, k, off, D), dacc = row_dot<DT>(gs, v, off, D);
          p = exp(sacc * scale - row_lse);
          uu = p * (dacc - c);
          mass += p;
          delta += uu;
        }
        const int n = kend - base < kWave ? static_cast<int>(kend - base) : kWave;
        for (int i0 = 0; i0 < n; i0 += RPW) {
          const int i = i0 + slot;  // <= 63: i0 < n <= 64 and RPW divides 64
          const double pi = __shfl(p, i, kWave);
          const double ui = __shfl(uu, i, kWave);
          const Raw8<DT> w = load8_raw<DT>(k, ((base + (i < n ? i : 0)) * G + g) * D + 8 * dch);
          if (i < n) {
            float x[8];
            unpack8<DT>(w, x);
#pragma unroll
            for (int u = 0; u < 8; ++u) {
              a[u] = fma(ui, static_cast<double>(x[u]), a[u]);
              bsum[u] = fma(pi, static_cast<double>(x[u]), bsum[u]);
            }
          }
        }
      }
    }
  }
  const double msum = wave_sum_f64(mass);
  const double dsum = wave_sum_f64(delta);
  const bool has = msum > 0.0;
  const double dhat = has ? dsum / msum : 0.0;
  if (dq) {
#pragma unroll
    for (int off = LPR; off < kWave; off <<= 1) {
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        a[u] += __shfl_xor(a[u], off, kWave);
        bsum[u] += __shfl_xor(bsum[u], off, kWave);
      }
    }
    if (slot == 0) {
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const double val = has ? static_cast<double>(scale) * (a[u] - dhat * bsum[u]) / msum : 0.0;
        store_from_f64<DT>(dq, th * D + 8 * dch + u, val);
      }
    }
  }
  if (lane == 0) {
    row_state[th * 4 + 1] = has ? msum : 1.0;
    row_state[th * 4 + 2] = c;
    row_state[th * 4 + 3] = dhat;
  }
}

// KV-pass backward: one wavefront per (key token, group); walks the key's
// (block, group) CSR row in order, all R heads of each edge.
template <int DT, int DPL>
__global__ __launch_bounds__(256) void attn_bwd_dkdv_valu(
    const void* __restrict__ q, const void* __restrict__ k, const void* __restrict__ v,
    const void* __restrict__ dout, const double* __restrict__ row_state, const int32_t* __restrict__ cu, const int32_t* __restrict__ cu_blocks, const int32_t* __restrict__ row_ptr,
    const int32_t* __restrict__ qidx, int nseq, int64_t T, int Hq, int G, int D, int B, double scale,
    void* __restrict__ dk, void* __restrict__ dv, int dc0) {
  const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t jg = static_cast<int64_t>(blockIdx.x) * 4 + wid;
  if (jg >= T * G) return;
  const int64_t j = jg / G;
  const int g = static_cast<int>(jg % G);
  const int s = find_seq(cu, nseq, j);
  const int64_t blk = (j - cu[s]) / B;
  const int64_t row = (static_cast<int64_t>(cu_blocks[s]) + blk) * G + g;
  const int64_t e0 = row_ptr[row], e1 = row_ptr[row + 1];
  const int R = Hq / G;
  // This launch's dims are dc0 + lane + 64 i (i < DPL). When they are all of D the key
  // and value rows stay in registers for the logits; otherwise (D above 64 x DPL, one
  // launch per 64 DPL dims) the logits loop over every dim from memory, in the same order.
  const bool whole = dc0 == 0 && D <= DPL * kWave;
  float kr[DPL], vr[DPL];
  double gk[DPL], gv[DPL];
#pragma unroll
  for (int i = 0; i < DPL; ++i) {
    const int d = dc0 + lane + i * kWave;
    kr[i] = d < D ? load_as_f32<DT>(k, jg * D + d) : 0.f;
    vr[i] = d < D ? load_as_f32<DT>(v, jg * D + d) : 0.f;
    gk[i] = gv[i] = 0.0;
  }
  for (int64_t e = e0; e < e1; ++e) {
    const int64_t t = qidx[e];
    if (t < j) continue;
    for (int r = 0; r < R; ++r) {
      const int64_t th = t * Hq + static_cast<int64_t>(g) * R + r;
      float qv[DPL], gdv[DPL];
      double sp = 0.0, dp = 0.0;
#pragma unroll
      for (int i = 0; i < DPL; ++i) {
        const int d = dc0 + lane + i * kWave;
        qv[i] = d < D ? load_as_f32<DT>(q, th * D + d) : 0.f;
        gdv[i] = d < D ? load_as_f32<DT>(dout, th * D + d) : 0.f;
        if (whole) {
          sp = fma(static_cast<double>(qv[i]), static_cast<double>(kr[i]), sp);
          dp = fma(static_cast<double>(gdv[i]), static_cast<double>(vr[i]), dp);
        }
      }
      if (!whole) {
        for (int d = lane; d < D; d += kWave) {
          sp = fma(static_cast<double>(load_as_f32<DT>(q, th * D + d)), static_cast<double>(load_as_f32<DT>(k, jg * D + d)), sp);
          dp = fma(static_cast<double>(load_as_f32<DT>(dout, th * D + d)), static_cast<double>(load_as_f32<DT>(v, jg * D + d)), dp);
        }
      }
      sp = wave_sum_f64(sp);
      dp = wave_sum_f64(dp);
      const double* rs = row_state + th * 4;
      const double mass = rs[1], c = rs[2], dhat = rs[3];
      const double p = exp(sp * scale - rs[0]) / mass;
      const double dsv = p * ((dp - c) - dhat) * scale;
#pragma unroll
      for (int i = 0; i < DPL; ++i) {
        gk[i] = fma(dsv, static_cast<double>(qv[i]), gk[i]);
        gv[i] = fma(p, static_cast<double>(gdv[i]), gv[i]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < DPL; ++i) {
    const int d = dc0 + lane + i * kWave;
    if (d < D) {
      if (dk) store_from_f64<DT>(dk, jg * D + d, gk[i]);
      if (dv) store_from_f64<DT>(dv, jg * D + d, gv[i]);
    }
  }
}

// KV-pass backward for head dims D = 8 LPR with LPR in {1, 2, 4, 8, 16}: one wavefront
// per (key token, group) as above, but LPR lanes per query row (8 dims each, 16-byte
// loads), so RPW = 64 / LPR rows of the key's CSR row go at once: row i = (e - e0) R + r
// (edge e, head r, in order) goes to slot i % RPW. A row's two dot products reduce over
// its LPR lanes only, and one exponential serves RPW rows. Each slot sums its rows in
// order; the slot sums are then added pairwise (a fixed butterfly over the slot index).
template <int DT, int LPR, int NC>
__global__ __launch_bounds__(256, DT == kF32 || NC == 2 ? 2 : 3) void attn_bwd_dkdv_rows(
    const void* __restrict__ q, const void* __restrict__ k, const void* __restrict__ v,
    const void* __restrict__ dout, const double* __restrict__ row_state, const int32_t* __restrict__ cu,
    const int32_t* __restrict__ cu_blocks, const int32_t* __restrict__ row_ptr, const int32_t* __restrict__ qidx,
    int nseq, int64_t T, int Hq, int G, int D, int B, double scale, void* __restrict__ dk, void* __restrict__ dv) {
  constexpr int RPW = kWave / LPR;
  const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t jg = static_cast<int64_t>(blockIdx.x) * 4 + wid;
  if (jg >= T * G) return;
  const int slot = lane / LPR, dch = lane % LPR;
  const int64_t j = jg / G;
  const int g = static_cast<int>(jg % G);
  const int s = find_seq(cu, nseq, j);
  const int64_t blk = (j - cu[s]) / B;
  const int64_t row = (static_cast<int64_t>(cu_blocks[s]) + blk) * G + g;
  const int64_t e0 = row_ptr[row], e1 = row_ptr[row + 1];
  const int R = Hq / G;
  constexpr int E = 8 * NC;  // dims per lane: [E dch, E dch + E)
  float kr[E], vr[E];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    load8_as_f32<DT>(k, jg * D + E * dch + 8 * c, *reinterpret_cast<float(*)[8]>(kr + 8 * c));
    load8_as_f32<DT>(v, jg * D + E * dch + 8 * c, *reinterpret_cast<float(*)[8]>(vr + 8 * c));
  }
  double gk[E], gv[E];
#pragma unroll
  for (int u = 0; u < E; ++u) gk[u] = gv[u] = 0.0;
  // Row i = (e - e0) R + r is walked as the pair (e, r), RPW rows a step. Software
  // pipeline: the query index two steps ahead, the rows one step ahead (positions past the
  // end read the row's first edge, so every load stays in bounds).
  struct Cursor { int64_t e; int r; };
  const int64_t estep = RPW / R;
  const int rstep = RPW % R;
  auto advance = [&](Cursor& c) {
    c.e += estep;
    c.r += rstep;
    if (c.r >= R) c.r -= R, ++c.e;
  };
  auto edge_of = [&](const Cursor& c) -> int64_t { return c.e < e1 ? c.e : e0; };
  struct Rows { Raw8<DT> qw[NC], gw[NC]; double2 rs01, rs23; };
  auto fetch = [&](const Cursor& c, int64_t t, Rows& x) {
    const int64_t th = t * Hq + static_cast<int64_t>(g) * R + (c.e < e1 ? c.r : 0);
#pragma unroll
    for (int z = 0; z < NC; ++z) {
      x.qw[z] = load8_raw<DT>(q, th * D + E * dch + 8 * z);
      x.gw[z] = load8_raw<DT>(dout, th * D + E * dch + 8 * z);
    }
    x.rs01 = reinterpret_cast<const double2*>(row_state)[th * 2];
    x.rs23 = reinterpret_cast<const double2*>(row_state)[th * 2 + 1];
  };
  if (e1 > e0) {
    Cursor cc{e0 + slot / R, slot % R};
    Cursor cn = cc;
    advance(cn);
    Cursor cnn = cn;
    advance(cnn);
    int64_t tc = qidx[edge_of(cc)];
    int64_t tn = qidx[edge_of(cn)];
    Rows cur;
    fetch(cc, tc, cur);
    // lane 0 holds a step's first row: the step is live while that row is
    while (__builtin_amdgcn_readfirstlane(static_cast<int>(cc.e < e1))) {
      Rows nxt;
      fetch(cn, tn, nxt);
      const int64_t tnn = qidx[edge_of(cnn)];
      const bool ok = cc.e < e1 && tc >= j;
      float qv[E], gdv[E];
#pragma unroll
      for (int z = 0; z < NC; ++z) {
        unpack8<DT>(cur.qw[z], *reinterpret_cast<float(*)[8]>(qv + 8 * z));
        unpack8<DT>(cur.gw[z], *reinterpret_cast<float(*)[8]>(gdv + 8 * z));
      }
      double sp = 0.0, dp = 0.0;
#pragma unroll
      for (int u = 0; u < E; ++u) {
        if constexpr (DT == kF32) {
          sp = fma(static_cast<double>(qv[u]), static_cast<double>(kr[u]), sp);
          dp = fma(static_cast<double>(gdv[u]), static_cast<double>(vr[u]), dp);
        } else {  // a product of two 2-byte floats is exact in fp32: the same FP64 sum
          sp += static_cast<double>(qv[u] * kr[u]);
          dp += static_cast<double>(gdv[u] * vr[u]);
        }
      }
#pragma unroll
      for (int o = 1; o < LPR; o <<= 1) {
        sp += __shfl_xor(sp, o, kWave);
        dp += __shfl_xor(dp, o, kWave);
      }
      if (ok) {
        const double p = exp(sp * scale - cur.rs01.x) / cur.rs01.y;
        const double dsv = p * ((dp - cur.rs23.x) - cur.rs23.y) * scale;
#pragma unroll
        for (int u = 0; u < E; ++u) {
          gk[u] = fma(dsv, static_cast<double>(qv[u]), gk[u]);
          gv[u] = fma(p, static_cast<double>(gdv[u]), gv[u]);
        }
      }
      cur = nxt;
      tc = tn;
      tn = tnn;
      cc = cn;
      cn = cnn;
      advance(cnn);
    }
  }
#pragma unroll
  for (int o = LPR; o < kWave; o <<= 1) {
#pragma unroll
    for (int u = 0; u < E; ++u) {
      gk[u] += __shfl_xor(gk[u], o, kWave);
      gv[u] += __shfl_xor(gv[u], o, kWave);
    }
  }
  if (slot == 0) {
#pragma unroll
    for (int u = 0; u < E; ++u) {
      if (dk) store_from_f64<DT>(dk, jg * D + E * dch + u, gk[u]);
      if (dv) store_from_f64<DT>(dv, jg * D + E * dch + u, gv[u]);
    }
  }
}

// The row-parallel kernels take D = 8 LPR (LPR a power of two up to 16) and rows that
// start on 16-byte boundaries.
template <typename... P>
bool rows_fit(int D, const P*... ptrs) {
  const uintptr_t bits = (reinterpret_cast<uintptr_t>(ptrs) | ...);
  return (D == 8 || D == 16 || D == 32 || D == 64 || D == 128) && (bits & 15) == 0;
}

#define MSA_ROWS_SWITCH(D, LAUNCH) \
  switch ((D) / 8) {               \
    case 1: LAUNCH(1); break;      \
    case 2: LAUNCH(2); break;      \
    case 4: LAUNCH(4); break;      \
    case 8: LAUNCH(8); break;      \
    default: LAUNCH(16); break;    \
  }

template <int DT, int DPL>
int attn_valu_launch_fwd(const void* q, const void* k, const void* v, const int32_t* idx, const int32_t* cu,
                         int nseq, int64_t T, int Hq, int G, int D, int K, int B, double scale, void* out,
                         float* lse, double* rs, float* o32, hipStream_t st) {
  if (rows_fit(D, q, k, v)) {
#define MSA_FWD_ROWS(LPRV) hipLaunchKernelGGL((attn_fwd_rows<DT, LPRV>), dim3(grid_1d(T * Hq, 4)), dim3(256), 4 * D * sizeof(float), st, q, k, v, idx, cu, nseq, T, Hq, G, D, K, B, scale, out, lse, rs, o32)
    MSA_ROWS_SWITCH(D, MSA_FWD_ROWS);
#undef MSA_FWD_ROWS
    return status_from(hipGetLastError());
  }
  for (int dc0 = 0; dc0 < D; dc0 += DPL * kWave)
    hipLaunchKernelGGL((attn_fwd_valu<DT, DPL>), dim3(grid_1d(T * Hq, 4)), dim3(256), 4 * D * sizeof(float), st, q,
                       k, v, idx, cu, nseq, T, Hq, G, D, K, B, scale, out, lse, rs, o32, dc0);
  return status_from(hipGetLastError());
}

template <int DT, int DPL>
int attn_valu_launch_dq(const void* q, const void* k, const void* v, const void* out, const void* dout, double* rs,
                        const int32_t* idx, const int32_t* cu, int nseq, int64_t T, int Hq, int G, int D, int K,
                        int B, double scale, void* dq, hipStream_t st) {
  if (rows_fit(D, q, k, v, dout)) {
#define MSA_DQ_ROWS(LPRV) hipLaunchKernelGGL((attn_bwd_dq_rows<DT, LPRV>), dim3(grid_1d(T * Hq, 4)), dim3(256), 8 * D * sizeof(float), st, q, k, v, out, dout, rs, idx, cu, nseq, T, Hq, G, D, K, B, scale, dq)
    MSA_ROWS_SWITCH(D, MSA_DQ_ROWS);
#undef MSA_DQ_ROWS
    return status_from(hipGetLastError());
  }
  for (int dc0 = 0; dc0 < D; dc0 += DPL * kWave)
    hipLaunchKernelGGL((attn_bwd_dq_valu<DT, DPL>), dim3(grid_1d(T * Hq, 4)), dim3(256), 8 * D * sizeof(float),
                       st, q, k, v, out, dout, rs, idx, cu, nseq, T, Hq, G, D, K, B, scale, dq, dc0);
  return status_from(hipGetLastError());
}

template <int DT, int DPL>
int attn_valu_launch_dkdv(const void* q, const void* k, const void* v, const void* dout, const double* rs,
                          const int32_t* cu, const int32_t* cu_blocks, const int32_t* row_ptr, const int32_t* qidx,
                          int nseq, int64_t T, int Hq, int G, int D, int B, double scale, void* dk, void* dv,
                          hipStream_t st) {
  if (rows_fit(D, q, k, v, dout, rs)) {
#define MSA_DKDV_ROWS(LPRV, NCV) hipLaunchKernelGGL((attn_bwd_dkdv_rows<DT, LPRV, NCV>), dim3(grid_1d(T * G, 4)), dim3(256), 0, st, q, k, v, dout, rs, cu, cu_blocks, row_ptr, qidx, nseq, T, Hq, G, D, B, scale, dk, dv)
    switch (D) {  // 2-byte types at D = 128: 16 dims a lane; otherwise 8
      case 8: MSA_DKDV_ROWS(1, 1); break;
      case 16: MSA_DKDV_ROWS(2, 1); break;
      case 32: MSA_DKDV_ROWS(4, 1); break;
      case 64: MSA_DKDV_ROWS(8, 1); break;
      default:
        if constexpr (DT == kF32) MSA_DKDV_ROWS(16, 1);
        else MSA_DKDV_ROWS(8, 2);
        break;
    }
#undef MSA_DKDV_ROWS
    return status_from(hipGetLastError());
  }
  for (int dc0 = 0; dc0 < D; dc0 += DPL * kWave)
    hipLaunchKernelGGL((attn_bwd_dkdv_valu<DT, DPL>), dim3(grid_1d(T * G, 4)), dim3(256), 0, st, q, k, v, dout, rs,
                       cu, cu_blocks, row_ptr, qidx, nseq, T, Hq, G, D, B, scale, dk, dv, dc0);
  return status_from(hipGetLastError());
}

#define MSA_DPL_DISPATCH(D, FN, ...)     \
  ((D) <= 64    ? FN<DT, 1>(__VA_ARGS__) \
   : (D) <= 128 ? FN<DT, 2>(__VA_ARGS__) \
   : (D) <= 256 ? FN<DT, 4>(__VA_ARGS__) \
                : FN<DT, 8>(__VA_ARGS__))

template <int DT>
int attn_fwd_valu_dispatch(const void* q, const void* k, const void* v, const int32_t* idx, const int32_t* cu,
                           int nseq, int64_t T, int Hq, int G, int D, int K, int B, double scale, void* out,
                           float* lse, double* rs, float* o32, hipStream_t st) {
  return MSA_DPL_DISPATCH(D, attn_valu_launch_fwd, q, k, v, idx, cu, nseq, T, Hq, G, D, K, B, scale, out, lse, rs,
                          o32, st);
}

template <int DT>
int attn_dq_valu_dispatch(const void* q, const void* k, const void* v, const void* out, const void* dout, double* rs,
                          const int32_t* idx, const int32_t* cu, int nseq, int64_t T, int Hq, int G, int D, int K,
                          int B, double scale, void* dq, hipStream_t st) {
  return MSA_DPL_DISPATCH(D, attn_valu_launch_dq, q, k, v, out, dout, rs, idx, cu, nseq, T, Hq, G, D, K, B, scale,
                          dq, st);
}

template <int DT>
int attn_dkdv_valu_dispatch(const void* q, const void* k, const void* v, const void* dout, const double* rs,
                            const int32_t* cu, const int32_t* cu_blocks, const int32_t* row_ptr, const int32_t* qidx,
                            int nseq, int64_t T, int Hq, int G, int D, int B, double scale, void* dk, void* dv,
                            hipStream_t st) {
  return MSA_DPL_DISPATCH(D, attn_valu_launch_dkdv, q, k, v, dout, rs, cu, cu_blocks, row_ptr, qidx, nseq, T, Hq, G,
                          D, B, scale, dk, dv, st);
}

#define MSA_INSTANTIATE_VALU(DT)                                                                                    \
  template int attn_fwd_valu_dispatch<DT>(const void*, const void*, const void*, const int32_t*, const int32_t*, int, \
                                          int64_t, int, int, int, int, int, double, void*, float*, double*, float*,  \
                                          hipStream_t);                                                              \
  template int attn_dq_valu_dispatch<DT>(const void*, const void*, const void*, const void*, const void*, double*,   \
                                         const int32_t*, const int32_t*, int, int64_t, int, int, int, int, int,      \
                                         double, void*, hipStream_t);                                                \
  template int attn_dkdv_valu_dispatch<DT>(const void*, const void*, const void*, const void*, const double*,       \
                                           const int32_t*, const int32_t*, const int32_t*, const int32_t*, int,      \
                                           int64_t, int, int, int, int, double, void*, void*, hipStream_t);
MSA_INSTANTIATE_VALU(kF32)
MSA_INSTANTIATE_VALU(kF16)
MSA_INSTANTIATE_VALU(kBF16)

}  // namespace msa
