// Stage 3 on MFMA (bf16 inputs): sparse GQA attention forward, query-pass
// backward (dQ + row statistics) and KV-pass backward (dK/dV over the k2q CSR).
//
// Matrix core: v_mfma_f32_16x16x32_bf16. Lane l (c = l % 16, q4 = l / 16) holds
//   A[c][8*q4 + j], B[8*q4 + j][c] (j = 0..7) and C[4*q4 + i][c] (i = 0..3).
// Logits q.k and dP = dO.v are always formed with the K (or V) row fragment and
// the Q (or dO) row fragment over the same dims in the same k-step order, so the
// forward, query and KV passes compute bitwise-identical fp32 logits/dP (MFMA
// results do not depend on which operand is A).
//
// Precision: fp32 operands of the second products (P in P.V, dS in dS.K,
// P^T in P^T.dO, dS^T in dS^T.Q) are split into three bf16 terms
// (hi + mid + lo, 24 significant bits), so every product is fp32-accurate.
// Softmax statistics that need it are kept in fp64.
//
// Work decomposition:
//   forward / query pass: one wavefront per (token, group, 16-head chunk); the
//     selected blocks are streamed 32 keys at a time; K/V row fragments come
//     straight from HBM in the A-operand layout and are re-written transposed
//     into per-wave LDS for the key-contraction products.
//   KV pass: one workgroup (4 waves x 32 keys) per (key block, group) row of the
//     CSR and per chunk of its edges; the edges' Q / dO rows are staged once in
//     LDS (row-major and transposed) and shared by the 4 waves. Rows longer than
//     one chunk write fp32 partials that a finalize kernel sums in chunk order
//     (deterministic, no floating-point atomics).
#include "attn_mfma.hpp"
#include "mfma_util.hpp"

namespace msa {

namespace {

struct SelRow {
  int64_t start;
  int64_t qb;
};

__device__ __forceinline__ SelRow sel_row(const int32_t* __restrict__ cu, int nseq, int64_t t, int B) {
  const int s = find_seq(cu, nseq, t);
  SelRow r;
  r.start = cu[s];
  r.qb = (t - r.start) / B;
  return r;
}

}  // namespace

// ---------------------------------------------------------------------------- forward

template <int NK>
__global__ __launch_bounds__(256) void attn_fwd_mfma_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const int32_t* __restrict__ indices, const int32_t* __restrict__ cu, int nseq, int64_t items, int Hq, int G,
    int D, int K, int B, float scale, uint16_t* __restrict__ out, float* __restrict__ lse,
    double* __restrict__ row_state) {
  constexpr int DP = 32 * NK, NDT = DP / 16;
  __shared__ uint16_t vt_all[4][DP * kTS];
  const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int c = lane & 15, q4 = lane >> 4;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + wid;
  if (item >= items) return;  // waves never synchronise with each other in this kernel
  uint16_t* vt = vt_all[wid];
  const int R = Hq / G, nhc = (R + 15) / 16;
  const int hc = static_cast<int>(item % nhc);
  const int64_t tg = item / nhc;
  const int g = static_cast<int>(tg % G);
  const int64_t t = tg / G;
  const int hl = hc * 16 + c;  // head inside the group owned by this lane's column
  const bool head_ok = hl < R;
  const int64_t th = t * Hq + static_cast<int64_t>(g) * R + hl;
  const SelRow sr = sel_row(cu, nseq, t, B);

  bf16x8 qf[NK];
#pragma unroll
  for (int kk = 0; kk < NK; ++kk) {
    const int d0 = 32 * kk + 8 * q4;
    qf[kk] = (head_ok && d0 < D) ? load_frag(q + th * D + d0) : zero_frag();
  }
  float m = -__builtin_inff();
  double l = 0.0;
  f32x4 o[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int32_t* sel = indices + (t * G + g) * K;
  for (int slot = 0; slot < K; ++slot) {
    const int blk = sel[slot];
    if (blk < 0 || blk > sr.qb) continue;
    const int64_t kb = sr.start + static_cast<int64_t>(blk) * B;
    const int64_t kend = (kb + B < t + 1) ? kb + B : t + 1;
    for (int64_t ck = kb; ck < kend; ck += 32) {
      // K fragments (A operand of S^T = K Q^T) and V fragments -> transposed LDS.
      bf16x8 kf[2][NK];
      compiler_fence();
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const int64_t key = ck + 16 * kt + c;
        const bool kv_ok = key < kend;
#pragma unroll
        for (int kk = 0; kk < NK; ++kk) {
          const int d0 = 32 * kk + 8 * q4;
          const bool ok = kv_ok && d0 < D;
          const int64_t off = (key * G + g) * D + d0;
          kf[kt][kk] = ok ? load_frag(k + off) : zero_frag();
          const bf16x8 vf = ok ? load_frag(v + off) : zero_frag();
          store_transposed(vt, d0, 16 * kt + c, vf);
        }
      }
      compiler_fence();
      float sv[2][4];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < NK; ++kk) acc = mfma(kf[kt][kk], qf[kk], acc);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int64_t key = ck + 16 * kt + 4 * q4 + i;
          sv[kt][i] = key < kend ? acc[i] * scale : -__builtin_inff();
        }
      }
      float mx = -__builtin_inff();
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) mx = fmaxf(mx, sv[kt][i]);
      mx = quad_max(mx);
      const float mn = fmaxf(m, mx);
      const float alpha = (m == -__builtin_inff()) ? 0.f : expf(m - mn);
      m = mn;
      Frag8 fh, fm, fl;
      float psum = 0.f;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = expf(sv[kt][i] - mn);
          psum += p;
          uint16_t a, b2, c2;
          split3(p, a, b2, c2);
          fh.set(4 * kt + i, a);
          fm.set(4 * kt + i, b2);
          fl.set(4 * kt + i, c2);
        }
      const bf16x8 ph = fh.vec(), pm = fm.vec(), pl = fl.vec();
      l = l * static_cast<double>(alpha) + static_cast<double>(psum);
      if (alpha != 1.f) {
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
          for (int i = 0; i < 4; ++i) o[dt][i] *= alpha;
      }
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const bf16x8 va = read_transposed(vt, dt * 16 + c, q4);
        o[dt] = mfma(va, pl, o[dt]);
        o[dt] = mfma(va, pm, o[dt]);
        o[dt] = mfma(va, ph, o[dt]);
      }
    }
  }
  const double lt = quad_sum(l);
  if (!head_ok) return;
  const double inv = lt > 0.0 ? 1.0 / lt : 0.0;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
    const int d0 = dt * 16 + 4 * q4;
    if (d0 < D) {
      uint16_t h4[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) h4[i] = f32_to_bf16_bits(static_cast<float>(static_cast<double>(o[dt][i]) * inv));
      *reinterpret_cast<uint2*>(out + th * D + d0) =
          make_uint2(h4[0] | (static_cast<uint32_t>(h4[1]) << 16), h4[2] | (static_cast<uint32_t>(h4[3]) << 16));
    }
  }
  if (q4 == 0) {
    const double full = lt > 0.0 ? static_cast<double>(m) + log(lt) : -__builtin_inf();
    lse[th] = static_cast<float>(full);
    if (row_state) row_state[th * 4] = full;
  }
}

// ---------------------------------------------------------------------------- query pass

// dQ = scale/mass * (sum_j p_j (dp_j - c) k_j - delta * sum_j p_j k_j) in one pass,
// with p_j = exp(s_j - lse), mass = sum_j p_j, c = O . dO, delta = sum p (dp - c) / mass.
template <int NK>
__global__ __launch_bounds__(256) void attn_dq_mfma_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint16_t* __restrict__ out, const uint16_t* __restrict__ dout, double* __restrict__ row_state,
    const int32_t* __restrict__ indices, const int32_t* __restrict__ cu, int nseq, int64_t items, int Hq, int G,
    int D, int K, int B, float scale, uint16_t* __restrict__ dq) {
  constexpr int DP = 32 * NK, NDT = DP / 16;
  __shared__ uint16_t kt_all[4][DP * kTS];
  const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int c = lane & 15, q4 = lane >> 4;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + wid;
  if (item >= items) return;
  uint16_t* ktile = kt_all[wid];
  const int R = Hq / G, nhc = (R + 15) / 16;
  const int hc = static_cast<int>(item % nhc);
  const int64_t tg = item / nhc;
  const int g = static_cast<int>(tg % G);
  const int64_t t = tg / G;
  const int hl = hc * 16 + c;
  const bool head_ok = hl < R;
  const int64_t th = t * Hq + static_cast<int64_t>(g) * R + hl;
  const SelRow sr = sel_row(cu, nseq, t, B);

  bf16x8 qf[NK], gf[NK];
  double cpart = 0.0;
#pragma unroll
  for (int kk = 0; kk < NK; ++kk) {
    const int d0 = 32 * kk + 8 * q4;
    const bool ok = head_ok && d0 < D;
    qf[kk] = ok ? load_frag(q + th * D + d0) : zero_frag();
    gf[kk] = ok ? load_frag(dout + th * D + d0) : zero_frag();
    if (ok) {
      const uint4 ow = *reinterpret_cast<const uint4*>(out + th * D + d0);
      const uint4 gw = __builtin_bit_cast(uint4, gf[kk]);
      const uint32_t o4[4] = {ow.x, ow.y, ow.z, ow.w}, g4[4] = {gw.x, gw.y, gw.z, gw.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        cpart = fma(static_cast<double>(__uint_as_float(o4[j] << 16)), static_cast<double>(__uint_as_float(g4[j] << 16)),
                    cpart);
        cpart = fma(static_cast<double>(__uint_as_float(o4[j] & 0xffff0000u)),
                    static_cast<double>(__uint_as_float(g4[j] & 0xffff0000u)), cpart);
      }
    }
  }
  const double center = quad_sum(cpart);
  const float cf = static_cast<float>(center);
  const double lse_row = head_ok ? row_state[th * 4] : -__builtin_inf();
  const float lse_f = static_cast<float>(lse_row);
  double mass = 0.0, delta = 0.0;
  f32x4 acc_u[NDT], acc_p[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) acc_u[dt] = acc_p[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int32_t* sel = indices + (t * G + g) * K;
  for (int slot = 0; slot < K; ++slot) {
    const int blk = sel[slot];
    if (blk < 0 || blk > sr.qb) continue;
    const int64_t kb = sr.start + static_cast<int64_t>(blk) * B;
    const int64_t kend = (kb + B < t + 1) ? kb + B : t + 1;
    for (int64_t ck = kb; ck < kend; ck += 32) {
      bf16x8 kf[2][NK], vf[2][NK];
      compiler_fence();
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const int64_t key = ck + 16 * kt + c;
        const bool kv_ok = key < kend;
#pragma unroll
        for (int kk = 0; kk < NK; ++kk) {
          const int d0 = 32 * kk + 8 * q4;
          const bool ok = kv_ok && d0 < D;
          const int64_t off = (key * G + g) * D + d0;
          kf[kt][kk] = ok ? load_frag(k + off) : zero_frag();
          vf[kt][kk] = ok ? load_frag(v + off) : zero_frag();
          store_transposed(ktile, d0, 16 * kt + c, kf[kt][kk]);
        }
      }
      compiler_fence();
      Frag8 fuh, fum, ful, fph, fpm, fpl;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        f32x4 sacc = {0.f, 0.f, 0.f, 0.f}, dacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < NK; ++kk) {
          sacc = mfma(kf[kt][kk], qf[kk], sacc);
          dacc = mfma(vf[kt][kk], gf[kk], dacc);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int64_t key = ck + 16 * kt + 4 * q4 + i;
          float p = 0.f, u = 0.f;
          if (key < kend && head_ok) {
            p = expf(sacc[i] * scale - lse_f);
            u = p * (dacc[i] - cf);
            mass += static_cast<double>(p);
            delta += static_cast<double>(u);
          }
          uint16_t a, b2, c2;
          split3(u, a, b2, c2);
          fuh.set(4 * kt + i, a);
          fum.set(4 * kt + i, b2);
          ful.set(4 * kt + i, c2);
          split3(p, a, b2, c2);
          fph.set(4 * kt + i, a);
          fpm.set(4 * kt + i, b2);
          fpl.set(4 * kt + i, c2);
        }
      }
      const bf16x8 uh = fuh.vec(), um = fum.vec(), ul = ful.vec();
      const bf16x8 ph = fph.vec(), pm = fpm.vec(), pl = fpl.vec();
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const bf16x8 ka = read_transposed(ktile, dt * 16 + c, q4);
        acc_u[dt] = mfma(ka, ul, acc_u[dt]);
        acc_u[dt] = mfma(ka, um, acc_u[dt]);
        acc_u[dt] = mfma(ka, uh, acc_u[dt]);
        acc_p[dt] = mfma(ka, pl, acc_p[dt]);
        acc_p[dt] = mfma(ka, pm, acc_p[dt]);
        acc_p[dt] = mfma(ka, ph, acc_p[dt]);
      }
    }
  }
  const double msum = quad_sum(mass);
  const double dsum = quad_sum(delta);
  if (!head_ok) return;
  const bool has = msum > 0.0;
  const double dhat = has ? dsum / msum : 0.0;
  if (dq) {
    const double f = has ? static_cast<double>(scale) / msum : 0.0;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const int d0 = dt * 16 + 4 * q4;
      if (d0 < D) {
        uint16_t h4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const double val = f * (static_cast<double>(acc_u[dt][i]) - dhat * static_cast<double>(acc_p[dt][i]));
          h4[i] = f32_to_bf16_bits(static_cast<float>(val));
        }
        *reinterpret_cast<uint2*>(dq + th * D + d0) =
            make_uint2(h4[0] | (static_cast<uint32_t>(h4[1]) << 16), h4[2] | (static_cast<uint32_t>(h4[3]) << 16));
      }
    }
  }
  if (q4 == 0) {
    row_state[th * 4 + 1] = has ? msum : 1.0;
    row_state[th * 4 + 2] = center;
    row_state[th * 4 + 3] = dhat;
  }
}

// ---------------------------------------------------------------------------- KV pass

constexpr int kEdgeChunk = 1024;  // CSR edges per work item

// item_start[r] = sum_{r' < r} max(1, ceil(len(r') / chunk)); one workgroup of 1024.
__global__ __launch_bounds__(1024) void kv_item_scan(const int32_t* __restrict__ row_ptr, int64_t rows, int chunk,
                                                     int32_t* __restrict__ item_start) {
  __shared__ int32_t wsum[16];
  __shared__ int32_t carry_s;
  if (threadIdx.x == 0) carry_s = 0;
  __syncthreads();
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  for (int64_t base = 0; base < rows; base += 1024) {
    const int64_t r = base + threadIdx.x;
    int32_t n = 0;
    if (r < rows) {
      const int32_t len = row_ptr[r + 1] - row_ptr[r];
      n = len > 0 ? (len + chunk - 1) / chunk : 1;
    }
    int32_t x = n;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int32_t y = __shfl_up(x, o, kWave);
      if (lane >= o) x += y;
    }
    if (lane == 63) wsum[wid] = x;
    __syncthreads();
    if (threadIdx.x < 16) {
      int32_t w = wsum[threadIdx.x];
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) {
        const int32_t y = __shfl_up(w, o, 16);
        if (static_cast<int>(threadIdx.x) >= o) w += y;
      }
      wsum[threadIdx.x] = w;
    }
    __syncthreads();
    const int32_t carry = carry_s;
    if (r < rows) item_start[r] = carry + (wid > 0 ? wsum[wid - 1] : 0) + x - n;
    __syncthreads();
    if (threadIdx.x == 0) carry_s = carry + wsum[15];
    __syncthreads();
  }
  if (threadIdx.x == 0) item_start[rows] = carry_s;
}

template <int NK>
struct KvSmem {
  static constexpr int DP = 32 * NK;
  static constexpr int RS = DP + 8;  // padded row stride of the row-major tiles
  uint16_t q_rm[32 * RS];
  uint16_t g_rm[32 * RS];
  uint16_t q_t[DP * kTS];
  uint16_t g_t[DP * kTS];
  float lse[32];
  float mass[32];
  float center[32];
  float dhat[32];
  int64_t tok[32];
};

// One workgroup per (CSR row, edge chunk). Wave w owns keys [32w, 32w+32) of the
// block (block_size <= 128). Partial rows (n_items > 1) write fp32 partials.
template <int NK>
__global__ __launch_bounds__(256) void attn_dkdv_mfma_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint16_t* __restrict__ dout, const double* __restrict__ row_state, const int32_t* __restrict__ cu,
    const int32_t* __restrict__ cu_blocks, const int32_t* __restrict__ row_ptr, const int32_t* __restrict__ qidx,
    const int32_t* __restrict__ item_start, int nseq, int64_t rows, int Hq, int G, int D, int B, float scale,
    uint16_t* __restrict__ dk, uint16_t* __restrict__ dv, float* __restrict__ partial) {
  constexpr int DP = 32 * NK, NDT = DP / 16, RS = KvSmem<NK>::RS;
  __shared__ KvSmem<NK> sm;
  const int64_t item = blockIdx.x;
  if (item >= item_start[rows]) return;  // whole workgroup exits together
  const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int c = lane & 15, q4 = lane >> 4;
  const int64_t row = upper_index(item_start, static_cast<int>(rows) + 1, item);
  // every row owns at least one item, so item_start is strictly increasing
  const int chunk_id = static_cast<int>(item - item_start[row]);
  const int n_items = item_start[row + 1] - item_start[row];
  const int64_t gb = row / G;
  const int g = static_cast<int>(row % G);
  int s = upper_index(cu_blocks, nseq + 1, gb);
  while (s < nseq && cu_blocks[s + 1] <= gb) ++s;
  const int64_t start = cu[s], end = cu[s + 1];
  const int64_t kb = start + (gb - cu_blocks[s]) * B;
  const int64_t kend = kb + B < end ? kb + B : end;
  const int R = Hq / G;
  const int64_t e_begin = static_cast<int64_t>(row_ptr[row]) + static_cast<int64_t>(chunk_id) * kEdgeChunk;
  int64_t e_end = e_begin + kEdgeChunk;
  if (e_end > row_ptr[row + 1]) e_end = row_ptr[row + 1];
  const int64_t nrows = (e_end > e_begin ? e_end - e_begin : 0) * R;

  // This wave's keys: kb + 32*wid + 16*kt + c.
  bf16x8 kf[2][NK], vf[2][NK];
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
    const int64_t key = kb + 32 * wid + 16 * kt + c;
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) {
      const int d0 = 32 * kk + 8 * q4;
      const bool ok = key < kend && d0 < D;
      const int64_t off = (key * G + g) * D + d0;
      kf[kt][kk] = ok ? load_frag(k + off) : zero_frag();
      vf[kt][kk] = ok ? load_frag(v + off) : zero_frag();
    }
  }
  f32x4 acc_k[2][NDT], acc_v[2][NDT];
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) acc_k[kt][dt] = acc_v[kt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int64_t r0 = 0; r0 < nrows; r0 += 32) {
    // ---- stage 32 (edge, head) rows of Q and dO, row-major and transposed
    __syncthreads();
    for (int e = threadIdx.x; e < 32 * (DP / 8); e += 256) {
      const int rr = e / (DP / 8), d0 = 8 * (e % (DP / 8));
      const int64_t rho = r0 + rr;
      bf16x8 qv = zero_frag(), gv = zero_frag();
      if (rho < nrows && d0 < D) {
        const int64_t tok = qidx[e_begin + rho / R];
        const int64_t th = tok * Hq + static_cast<int64_t>(g) * R + rho % R;
        qv = load_frag(q + th * D + d0);
        gv = load_frag(dout + th * D + d0);
      }
      *reinterpret_cast<uint4*>(sm.q_rm + rr * RS + d0) = __builtin_bit_cast(uint4, qv);
      *reinterpret_cast<uint4*>(sm.g_rm + rr * RS + d0) = __builtin_bit_cast(uint4, gv);
      store_transposed(sm.q_t, d0, rr, qv);
      store_transposed(sm.g_t, d0, rr, gv);
    }
    if (threadIdx.x < 32) {
      const int rr = threadIdx.x;
      const int64_t rho = r0 + rr;
      if (rho < nrows) {
        const int64_t tok = qidx[e_begin + rho / R];
        const int64_t th = tok * Hq + static_cast<int64_t>(g) * R + rho % R;
        const double* rs = row_state + th * 4;
        sm.lse[rr] = static_cast<float>(rs[0]);
        sm.mass[rr] = static_cast<float>(rs[1]);
        sm.center[rr] = static_cast<float>(rs[2]);
        sm.dhat[rr] = static_cast<float>(rs[3]);
        sm.tok[rr] = tok;
      } else {
        sm.lse[rr] = 0.f;
        sm.mass[rr] = 1.f;
        sm.center[rr] = 0.f;
        sm.dhat[rr] = 0.f;
        sm.tok[rr] = -1;  // masks every key
      }
    }
    __syncthreads();
    // ---- S = Q K^T and dP = dO V^T for 32 rows x this wave's 32 keys
    f32x4 sacc[2][2], dacc[2][2];  // [row tile][key tile]
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      bf16x8 qa[NK], ga[NK];
#pragma unroll
      for (int kk = 0; kk < NK; ++kk) {
        const int off = (16 * rt + c) * RS + 32 * kk + 8 * q4;
        qa[kk] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(sm.q_rm + off));
        ga[kk] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(sm.g_rm + off));
      }
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        f32x4 a = {0.f, 0.f, 0.f, 0.f}, b = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < NK; ++kk) {
          a = mfma(qa[kk], kf[kt][kk], a);
          b = mfma(ga[kk], vf[kt][kk], b);
        }
        sacc[rt][kt] = a;
        dacc[rt][kt] = b;
      }
    }
    // Lane (c, q4) holds S[row 16*rt + 4*q4 + i][key 16*kt + c] (and dP likewise).
    // ---- probabilities and dS per element, split into bf16 terms; element
    // 4*rt + i of a fragment is row pi(q4, 4*rt + i) = 16*rt + 4*q4 + i.
    Frag8 fph[2], fpm[2], fpl[2], fsh[2], fsm[2], fsl[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      const int64_t key = kb + 32 * wid + 16 * kt + c;
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int rr = 16 * rt + 4 * q4 + i;
          float p = 0.f, dsv = 0.f;
          if (key < kend && key <= sm.tok[rr]) {
            p = expf(sacc[rt][kt][i] * scale - sm.lse[rr]) / sm.mass[rr];
            dsv = p * ((dacc[rt][kt][i] - sm.center[rr]) - sm.dhat[rr]) * scale;
          }
          uint16_t a, b2, c2;
          split3(p, a, b2, c2);
          fph[kt].set(4 * rt + i, a);
          fpm[kt].set(4 * rt + i, b2);
          fpl[kt].set(4 * rt + i, c2);
          split3(dsv, a, b2, c2);
          fsh[kt].set(4 * rt + i, a);
          fsm[kt].set(4 * rt + i, b2);
          fsl[kt].set(4 * rt + i, c2);
        }
      }
    }
    bf16x8 ph[2], pm[2], pl[2], sh[2], smid[2], sl[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      ph[kt] = fph[kt].vec();
      pm[kt] = fpm[kt].vec();
      pl[kt] = fpl[kt].vec();
      sh[kt] = fsh[kt].vec();
      smid[kt] = fsm[kt].vec();
      sl[kt] = fsl[kt].vec();
    }
    // dV^T (dims x keys) += dO^T (dims x rows) . P (rows x keys) and
    // dK^T (dims x keys) += Q^T (dims x rows) . dS (rows x keys); the A operands
    // come from the transposed row tiles in the same row order pi(.).
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const bf16x8 ga_t = read_transposed(sm.g_t, dt * 16 + c, q4);
      const bf16x8 qa_t = read_transposed(sm.q_t, dt * 16 + c, q4);
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        acc_v[kt][dt] = mfma(ga_t, pl[kt], acc_v[kt][dt]);
        acc_v[kt][dt] = mfma(ga_t, pm[kt], acc_v[kt][dt]);
        acc_v[kt][dt] = mfma(ga_t, ph[kt], acc_v[kt][dt]);
        acc_k[kt][dt] = mfma(qa_t, sl[kt], acc_k[kt][dt]);
        acc_k[kt][dt] = mfma(qa_t, smid[kt], acc_k[kt][dt]);
        acc_k[kt][dt] = mfma(qa_t, sh[kt], acc_k[kt][dt]);
      }
    }
  }
  // acc_*[kt][dt] lane (c, q4) holds dX^T[dim dt*16 + 4*q4 + i][key 32*wid + 16*kt + c].
  const bool direct = n_items == 1;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
    const int kl = 32 * wid + 16 * kt + c;  // key offset in block
    const int64_t key = kb + kl;
    if (key >= kend) continue;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const int d0 = dt * 16 + 4 * q4;
      if (d0 >= D) continue;
      if (direct) {
        uint16_t hk[4], hv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          hk[i] = f32_to_bf16_bits(acc_k[kt][dt][i]);
          hv[i] = f32_to_bf16_bits(acc_v[kt][dt][i]);
        }
        const int64_t off = (key * G + g) * D + d0;
        if (dk)
          *reinterpret_cast<uint2*>(dk + off) =
              make_uint2(hk[0] | (static_cast<uint32_t>(hk[1]) << 16), hk[2] | (static_cast<uint32_t>(hk[3]) << 16));
        if (dv)
          *reinterpret_cast<uint2*>(dv + off) =
              make_uint2(hv[0] | (static_cast<uint32_t>(hv[1]) << 16), hv[2] | (static_cast<uint32_t>(hv[3]) << 16));
      } else {
        float* pk = partial + (item * 2 * 128 + kl) * DP + d0;
        float* pv = pk + 128 * DP;
        *reinterpret_cast<float4*>(pk) = make_float4(acc_k[kt][dt][0], acc_k[kt][dt][1], acc_k[kt][dt][2], acc_k[kt][dt][3]);
        *reinterpret_cast<float4*>(pv) = make_float4(acc_v[kt][dt][0], acc_v[kt][dt][1], acc_v[kt][dt][2], acc_v[kt][dt][3]);
      }
    }
  }
}

// Sums the fp32 partials of rows split into several items, in item order (fp64).
template <int NK>
__global__ __launch_bounds__(256) void attn_dkdv_finalize(const int32_t* __restrict__ cu,
                                                          const int32_t* __restrict__ cu_blocks,
                                                          const int32_t* __restrict__ item_start, int nseq,
                                                          int64_t rows, int G, int D, int B,
                                                          const float* __restrict__ partial, uint16_t* __restrict__ dk,
                                                          uint16_t* __restrict__ dv) {
  constexpr int DP = 32 * NK;
  const int64_t row = blockIdx.x;
  const int n = item_start[row + 1] - item_start[row];
  if (n <= 1) return;
  const int64_t gb = row / G;
  const int g = static_cast<int>(row % G);
  int s = upper_index(cu_blocks, nseq + 1, gb);
  while (s < nseq && cu_blocks[s + 1] <= gb) ++s;
  const int64_t start = cu[s], end = cu[s + 1];
  const int64_t kb = start + (gb - cu_blocks[s]) * B;
  const int64_t kend = kb + B < end ? kb + B : end;
  const int nk = static_cast<int>(kend - kb);
  for (int e = threadIdx.x; e < nk * DP; e += blockDim.x) {
    const int kl = e / DP, d = e % DP;
    if (d >= D) continue;
    double sk = 0.0, sv = 0.0;
    for (int it = 0; it < n; ++it) {
      const float* pk = partial + ((static_cast<int64_t>(item_start[row]) + it) * 2 * 128 + kl) * DP + d;
      sk += static_cast<double>(pk[0]);
      sv += static_cast<double>(pk[128 * DP]);
    }
    const int64_t off = ((kb + kl) * G + g) * D + d;
    if (dk) dk[off] = f32_to_bf16_bits(static_cast<float>(sk));
    if (dv) dv[off] = f32_to_bf16_bits(static_cast<float>(sv));
  }
}

// ---------------------------------------------------------------------------- host side

bool attn_mfma_supported(int64_t ratio, int64_t head_dim, int64_t block_size) {
  // ratio <= 512: one (edge, head) work item holds whole edges of at most 512 rows
  return ratio >= 1 && ratio <= 512 && head_dim >= 8 && head_dim <= 128 && head_dim % 8 == 0 && block_size >= 1 &&
         block_size <= 128;
}

static int nk_of(int D) { return D <= 32 ? 1 : (D <= 64 ? 2 : 4); }

int attn_fwd_mfma(const void* q, const void* k, const void* v, const int32_t* indices, const int32_t* cu, int nseq,
                  int64_t T, int Hq, int G, int D, int K, int B, float scale, void* out, float* lse, double* rs,
                  hipStream_t st) {
  const int R = Hq / G, nhc = (R + 15) / 16;
  const int64_t items = T * G * nhc;
  const dim3 grid(grid_1d(items, 4)), block(256);
  const auto* qb = static_cast<const uint16_t*>(q);
  const auto* kb = static_cast<const uint16_t*>(k);
  const auto* vb = static_cast<const uint16_t*>(v);
  auto* ob = static_cast<uint16_t*>(out);
  switch (nk_of(D)) {
    case 1: hipLaunchKernelGGL(attn_fwd_mfma_kernel<1>, grid, block, 0, st, qb, kb, vb, indices, cu, nseq, items, Hq, G, D, K, B, scale, ob, lse, rs); break;
    case 2: hipLaunchKernelGGL(attn_fwd_mfma_kernel<2>, grid, block, 0, st, qb, kb, vb, indices, cu, nseq, items, Hq, G, D, K, B, scale, ob, lse, rs); break;
    default: hipLaunchKernelGGL(attn_fwd_mfma_kernel<4>, grid, block, 0, st, qb, kb, vb, indices, cu, nseq, items, Hq, G, D, K, B, scale, ob, lse, rs); break;
  }
  return status_from(hipGetLastError());
}

int attn_bwd_dq_mfma(const void* q, const void* k, const void* v, const void* out, const void* dout, double* rs,
                     const int32_t* indices, const int32_t* cu, int nseq, int64_t T, int Hq, int G, int D, int K,
                     int B, float scale, void* dq, hipStream_t st) {
  const int R = Hq / G, nhc = (R + 15) / 16;
  const int64_t items = T * G * nhc;
  const dim3 grid(grid_1d(items, 4)), block(256);
  const auto* qb = static_cast<const uint16_t*>(q);
  const auto* kb = static_cast<const uint16_t*>(k);
  const auto* vb = static_cast<const uint16_t*>(v);
  const auto* ob = static_cast<const uint16_t*>(out);
  const auto* gb = static_cast<const uint16_t*>(dout);
  auto* dqb = static_cast<uint16_t*>(dq);
  switch (nk_of(D)) {
    case 1: hipLaunchKernelGGL(attn_dq_mfma_kernel<1>, grid, block, 0, st, qb, kb, vb, ob, gb, rs, indices, cu, nseq, items, Hq, G, D, K, B, scale, dqb); break;
    case 2: hipLaunchKernelGGL(attn_dq_mfma_kernel<2>, grid, block, 0, st, qb, kb, vb, ob, gb, rs, indices, cu, nseq, items, Hq, G, D, K, B, scale, dqb); break;
    default: hipLaunchKernelGGL(attn_dq_mfma_kernel<4>, grid, block, 0, st, qb, kb, vb, ob, gb, rs, indices, cu, nseq, items, Hq, G, D, K, B, scale, dqb); break;
  }
  return status_from(hipGetLastError());
}

static int64_t kv_max_items(int64_t T, int64_t G, int64_t K, int64_t total_blocks) {
  return total_blocks * G + (T * G * K) / kEdgeChunk + 1;
}

int64_t attn_dkdv_mfma_workspace_bytes(int64_t T, int64_t Hq, int64_t G, int64_t D, int64_t K, int64_t total_blocks,
                                       int64_t B) {
  (void)Hq;
  (void)B;
  const int64_t rows = total_blocks * G;
  const int64_t items = kv_max_items(T, G, K, total_blocks);
  const int64_t dp = 32 * nk_of(static_cast<int>(D));
  const int64_t scan_bytes = ((rows + 1) * 4 + 255) / 256 * 256;
  return scan_bytes + items * 2 * 128 * dp * 4;
}

int attn_bwd_dkdv_mfma(const void* q, const void* k, const void* v, const void* dout, const double* rs,
                       const int32_t* cu, const int32_t* cu_blocks, const int32_t* row_ptr, const int32_t* qidx,
                       int nseq, int64_t T, int Hq, int G, int D, int64_t total_blocks, int B, float scale, void* dk,
                       void* dv, void* ws, int64_t ws_bytes, hipStream_t st) {
  if (B > 128) return kErrUnsupported;
  const int64_t rows = total_blocks * G;
  if (rows == 0) return kOk;
  const int64_t scan_bytes = ((rows + 1) * 4 + 255) / 256 * 256;
  int32_t* item_start = static_cast<int32_t*>(ws);
  float* partial = reinterpret_cast<float*>(static_cast<char*>(ws) + scan_bytes);
  const int64_t dp = 32 * nk_of(D);
  const int64_t max_items = (ws_bytes - scan_bytes) / (2 * 128 * dp * 4);
  if (max_items < rows) return kErrInvalidArgument;
  hipLaunchKernelGGL(kv_item_scan, dim3(1), dim3(1024), 0, st, row_ptr, rows, kEdgeChunk, item_start);
  const dim3 grid(static_cast<unsigned>(max_items)), block(256);
  const auto* qb = static_cast<const uint16_t*>(q);
  const auto* kb = static_cast<const uint16_t*>(k);
  const auto* vb = static_cast<const uint16_t*>(v);
  const auto* gb = static_cast<const uint16_t*>(dout);
  auto* dkb = static_cast<uint16_t*>(dk);
  auto* dvb = static_cast<uint16_t*>(dv);
  switch (nk_of(D)) {
    case 1:
      hipLaunchKernelGGL(attn_dkdv_mfma_kernel<1>, grid, block, 0, st, qb, kb, vb, gb, rs, cu, cu_blocks, row_ptr, qidx, item_start, nseq, rows, Hq, G, D, B, scale, dkb, dvb, partial);
      hipLaunchKernelGGL(attn_dkdv_finalize<1>, dim3(static_cast<unsigned>(rows)), block, 0, st, cu, cu_blocks, item_start, nseq, rows, G, D, B, partial, dkb, dvb);
      break;
    case 2:
      hipLaunchKernelGGL(attn_dkdv_mfma_kernel<2>, grid, block, 0, st, qb, kb, vb, gb, rs, cu, cu_blocks, row_ptr, qidx, item_start, nseq, rows, Hq, G, D, B, scale, dkb, dvb, partial);
      hipLaunchKernelGGL(attn_dkdv_finalize<2>, dim3(static_cast<unsigned>(rows)), block, 0, st, cu, cu_blocks, item_start, nseq, rows, G, D, B, partial, dkb, dvb);
      break;
    default:
      hipLaunchKernelGGL(attn_dkdv_mfma_kernel<4>, grid, block, 0, st, qb, kb, vb, gb, rs, cu, cu_blocks, row_ptr, qidx, item_start, nseq, rows, Hq, G, D, B, scale, dkb, dvb, partial);
      hipLaunchKernelGGL(attn_dkdv_finalize<4>, dim3(static_cast<unsigned>(rows)), block, 0, st, cu, cu_blocks, item_start, nseq, rows, G, D, B, partial, dkb, dvb);
      break;
  }
  return status_from(hipGetLastError());
}

}  // namespace msa
