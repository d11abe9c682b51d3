// Stage 3 backward, KV-major (bf16 inputs).
//
// Notation per (token t, head h) row with selected keys j: x_j = fl(q.k_j * scale2)
// (scale2 = scale * log2 e), p_j = 2^(x_j - lse2) with the forward's base-2 lse,
// dp_j = dO . v_j, c = O . dO (bf16 output, fp64), and
//   mass = sum_j p_j,  delta = sum_j p_j (dp_j - c) / mass,
//   P_j = p_j / mass,  dS_j = P_j ((dp_j - c) - delta) * scale,
//   dQ = sum_j dS_j k_j,  dK_j = sum_rows dS_j q,  dV_j = sum_rows P_j dO.
// This is the reference's centred softmax derivative (tests/reference_fp64.py,
// triton/sparse_attention.py:96-197): delta is formed from the same p_j and dp_j
// as dS, so sum_j dS_j vanishes to rounding even when dp_j are large and close.
//
// Passes (query tokens in chunks, as in the forward):
//   center        c per row                                 (elementwise)
//   stats   (B1)  per (row, block): sum p, sum p (dp - c)    KV-major, rows per wave
//   combine       mass, delta per row (FP64, slot order)
//   main    (B2)  dK, dV per key block (registers) and dQ per (row, block)
//                 partials                                  KV-major, keys per wave
//   accumulate    dK, dV item partials -> FP32 key accumulators (item order)
//   dq combine    dQ = sum of the row's block partials (FP64, slot order)
//   finalize      FP32 key accumulators -> bf16 dK, dV
// No floating-point atomics; every sum has a fixed order.
#include "attn_kv_common.hpp"

// Logits are x = fl(acc * scale2) with their own rounding, and exponent arguments
// x - m with another: no fused multiply-adds, so a row's maximum gets p == 1 exactly.
#pragma clang fp contract(off)

namespace msa {

namespace {

constexpr int kStatRowsPerTile = 128;  // B1: (edge, head) rows per tile (4 waves x 32)
constexpr int kStatTilesPerItem = 4;
constexpr int kStatItemRows = kStatRowsPerTile * kStatTilesPerItem;
constexpr int kMainEdges = 512;        // B2: CSR edges per work item
constexpr int kMetaRows = 256;         // B2: row metadata staged per block of 8 tiles

template <int NK>
struct StatSmem {
  static constexpr int DP = 32 * NK;
  static constexpr int KS = DP + 8;
  alignas(16) uint16_t k[128 * KS];
  alignas(16) uint16_t v[128 * KS];
  int32_t th[kStatItemRows];
  int32_t tok[kStatItemRows];
  int32_t rec[kStatItemRows];
  float lse2[kStatItemRows];
  float cen[kStatItemRows];
};

template <int NK>
struct MainSmem {
  static constexpr int DP = 32 * NK;
  static constexpr int KS = DP + 8;   // row stride of the K block and of the Q / dO row tiles
  static constexpr int PS = 32 + 16;  // row stride of the dS planes [key][row]
  alignas(16) uint16_t k[128 * KS];   // K block [key][dim]
  alignas(16) uint16_t qs[32 * KS];   // Q rows [row][dim]
  alignas(16) uint16_t gs[32 * KS];   // dO rows
  alignas(16) uint16_t ds[3][128 * PS];  // dS split planes (hi, mid, lo) [key][row]
  float4 stats[kMetaRows];            // lse2, 1 / mass, c, delta
  int32_t th[kMetaRows];
  int32_t tok[kMetaRows];
  int32_t rec[kMetaRows];
};

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

}  // namespace

// c = O . dO per (token, head) in FP64 (exact products of bf16 values); 32 lanes per row.
__global__ __launch_bounds__(256) void kv_bwd_center(const uint16_t* __restrict__ out,
                                                     const uint16_t* __restrict__ dout, int64_t rows_th, int D,
                                                     double* __restrict__ row_state) {
  const int sub = threadIdx.x & 31;
  const int64_t th = static_cast<int64_t>(blockIdx.x) * 8 + (threadIdx.x >> 5);
  if (th >= rows_th) return;
  double acc = 0.0;
  for (int d0 = 4 * sub; d0 < D; d0 += 128) {
    const uint2 o = *reinterpret_cast<const uint2*>(out + th * D + d0);
    const uint2 g = *reinterpret_cast<const uint2*>(dout + th * D + d0);
    acc = fma(static_cast<double>(bf16_lo(o.x)), static_cast<double>(bf16_lo(g.x)), acc);
    acc = fma(static_cast<double>(bf16_hi(o.x)), static_cast<double>(bf16_hi(g.x)), acc);
    acc = fma(static_cast<double>(bf16_lo(o.y)), static_cast<double>(bf16_lo(g.y)), acc);
    acc = fma(static_cast<double>(bf16_hi(o.y)), static_cast<double>(bf16_hi(g.y)), acc);
  }
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 32);
  if (sub == 0) row_state[th * 4 + 2] = acc;
}

// B1: per (edge, head) row and key block, sum_j p_j and sum_j p_j (dp_j - c).
// Structure of the forward partial kernel: K and V blocks row-major in LDS,
// 4 waves x 32 rows per tile; S^T = K Q^T and dP^T = V dO^T (lane: row c, keys 4*q4 + i).
template <int NK, bool FULLD>
__global__ __launch_bounds__(256, 2) void kv_bwd_stats_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint16_t* __restrict__ dout, const double* __restrict__ row_state, const int32_t* __restrict__ cu,
    const int32_t* __restrict__ cu_blocks, const int32_t* __restrict__ qidx, const int32_t* __restrict__ sidx,
    const int32_t* __restrict__ e_hi, const int32_t* __restrict__ n_items, const int2* __restrict__ items, int nseq,
    int Hq, int G, int D, int K, int B, float scale2, int epi, int t0, float2* __restrict__ spart) {
  constexpr int DP = 32 * NK, KS = StatSmem<NK>::KS;
  __shared__ StatSmem<NK> sm;
  const int item = blockIdx.x;
  if (item >= *n_items) return;
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63, c = lane & 15, q4 = lane >> 4;
  const int2 it = items[item];
  const int row = it.x, e_begin = it.y;
  const RowGeom rg = row_geom(cu, cu_blocks, nseq, row, G, B);
  const int R = Hq / G;
  const int e_end = e_begin + epi < e_hi[row] ? e_begin + epi : e_hi[row];
  const int nrows = (e_end - e_begin) * R;  // 1 <= nrows <= kStatItemRows

  constexpr int KVI = 128 * (DP / 8) / 256;
  uint4 kw[KVI], vw[KVI];
#pragma unroll
  for (int i = 0; i < KVI; ++i) {
    const int e = tid + 256 * i;
    const int kl = e / (DP / 8), d0 = 8 * (e % (DP / 8));
    const int klc = kl < rg.nk ? kl : rg.nk - 1, d0c = (FULLD || d0 < D) ? d0 : D - 8;
    const int64_t off = ((rg.kb + klc) * G + rg.g) * D + d0c;
    kw[i] = *reinterpret_cast<const uint4*>(k + off);
    vw[i] = *reinterpret_cast<const uint4*>(v + off);
  }
  constexpr int MI = kStatItemRows / 256;
  int32_t mtok[MI], mslot[MI];
#pragma unroll
  for (int j = 0; j < MI; ++j) {
    const int rho = tid + 256 * j;
    const int eo = (rho < nrows ? rho : nrows - 1) / R;
    mtok[j] = qidx[e_begin + eo];
    mslot[j] = sidx[e_begin + eo];
  }
#pragma unroll
  for (int i = 0; i < KVI; ++i) {
    const int e = tid + 256 * i;
    const int kl = e / (DP / 8), d0 = 8 * (e % (DP / 8));
    const bool ok = kl < rg.nk && (FULLD || d0 < D);
    *reinterpret_cast<uint4*>(sm.k + kl * KS + d0) = ok ? kw[i] : make_uint4(0u, 0u, 0u, 0u);
    *reinterpret_cast<uint4*>(sm.v + kl * KS + d0) = ok ? vw[i] : make_uint4(0u, 0u, 0u, 0u);
  }
#pragma unroll
  for (int j = 0; j < MI; ++j) {
    const int rho = tid + 256 * j;
    if (rho < nrows) {
      const int eo = rho / R;
      const int h = rg.g * R + (rho - eo * R);
      const int th = mtok[j] * Hq + h;
      sm.th[rho] = th;
      sm.tok[rho] = mtok[j];
      sm.rec[rho] = ((mtok[j] - t0) * Hq + h) * K + mslot[j];
      sm.lse2[rho] = static_cast<float>(row_state[static_cast<int64_t>(th) * 4]);
      sm.cen[rho] = static_cast<float>(row_state[static_cast<int64_t>(th) * 4 + 2]);
    }
  }
  __syncthreads();

  const int ntiles = (nrows + kStatRowsPerTile - 1) / kStatRowsPerTile;
  for (int tile = 0; tile < ntiles; ++tile) {
    const int rbase = tile * kStatRowsPerTile + 32 * wid;
    if (rbase >= nrows) break;  // wave-uniform
    bf16x8 qf[2][NK], gf[2][NK];
    int lim[2];
    float lse2[2], cen[2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const int rho = rbase + 16 * rt + c;
      const bool ok = rho < nrows;
      const int64_t th = ok ? sm.th[rho] : 0;
      const int64_t vis = ok ? static_cast<int64_t>(sm.tok[rho]) - rg.kb + 1 : 0;
      lim[rt] = vis < rg.nk ? static_cast<int>(vis) : rg.nk;
      lse2[rt] = ok ? sm.lse2[rho] : 0.f;
      cen[rt] = ok ? sm.cen[rho] : 0.f;
#pragma unroll
      for (int kk = 0; kk < NK; ++kk) {
        const int d0 = 32 * kk + 8 * q4;
        const bool dok = ok && (FULLD || d0 < D);
        qf[rt][kk] = dok ? load_frag(q + th * D + d0) : zero_frag();
        gf[rt][kk] = dok ? load_frag(dout + th * D + d0) : zero_frag();
      }
    }
    float psum[2] = {0.f, 0.f}, usum[2] = {0.f, 0.f};
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) {
      bf16x8 kf[NK], vf[NK];
#pragma unroll
      for (int kk = 0; kk < NK; ++kk) {
        kf[kk] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(sm.k + (16 * kt + c) * KS + 32 * kk + 8 * q4));
        vf[kk] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(sm.v + (16 * kt + c) * KS + 32 * kk + 8 * q4));
      }
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        f32x4 sa = {0.f, 0.f, 0.f, 0.f}, da = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < NK; ++kk) {
          sa = mfma(kf[kk], qf[rt][kk], sa);
          da = mfma(vf[kk], gf[rt][kk], da);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const bool vis = 16 * kt + 4 * q4 + i < lim[rt];
          const float p = vis ? __builtin_amdgcn_exp2f(sa[i] * scale2 - lse2[rt]) : 0.f;
          psum[rt] += p;
          usum[rt] += p * (da[i] - cen[rt]);
        }
      }
    }
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      float a = psum[rt], b = usum[rt];
      a += __shfl_xor(a, 16, kWave);
      b += __shfl_xor(b, 16, kWave);
      a += __shfl_xor(a, 32, kWave);
      b += __shfl_xor(b, 32, kWave);
      const int rho = rbase + 16 * rt + c;
      if (q4 == 0 && rho < nrows) spart[sm.rec[rho]] = make_float2(a, b);
    }
  }
}

// mass = sum_s A_s, delta = sum_s B_s / mass over the row's valid slots (FP64);
// 32 lanes per (token, head), slots lane-parallel then a fixed shuffle tree.
__global__ __launch_bounds__(256) void kv_bwd_stats_combine(const int32_t* __restrict__ indices,
                                                            const int32_t* __restrict__ cu, int nseq, int64_t t0,
                                                            int64_t t1, int Hq, int G, int K, int B,
                                                            const float2* __restrict__ spart,
                                                            double* __restrict__ row_state) {
  const int sub = threadIdx.x & 31;
  const int64_t th = t0 * Hq + static_cast<int64_t>(blockIdx.x) * 8 + (threadIdx.x >> 5);
  if (th >= t1 * Hq) return;
  const int64_t t = th / Hq;
  const int h = static_cast<int>(th % Hq);
  const int g = h / (Hq / G);
  const int s = find_seq(cu, nseq, t);
  const int64_t qb = (t - cu[s]) / B;
  const int32_t* sel = indices + (t * G + g) * K;
  const int64_t rec0 = ((t - t0) * Hq + h) * static_cast<int64_t>(K);
  double a = 0.0, b = 0.0;
  for (int slot = sub; slot < K; slot += 32) {
    const int id = sel[slot];
    if (id >= 0 && id <= qb) {
      const float2 ab = spart[rec0 + slot];
      a += static_cast<double>(ab.x);
      b += static_cast<double>(ab.y);
    }
  }
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) {
    a += __shfl_xor(a, o, 32);
    b += __shfl_xor(b, o, 32);
  }
  if (sub == 0) {
    const bool has = a > 0.0;
    row_state[th * 4 + 1] = has ? a : 1.0;
    row_state[th * 4 + 3] = has ? b / a : 0.0;
  }
}

// B2: one workgroup per work item (key block row, <= kMainEdges edges); wave w owns
// keys 32w .. 32w + 31 of the block. Per 32-row tile (all waves, same rows):
//   S = Q K^T, dP = dO V^T (C[row][key]: lane = key c, rows 4*q4 + i),
//   dV += P^T dO and dK += dS^T Q (B operands read transposed from the row tiles),
//   dS -> three bf16 planes [key][row] in LDS, then dQ^T = K^T dS^T over all 128
//   keys for the wave's dim tiles (lane: row c, 4 consecutive dims) -> per-(row,
//   block) partial. The next tile's Q / dO rows are loaded during the current one.
template <int NK, bool FULLD>
__global__ __launch_bounds__(256, 1) void kv_bwd_main_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint16_t* __restrict__ dout, const double* __restrict__ row_state, const int32_t* __restrict__ cu,
    const int32_t* __restrict__ cu_blocks, const int32_t* __restrict__ qidx, const int32_t* __restrict__ sidx,
    const int32_t* __restrict__ e_hi, const int32_t* __restrict__ n_items, const int2* __restrict__ items, int nseq,
    int Hq, int G, int D, int K, int B, float scale2, float scale, int epi, int t0, float* __restrict__ dqpart,
    float* __restrict__ kvpart) {
  constexpr int DP = 32 * NK, NDT = DP / 16, KS = MainSmem<NK>::KS, PS = MainSmem<NK>::PS;
  constexpr int NQT = (NDT + 3) / 4;  // dQ dim tiles per wave
  constexpr int SI = 32 * (DP / 8) / 256 > 0 ? 32 * (DP / 8) / 256 : 1;  // 16-byte row loads per thread
  __shared__ MainSmem<NK> sm;
  const int item = blockIdx.x;
  if (item >= *n_items) return;
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63, c = lane & 15, q4 = lane >> 4;
  const int2 it = items[item];
  const int row = it.x, e_begin = it.y;
  const RowGeom rg = row_geom(cu, cu_blocks, nseq, row, G, B);
  const int R = Hq / G;
  const int e_end = e_begin + epi < e_hi[row] ? e_begin + epi : e_hi[row];
  const int nrows = (e_end - e_begin) * R;

  // ---- K / V fragments of this wave's keys (B operands of S and dP); K block in LDS
  bf16x8 kf[2][NK], vf[2][NK];
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
    const int kl = 32 * wid + 16 * kt + c;
    const int klc = kl < rg.nk ? kl : rg.nk - 1;
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) {
      const int d0 = 32 * kk + 8 * q4;
      const int d0c = (FULLD || d0 < D) ? d0 : D - 8;
      const int64_t off = ((rg.kb + klc) * G + rg.g) * D + d0c;
      const bool ok = kl < rg.nk && (FULLD || d0 < D);
      const bf16x8 kx = load_frag(k + off), vx = load_frag(v + off);
      kf[kt][kk] = ok ? kx : zero_frag();
      vf[kt][kk] = ok ? vx : zero_frag();
    }
  }
  {
    constexpr int KVI = 128 * (DP / 8) / 256;
    uint4 kw[KVI];
#pragma unroll
    for (int i = 0; i < KVI; ++i) {
      const int e = tid + 256 * i;
      const int kl = e / (DP / 8), d0 = 8 * (e % (DP / 8));
      const int klc = kl < rg.nk ? kl : rg.nk - 1, d0c = (FULLD || d0 < D) ? d0 : D - 8;
      kw[i] = *reinterpret_cast<const uint4*>(k + ((rg.kb + klc) * G + rg.g) * D + d0c);
    }
#pragma unroll
    for (int i = 0; i < KVI; ++i) {
      const int e = tid + 256 * i;
      const int kl = e / (DP / 8), d0 = 8 * (e % (DP / 8));
      const bool ok = kl < rg.nk && (FULLD || d0 < D);
      *reinterpret_cast<uint4*>(sm.k + kl * KS + d0) = ok ? kw[i] : make_uint4(0u, 0u, 0u, 0u);
    }
  }

  f32x4 dk[2][NDT], dv[2][NDT];
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) dk[kt][dt] = dv[kt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // 32 Q / dO rows of a tile: thread e covers row e % 32, dims 8 * (e / 32) .. +7
  uint4 qw[SI], gw[SI];
  auto load_rows = [&](int r0, int mb, int mend) {
#pragma unroll
    for (int i = 0; i < SI; ++i) {
      const int e = tid + 256 * i;
      const int rr = e & 31, d0 = 8 * (e >> 5);
      const int rho = r0 + rr < mend ? r0 + rr : mend - 1;
      const int d0c = d0 < DP ? ((FULLD || d0 < D) ? d0 : D - 8) : 0;
      const int64_t off = static_cast<int64_t>(sm.th[rho - mb]) * D + d0c;
      qw[i] = *reinterpret_cast<const uint4*>(q + off);
      gw[i] = *reinterpret_cast<const uint4*>(dout + off);
    }
  };
  auto store_rows = [&](int r0, int mend) {
#pragma unroll
    for (int i = 0; i < SI; ++i) {
      const int e = tid + 256 * i;
      const int rr = e & 31, d0 = 8 * (e >> 5);
      if (d0 < DP) {
        const bool ok = r0 + rr < mend && (FULLD || d0 < D);
        *reinterpret_cast<uint4*>(sm.qs + rr * KS + d0) = ok ? qw[i] : make_uint4(0u, 0u, 0u, 0u);
        *reinterpret_cast<uint4*>(sm.gs + rr * KS + d0) = ok ? gw[i] : make_uint4(0u, 0u, 0u, 0u);
      }
    }
  };

  for (int mb = 0; mb < nrows; mb += kMetaRows) {
    const int mend = mb + kMetaRows < nrows ? mb + kMetaRows : nrows;
    __syncthreads();  // previous metadata block no longer read (also publishes the K block on entry)
    if (tid < kMetaRows) {
      const int rho = mb + tid;
      if (rho < mend) {
        const int eo = rho / R;
        const int h = rg.g * R + (rho - eo * R);
        const int32_t tk = qidx[e_begin + eo];
        const int th = tk * Hq + h;
        const double* rs = row_state + static_cast<int64_t>(th) * 4;
        sm.th[tid] = th;
        sm.tok[tid] = tk;
        sm.rec[tid] = ((tk - t0) * Hq + h) * K + sidx[e_begin + eo];
        sm.stats[tid] = make_float4(static_cast<float>(rs[0]), static_cast<float>(1.0 / rs[1]),
                                    static_cast<float>(rs[2]), static_cast<float>(rs[3]));
      }
    }
    __syncthreads();
    load_rows(mb, mb, mend);

    for (int r0 = mb; r0 < mend; r0 += 32) {
      // All waves passed the previous tile's mid barrier: the row tiles are free.
      store_rows(r0, mend);
      __syncthreads();
      if (r0 + 32 < mend) load_rows(r0 + 32, mb, mend);

      // ---- S and dP: C[row 16*rt + 4*q4 + i][key 32*wid + 16*kt + c]
      f32x4 s[2][2], dp[2][2];
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        bf16x8 qa[NK], ga[NK];
#pragma unroll
        for (int kk = 0; kk < NK; ++kk) {
          qa[kk] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(sm.qs + (16 * rt + c) * KS + 32 * kk + 8 * q4));
          ga[kk] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(sm.gs + (16 * rt + c) * KS + 32 * kk + 8 * q4));
        }
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
          f32x4 a = {0.f, 0.f, 0.f, 0.f}, b = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kk = 0; kk < NK; ++kk) {
            a = mfma(qa[kk], kf[kt][kk], a);
            b = mfma(ga[kk], vf[kt][kk], b);
          }
          s[rt][kt] = a;
          dp[rt][kt] = b;
        }
      }
      // ---- P and dS (masked) as split bf16 A operands [key c][rows pi(q4, j)], j = 4*rt + i
      bf16x8 ap[2][3], ad[2][3];  // [kt][hi, mid, lo]
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        uint32_t ph[8], pm[8], pl[8], dh[8], dm[8], dl[8];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int rho = r0 + 16 * rt + 4 * q4 + i;
            const bool rok = rho < mend;
            const float4 st = sm.stats[(rok ? rho : mend - 1) - mb];
            const int64_t vis = rok ? static_cast<int64_t>(sm.tok[rho - mb]) - rg.kb + 1 : 0;
            const int kl = 32 * wid + 16 * kt + c;
            const bool ok = kl < vis && kl < rg.nk;
            const float p = ok ? __builtin_amdgcn_exp2f(s[rt][kt][i] * scale2 - st.x) : 0.f;
            const float P = p * st.y;
            const float dS = ok ? P * ((dp[rt][kt][i] - st.z) - st.w) * scale : 0.f;
            split3_bits(P, ph[4 * rt + i], pm[4 * rt + i], pl[4 * rt + i]);
            split3_bits(dS, dh[4 * rt + i], dm[4 * rt + i], dl[4 * rt + i]);
          }
        uint32_t w[3][4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          w[0][jj] = pack_hi16(dh[2 * jj], dh[2 * jj + 1]);
          w[1][jj] = pack_hi16(dm[2 * jj], dm[2 * jj + 1]);
          w[2][jj] = pack_hi16(dl[2 * jj], dl[2 * jj + 1]);
        }
#pragma unroll
        for (int pl3 = 0; pl3 < 3; ++pl3) {
          ad[kt][pl3] = __builtin_bit_cast(bf16x8, make_uint4(w[pl3][0], w[pl3][1], w[pl3][2], w[pl3][3]));
          // dS plane rows: key 32*wid + 16*kt + c, columns (rows) 16*rt + 4*q4 .. +3
          uint16_t* dst = sm.ds[pl3] + (32 * wid + 16 * kt + c) * PS + 4 * q4;
          *reinterpret_cast<uint2*>(dst) = make_uint2(w[pl3][0], w[pl3][1]);
          *reinterpret_cast<uint2*>(dst + 16) = make_uint2(w[pl3][2], w[pl3][3]);
        }
        ap[kt][0] = __builtin_bit_cast(bf16x8, make_uint4(pack_hi16(ph[0], ph[1]), pack_hi16(ph[2], ph[3]), pack_hi16(ph[4], ph[5]), pack_hi16(ph[6], ph[7])));
        ap[kt][1] = __builtin_bit_cast(bf16x8, make_uint4(pack_hi16(pm[0], pm[1]), pack_hi16(pm[2], pm[3]), pack_hi16(pm[4], pm[5]), pack_hi16(pm[6], pm[7])));
        ap[kt][2] = __builtin_bit_cast(bf16x8, make_uint4(pack_hi16(pl[0], pl[1]), pack_hi16(pl[2], pl[3]), pack_hi16(pl[4], pl[5]), pack_hi16(pl[6], pl[7])));
      }
      // ---- dV += P^T dO, dK += dS^T Q: B = X[rows pi(q4, j)][dim 16*dt + c], read transposed
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const bf16x8 gb = frag_tr(sm.gs, KS, 4 * q4, 16 + 4 * q4, 16 * dt, c);
        const bf16x8 qb = frag_tr(sm.qs, KS, 4 * q4, 16 + 4 * q4, 16 * dt, c);
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
          f32x4 a = dv[kt][dt];
          a = mfma(ap[kt][2], gb, a);
          a = mfma(ap[kt][1], gb, a);
          dv[kt][dt] = mfma(ap[kt][0], gb, a);
          f32x4 b = dk[kt][dt];
          b = mfma(ad[kt][2], qb, b);
          b = mfma(ad[kt][1], qb, b);
          dk[kt][dt] = mfma(ad[kt][0], qb, b);
        }
      }
      __syncthreads();  // dS planes complete; row tiles no longer read
      // ---- dQ^T = K^T dS^T for dim tiles dt = wid + 4 * n: C[dim 16*dt + 4*q4 + i][row 16*rt + c]
      if (wid < NDT) {
        f32x4 acc[NQT][2];
#pragma unroll
        for (int n = 0; n < NQT; ++n) acc[n][0] = acc[n][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kc = 0; kc < 4; ++kc) {
          bf16x8 ka[NQT];
#pragma unroll
          for (int n = 0; n < NQT; ++n) {
            const int dt = wid + 4 * n;
            ka[n] = dt < NDT ? frag_tr(sm.k, KS, 32 * kc + 8 * q4, 32 * kc + 8 * q4 + 4, 16 * dt, c) : zero_frag();
          }
#pragma unroll
          for (int rt = 0; rt < 2; ++rt) {
            const bf16x8 bl = frag_tr(sm.ds[2], PS, 32 * kc + 8 * q4, 32 * kc + 8 * q4 + 4, 16 * rt, c);
            const bf16x8 bm = frag_tr(sm.ds[1], PS, 32 * kc + 8 * q4, 32 * kc + 8 * q4 + 4, 16 * rt, c);
            const bf16x8 bh = frag_tr(sm.ds[0], PS, 32 * kc + 8 * q4, 32 * kc + 8 * q4 + 4, 16 * rt, c);
#pragma unroll
            for (int n = 0; n < NQT; ++n) {
              acc[n][rt] = mfma(ka[n], bl, acc[n][rt]);
              acc[n][rt] = mfma(ka[n], bm, acc[n][rt]);
              acc[n][rt] = mfma(ka[n], bh, acc[n][rt]);
            }
          }
        }
#pragma unroll
        for (int n = 0; n < NQT; ++n) {
          const int dt = wid + 4 * n;
#pragma unroll
          for (int rt = 0; rt < 2; ++rt) {
            const int rho = r0 + 16 * rt + c;
            const int d0 = 16 * dt + 4 * q4;
            if (dt < NDT && rho < mend && (FULLD || d0 < D))
              *reinterpret_cast<f32x4*>(dqpart + static_cast<int64_t>(sm.rec[rho - mb]) * D + d0) = acc[n][rt];
          }
        }
      }
    }
  }

  // ---- this item's dK / dV contribution: kvpart[item][0 = dK, 1 = dV][key][dim]
  float* base = kvpart + static_cast<int64_t>(item) * 2 * 128 * DP;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = 32 * wid + 16 * kt + 4 * q4 + i, d = 16 * dt + c;
        base[key * DP + d] = dk[kt][dt][i];
        base[128 * DP + key * DP + d] = dv[kt][dt][i];
      }
}

// For chunk c: add each row's item partials (in item order) into the FP32 key
// accumulators acc[0 = dK, 1 = dV][key][group][dim]. grid (rows, 128 * DP / 256).
template <int DP>
__global__ __launch_bounds__(256) void kv_bwd_accumulate(const int32_t* __restrict__ cu,
                                                         const int32_t* __restrict__ cu_blocks,
                                                         const int32_t* __restrict__ starts, int nseq, int G, int D,
                                                         int B, int64_t T, const float* __restrict__ kvpart,
                                                         float* __restrict__ acc) {
  const int64_t row = blockIdx.x;
  const int i0 = starts[row], i1 = starts[row + 1];
  if (i0 == i1) return;
  const RowGeom rg = row_geom(cu, cu_blocks, nseq, row, G, B);
  const int e = blockIdx.y * 256 + threadIdx.x;  // element of the 128 x DP block
  const int kl = e / DP, d = e % DP;
  if (kl >= rg.nk || d >= D) return;
  float sk = 0.f, sv = 0.f;
  for (int i = i0; i < i1; ++i) {
    const float* p = kvpart + static_cast<int64_t>(i) * 2 * 128 * DP;
    sk += p[kl * DP + d];
    sv += p[128 * DP + kl * DP + d];
  }
  const int64_t off = ((rg.kb + kl) * G + rg.g) * D + d;
  acc[off] += sk;
  acc[T * G * D + off] += sv;
}

// dQ = sum of the row's block partials over its valid slots (FP64, slot order); 32 lanes per row.
__global__ __launch_bounds__(256) void kv_bwd_dq_combine(const int32_t* __restrict__ indices,
                                                         const int32_t* __restrict__ cu, int nseq, int64_t t0,
                                                         int64_t t1, int Hq, int G, int D, int K, int B,
                                                         const float* __restrict__ dqpart,
                                                         uint16_t* __restrict__ dq) {
  const int sub = threadIdx.x & 31;
  const int64_t th = t0 * Hq + static_cast<int64_t>(blockIdx.x) * 8 + (threadIdx.x >> 5);
  if (th >= t1 * Hq) return;
  const int64_t t = th / Hq;
  const int h = static_cast<int>(th % Hq);
  const int g = h / (Hq / G);
  const int s = find_seq(cu, nseq, t);
  const int64_t qb = (t - cu[s]) / B;
  const int32_t* sel = indices + (t * G + g) * K;
  const int64_t rec0 = ((t - t0) * Hq + h) * static_cast<int64_t>(K);
  if (4 * sub >= D) return;
  double a0 = 0.0, a1 = 0.0, a2 = 0.0, a3 = 0.0;
  for (int slot = 0; slot < K; ++slot) {
    const int id = sel[slot];
    if (id < 0 || id > qb) continue;
    const float4 x = *reinterpret_cast<const float4*>(dqpart + (rec0 + slot) * D + 4 * sub);
    a0 += static_cast<double>(x.x);
    a1 += static_cast<double>(x.y);
    a2 += static_cast<double>(x.z);
    a3 += static_cast<double>(x.w);
  }
  const uint32_t w0 = f32_to_bf16_bits(static_cast<float>(a0)) | (static_cast<uint32_t>(f32_to_bf16_bits(static_cast<float>(a1))) << 16);
  const uint32_t w1 = f32_to_bf16_bits(static_cast<float>(a2)) | (static_cast<uint32_t>(f32_to_bf16_bits(static_cast<float>(a3))) << 16);
  *reinterpret_cast<uint2*>(dq + th * D + 4 * sub) = make_uint2(w0, w1);
}

__global__ __launch_bounds__(256) void kv_bwd_zero(float* __restrict__ p, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) p[i] = 0.f;
}

// FP32 key accumulators -> bf16 dK (acc[0]) and dV (acc[1]).
__global__ __launch_bounds__(256) void kv_bwd_finalize(const float* __restrict__ acc, int64_t n,
                                                       uint16_t* __restrict__ dk, uint16_t* __restrict__ dv) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  if (dk) dk[i] = f32_to_bf16_bits(acc[i]);
  if (dv) dv[i] = f32_to_bf16_bits(acc[n + i]);
}

// ---------------------------------------------------------------------------- host side

static int nk_of_dim(int D) { return D <= 32 ? 1 : (D <= 64 ? 2 : 4); }

struct BwdLayout {
  KvPlan stat_plan, main_plan;
  int64_t stat_base, main_base, spart, dqpart, kvpart, acc, total;
};

static BwdLayout bwd_layout(int64_t T, int64_t Hq, int64_t G, int64_t D, int64_t K, int64_t total_blocks) {
  BwdLayout b;
  const int64_t rows = total_blocks * G;
  const int64_t R = Hq / (G > 0 ? G : 1);
  const int64_t DP = 32 * nk_of_dim(static_cast<int>(D));
  const int64_t tc = kv_chunk_tokens(T, Hq, K, D * 4 + 8);
  int64_t sepi = static_cast<int64_t>(kStatItemRows) / (R > 0 ? R : 1);
  if (sepi < 1) sepi = 1;
  b.stat_plan = kv_plan_layout(T, rows, G, K, tc, sepi);
  b.main_plan = kv_plan_layout(T, rows, G, K, tc, kMainEdges);
  b.stat_base = 0;
  b.main_base = b.stat_plan.bytes;
  b.spart = b.main_base + b.main_plan.bytes;
  b.dqpart = b.spart + align256(tc * Hq * K * 8);
  b.kvpart = b.dqpart + align256(tc * Hq * K * D * 4);
  b.acc = b.kvpart + align256(b.main_plan.max_items * 2 * 128 * DP * 4);
  b.total = b.acc + align256(2 * T * G * D * 4);
  return b;
}

int64_t attn_bwd_kv_workspace_bytes(int64_t T, int64_t Hq, int64_t G, int64_t D, int64_t K, int64_t total_blocks) {
  return bwd_layout(T, Hq, G, D, K, total_blocks).total;
}

int attn_bwd_kv(const void* q, const void* k, const void* v, const void* out, const void* dout, double* rs,
                const int32_t* indices, const int32_t* cu, int nseq, int64_t T, int Hq, int G, int D, int K, int B,
                float scale, const int32_t* cu_blocks, int64_t total_blocks, const int32_t* row_ptr,
                const int32_t* qidx, const int32_t* sidx, void* dq, void* dk, void* dv, void* ws, int64_t ws_bytes,
                hipStream_t st) {
  const int64_t rows = total_blocks * G;
  const BwdLayout L = bwd_layout(T, Hq, G, D, K, total_blocks);
  if (ws_bytes < L.total) return kErrInvalidArgument;
  if (T * Hq * (K > 0 ? K : 1) >= (int64_t(1) << 31) || rows >= (int64_t(1) << 31)) return kErrUnsupported;
  if (T == 0) return kOk;
  char* base = static_cast<char*>(ws);
  void* sbase = base + L.stat_base;
  void* mbase = base + L.main_base;
  float2* spart = reinterpret_cast<float2*>(base + L.spart);
  float* dqpart = reinterpret_cast<float*>(base + L.dqpart);
  float* kvpart = reinterpret_cast<float*>(base + L.kvpart);
  float* acc = reinterpret_cast<float*>(base + L.acc);
  const auto* qb = static_cast<const uint16_t*>(q);
  const auto* kb = static_cast<const uint16_t*>(k);
  const auto* vb = static_cast<const uint16_t*>(v);
  const auto* ob = static_cast<const uint16_t*>(out);
  const auto* gb = static_cast<const uint16_t*>(dout);
  const float scale2 = scale * kLog2e;
  const int nk = nk_of_dim(D);
  const bool fd = D == 32 * nk;
  const int64_t nacc = T * G * D;
  const bool need_kv = dk != nullptr || dv != nullptr;

  hipLaunchKernelGGL(kv_bwd_center, dim3(grid_1d(T * Hq, 8)), dim3(256), 0, st, ob, gb, T * Hq, D, rs);
  if (need_kv) hipLaunchKernelGGL(kv_bwd_zero, dim3(grid_1d(2 * nacc, 256)), dim3(256), 0, st, acc, 2 * nacc);
  kv_plan_launch(L.stat_plan, row_ptr, qidx, T, sbase, st);
  kv_plan_launch(L.main_plan, row_ptr, qidx, T, mbase, st);
  const KvPlan& sp = L.stat_plan;
  const KvPlan& mp = L.main_plan;
  for (int64_t c = 0; c < sp.nch; ++c) {
    const int64_t t0 = c * sp.tc, t1 = t0 + sp.tc < T ? t0 + sp.tc : T;
    const int it0 = static_cast<int>(t0);
    if (rows > 0) {
      const int32_t* hi = kv_plan_hi(sp, sbase, c);
      const int32_t* nit = kv_plan_count(sp, sbase, c);
      const int2* its = kv_plan_items(sp, sbase, c);
      const int sepi = static_cast<int>(sp.epi);
      const dim3 grid(static_cast<unsigned>(sp.max_items)), block(256);
#define MSA_BWD_STATS(NKV, FD) hipLaunchKernelGGL((kv_bwd_stats_kernel<NKV, FD>), grid, block, 0, st, qb, kb, vb, gb, rs, cu, cu_blocks, qidx, sidx, hi, nit, its, nseq, Hq, G, D, K, B, scale2, sepi, it0, spart)
      if (nk == 1) { if (fd) MSA_BWD_STATS(1, true); else MSA_BWD_STATS(1, false); }
      else if (nk == 2) { if (fd) MSA_BWD_STATS(2, true); else MSA_BWD_STATS(2, false); }
      else { if (fd) MSA_BWD_STATS(4, true); else MSA_BWD_STATS(4, false); }
#undef MSA_BWD_STATS
    }
    hipLaunchKernelGGL(kv_bwd_stats_combine, dim3(grid_1d((t1 - t0) * Hq, 8)), dim3(256), 0, st, indices, cu, nseq,
                       t0, t1, Hq, G, K, B, spart, rs);
    if (rows > 0) {
      const int32_t* hi = kv_plan_hi(mp, mbase, c);
      const int32_t* nit = kv_plan_count(mp, mbase, c);
      const int2* its = kv_plan_items(mp, mbase, c);
      const int mepi = static_cast<int>(mp.epi);
      const dim3 grid(static_cast<unsigned>(mp.max_items)), block(256);
#define MSA_BWD_MAIN(NKV, FD) hipLaunchKernelGGL((kv_bwd_main_kernel<NKV, FD>), grid, block, 0, st, qb, kb, vb, gb, rs, cu, cu_blocks, qidx, sidx, hi, nit, its, nseq, Hq, G, D, K, B, scale2, scale, mepi, it0, dqpart, kvpart)
      if (nk == 1) { if (fd) MSA_BWD_MAIN(1, true); else MSA_BWD_MAIN(1, false); }
      else if (nk == 2) { if (fd) MSA_BWD_MAIN(2, true); else MSA_BWD_MAIN(2, false); }
      else { if (fd) MSA_BWD_MAIN(4, true); else MSA_BWD_MAIN(4, false); }
#undef MSA_BWD_MAIN
      if (need_kv) {
        const int32_t* starts = kv_plan_starts(mp, mbase, c);
        const dim3 agrid(static_cast<unsigned>(rows), static_cast<unsigned>(128 * 32 * nk / 256));
        if (nk == 1) hipLaunchKernelGGL(kv_bwd_accumulate<32>, agrid, dim3(256), 0, st, cu, cu_blocks, starts, nseq, G, D, B, T, kvpart, acc);
        else if (nk == 2) hipLaunchKernelGGL(kv_bwd_accumulate<64>, agrid, dim3(256), 0, st, cu, cu_blocks, starts, nseq, G, D, B, T, kvpart, acc);
        else hipLaunchKernelGGL(kv_bwd_accumulate<128>, agrid, dim3(256), 0, st, cu, cu_blocks, starts, nseq, G, D, B, T, kvpart, acc);
      }
    }
    if (dq)
      hipLaunchKernelGGL(kv_bwd_dq_combine, dim3(grid_1d((t1 - t0) * Hq, 8)), dim3(256), 0, st, indices, cu, nseq, t0,
                         t1, Hq, G, D, K, B, dqpart, static_cast<uint16_t*>(dq));
  }
  if (need_kv)
    hipLaunchKernelGGL(kv_bwd_finalize, dim3(grid_1d(nacc, 256)), dim3(256), 0, st, acc, nacc,
                       static_cast<uint16_t*>(dk), static_cast<uint16_t*>(dv));
  return status_from(hipGetLastError());
}

}  // namespace msa
