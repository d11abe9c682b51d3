// Stage 3 backward, KV-major (bf16 and fp16 inputs).
//
// Notation per (token t, head h) row with selected keys j: x_j = fl(q.k_j * scale2)
// (scale2 = scale * log2 e), p_j = 2^(x_j - lse2) with the forward's base-2 lse,
// dp_j = dO . v_j, c = O . dO (bf16 output, fp64), and
//   mass = sum_j p_j,  delta = sum_j p_j (dp_j - c) / mass,
//   P_j = p_j / mass,  dS_j = P_j ((dp_j - c) - delta),
//   dQ = scale sum_j dS_j k_j,  dK_j = scale sum_rows dS_j q,  dV_j = sum_rows P_j dO.
// This is the reference's centred softmax derivative (tests/reference_fp64.py,
// triton/sparse_attention.py:96-197): delta is formed from the same p_j and dp_j
// as dS, so sum_j dS_j vanishes to rounding even when dp_j are large and close.
//
// Passes (query tokens in chunks, as in the forward):
//   center        c per row                                 (elementwise)
//   stats   (B1)  per (row, block): sum p, sum p (dp - c)    KV-major, rows per wave
//   combine       mass, delta per row (FP64, slot order)
//   main    (B2)  dK, dV per key block (registers) and dQ per (row, block)
//                 partials                                  KV-major, 16 keys per wave
//   accumulate    dK, dV item partials -> FP32 key accumulators (item order);
//                 the last chunk writes bf16 dK (times scale), dV
//   dq combine    dQ = scale * sum of the row's block partials (FP64, slot order)
// No floating-point atomics; every sum has a fixed order. Partial records are
// written and read once each, with non-temporal (streaming) stores and loads.
#include <type_traits>

#include "attn_kv_common.hpp"
#include "profile.hpp"

// Logits are x = fl(acc * scale2) and exponent arguments fl(x - lse2), each with its
// own rounding and formed identically in the stats and main passes, so the p_j
// summed into mass and delta are the p_j of dS. Only explicit fmaf calls fuse.
#pragma clang fp contract(off)

namespace msa {

namespace {

// B1: 8 waves per workgroup, one 16-row group per wave and tile (102 VGPRs, so two
// workgroups give 4 waves per SIMD to hide the Q/dO fragment loads; 4 waves x 2 groups
// and 8 waves x 2 groups measured slower)
constexpr int kStatWaves = 8;
constexpr int kStatRT = 1;
constexpr int kStatThreads = 64 * kStatWaves;
constexpr int kStatRowsPerTile = 16 * kStatRT * kStatWaves;  // (edge, head) rows per tile
constexpr int kStatTilesPerItem = 512 / kStatRowsPerTile;
constexpr int kStatItemRows = kStatRowsPerTile * kStatTilesPerItem;
constexpr int kCenterRows = 2;  // rows per 32-lane segment of the centre pass (1: +7 %, 4: same as 2)
constexpr int kMainEdges = 512;        // B2: CSR edges per work item
constexpr int kMainThreads = 512;      // B2: 8 waves, 16 keys each (S, dP, dV, dK), 16 rows x 32 dims each (dQ)

// LDS rows of K / V blocks and of Q / dO tiles are DP + 16 halves apart (a 288-byte
// stride at DP = 128): both the row-fragment reads (ds_read_b128, lane c -> row c)
// and the transposed reads (ds_read_b64_tr_b16, four rows x 32 bytes per 16 lanes)
// then spread over all 64 banks. A DP + 8 stride leaves both 2-way conflicted.
template <int DP>
constexpr int lds_row_stride() { return DP + 16; }

// dS planes [key][tile row] are unpadded (64 bytes per key); the 8-byte piece p
// (tile rows 4p .. 4p + 3) of key k sits at piece p ^ ((k >> 1) & 7). The writes
// (lane c -> key c, pieces q4 and 4 + q4) and the transposed reads of the dQ pass
// (lanes c / 4 + 8 q4 -> keys, c % 4 -> pieces) then hit distinct banks (measured with
// SQ_LDS_BANK_CONFLICT: 0.18 conflict cycles per LDS instruction of the kernel with
// this swizzle, 0.44 with p ^ ((k >> 1) & 6), 2.6 unswizzled).
__device__ __forceinline__ int plane_offset(int key, int piece) { return key * 32 + 4 * (piece ^ ((key >> 1) & 7)); }

template <int NK>
struct StatSmem {
  static constexpr int DP = 32 * NK;
  static constexpr int KS = lds_row_stride<DP>();
  alignas(16) uint16_t k[128 * KS];
  alignas(16) uint16_t v[128 * KS];
  int32_t th[kStatItemRows];   // (token - t0) * Hq + head of each (compacted) row (chunk-local)
  int32_t rec[kStatItemRows];
  float lse2[kStatItemRows];
  float cen[kStatItemRows];
};

template <int NK>
struct MainSmem {
  static constexpr int DP = 32 * NK;
  static constexpr int KS = lds_row_stride<DP>();       // row stride of the K block and the Q / dO row tiles
  alignas(16) uint16_t k[128 * KS];                     // K block [key][dim]
  alignas(16) uint16_t qs[2][32 * KS];                  // Q rows of a tile [row][dim], double-buffered
  alignas(16) uint16_t gs[2][32 * KS];                  // dO rows
  alignas(16) uint16_t ds[2][3][128 * 32];              // dS split planes (hi, mid, lo) [key][row], swizzled
  alignas(16) float4 st[2][32];                         // (lse2, 1 / mass, c, delta) per tile row
  alignas(16) int32_t vis[2][32];                       // visible keys of the block per tile row (0 past the end)
  alignas(16) int32_t rec[2][32];                       // dQ partial record per tile row (-1 past the end)
  int32_t etok[kMainEdges];                             // the item's edges: query token and slot
  int32_t eslot[kMainEdges];
};

// 256 dims: the K block is read only while the item's register fragments are built, so
// it shares its LDS with the row tiles (exactly their size: 128 rows = 2 x 2 x 32 rows),
// 122 KiB in all instead of 190 (a barrier separates the last fragment read from the
// first tile's rows).
template <>
struct MainSmem<8> {
  static constexpr int DP = 256;
  static constexpr int KS = lds_row_stride<DP>();
  union {
    alignas(16) uint16_t k[128 * KS];
    struct {
      alignas(16) uint16_t qs[2][32 * KS];
      alignas(16) uint16_t gs[2][32 * KS];
    };
  };
  alignas(16) uint16_t ds[2][3][128 * 32];
  alignas(16) float4 st[2][32];
  alignas(16) int32_t vis[2][32];
  alignas(16) int32_t rec[2][32];
  int32_t etok[kMainEdges];
  int32_t eslot[kMainEdges];
};

}  // namespace

// O . dO per (token, head) in FP64 (exact products); 32 lanes per row, NR rows per
// 32-lane segment.
// Rows that take the statistics pass (all rows without o32; with o32 those the
// forward marked peaked, slot 1 < 0): c = O . dO of the rounded output, the
// center that pass refines. Other rows (flat, with o32, the forward's FP32
// output): delta = O . dO itself, kept as c = float(delta) plus the residual
// delta - c (slots 2 and 3).
template <int DT, int NR>
__global__ __launch_bounds__(256) void kv_bwd_center(const uint16_t* __restrict__ out, const float* __restrict__ o32,
                                                     const uint16_t* __restrict__ dout, int64_t rows_th, int D,
                                                     double* __restrict__ row_state) {
  const int sub = threadIdx.x & 31;
  // NR consecutive rows per 32-lane segment, all of their loads in flight together
  const int64_t th0 = (static_cast<int64_t>(blockIdx.x) * 8 + (threadIdx.x >> 5)) * NR;
  if (th0 >= rows_th) return;
  double acc[NR];
  bool flat[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int64_t th = th0 + r < rows_th ? th0 + r : rows_th - 1;
    flat[r] = o32 && row_state[th * 4 + 1] > 0.0;  // uniform over the row's 32 lanes
    acc[r] = 0.0;
  }
  for (int d0 = 4 * sub; d0 < D; d0 += 128) {
    uint2 g[NR];
    float o[NR][4];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const int64_t th = th0 + r < rows_th ? th0 + r : rows_th - 1;
      g[r] = *reinterpret_cast<const uint2*>(dout + th * D + d0);
      if (flat[r]) {
        const float4 x = *reinterpret_cast<const float4*>(o32 + th * D + d0);
        o[r][0] = x.x, o[r][1] = x.y, o[r][2] = x.z, o[r][3] = x.w;
      } else {
        const uint2 x = *reinterpret_cast<const uint2*>(out + th * D + d0);
        o[r][0] = lo16_f32<DT>(x.x), o[r][1] = hi16_f32<DT>(x.x), o[r][2] = lo16_f32<DT>(x.y), o[r][3] = hi16_f32<DT>(x.y);
      }
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      acc[r] = fma(static_cast<double>(o[r][0]), static_cast<double>(lo16_f32<DT>(g[r].x)), acc[r]);
      acc[r] = fma(static_cast<double>(o[r][1]), static_cast<double>(hi16_f32<DT>(g[r].x)), acc[r]);
      acc[r] = fma(static_cast<double>(o[r][2]), static_cast<double>(lo16_f32<DT>(g[r].y)), acc[r]);
      acc[r] = fma(static_cast<double>(o[r][3]), static_cast<double>(hi16_f32<DT>(g[r].y)), acc[r]);
    }
  }
#pragma unroll
  for (int r = 0; r < NR; ++r) {
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) acc[r] += __shfl_xor(acc[r], o, 32);
  }
  if (sub == 0) {
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const int64_t th = th0 + r;
      if (th < rows_th) {
        if (flat[r]) {
          const double c = static_cast<double>(static_cast<float>(acc[r]));
          row_state[th * 4 + 2] = c;
          row_state[th * 4 + 3] = acc[r] - c;
        } else {
          row_state[th * 4 + 2] = acc[r];
        }
      }
    }
  }
}

// B1: per (edge, head) row and key block, sum_j p_j and sum_j p_j (dp_j - c), for every
// row (all_rows) or for the rows the forward marked peaked (row_state slot 1 < 0).
// Structure of the forward partial kernel: K and V blocks row-major in LDS,
// kStatWaves waves x 16 kStatRT rows per tile; S^T = K Q^T and dP^T = V dO^T (lane: row c, keys 4*q4 + i).
template <int DT, int NK, bool FULLD>
__global__ __launch_bounds__(kStatThreads, NK == 8 ? 1 : 2) void kv_bwd_stats_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint16_t* __restrict__ dout, const double* __restrict__ row_state, const int32_t* __restrict__ cu,
    const int32_t* __restrict__ cu_blocks, const int32_t* __restrict__ qidx, const int32_t* __restrict__ sidx,
    const int32_t* __restrict__ e_hi, const int32_t* __restrict__ n_items, const int2* __restrict__ items, const int32_t* __restrict__ order, int nseq,
    int Hq, int G, int D, int K, int B, float scale2, int epi, int t0, int all_rows, float2* __restrict__ spart) {
  constexpr int DP = 32 * NK, KS = StatSmem<NK>::KS;
  __shared__ StatSmem<NK> sm;
  if (static_cast<int>(blockIdx.x) >= *n_items) return;
  const int item = order ? order[blockIdx.x] : static_cast<int>(blockIdx.x);  // no order: row order
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63, c = lane & 15, q4 = lane >> 4;
  const int2 it = items[item];
  const int row = it.x, e_begin = it.y;
  const RowGeom rg = row_geom(cu, cu_blocks, nseq, row, G, B);
  const int R = Hq / G;
  const int e_end = e_begin + epi < e_hi[row] ? e_begin + epi : e_hi[row];
  const int nrows = (e_end - e_begin) * R;  // 1 <= nrows <= kStatItemRows

  // The rows that take the pass, compacted in (edge, head) order (so still in token
  // order); the per-wave counts borrow the K block's LDS before it is filled.
  constexpr int MI = kStatItemRows / kStatThreads;
  int32_t* wcnt = reinterpret_cast<int32_t*>(sm.k);
  int nsel = 0;
#pragma unroll
  for (int j = 0; j < MI; ++j) {
    const int rho = tid + kStatThreads * j;
    bool take = false;
    int th = 0, rec = 0;
    float l2 = 0.f, ce = 0.f;
    if (rho < nrows) {
      const int eo = rho / R;
      const int h = rg.g * R + (rho - eo * R);
      const int tok = qidx[e_begin + eo];
      th = (tok - t0) * Hq + h;  // < tc * Hq (chunk records fit in int32, checked on the host)
      const double* rs = row_state + (static_cast<int64_t>(tok) * Hq + h) * 4;
      const double2 lm = *reinterpret_cast<const double2*>(rs);
      take = all_rows || lm.y < 0.0;
      rec = ((tok - t0) * Hq + h) * K + sidx[e_begin + eo];
      l2 = static_cast<float>(lm.x);
      ce = static_cast<float>(rs[2]);
    }
    const uint64_t bal = __ballot(take);
    if (lane == 0) wcnt[wid] = __popcll(bal);
    __syncthreads();
    int before = nsel, total = 0;
#pragma unroll
    for (int w = 0; w < kStatWaves; ++w) {
      const int n = wcnt[w];
      before += w < wid ? n : 0;
      total += n;
    }
    if (take) {
      const int pos = before + __popcll(bal & ((uint64_t(1) << lane) - 1));
      sm.th[pos] = th;
      sm.rec[pos] = rec;
      sm.lse2[pos] = l2;
      sm.cen[pos] = ce;
    }
    nsel += total;
    __syncthreads();  // counts read before the K block overwrites them
  }
  if (nsel == 0) return;  // workgroup-uniform

  constexpr int KVI = 128 * (DP / 8) / kStatThreads;
  uint4 kw[KVI], vw[KVI];
#pragma unroll
  for (int i = 0; i < KVI; ++i) {
    const int e = tid + kStatThreads * i;
    const int kl = e / (DP / 8), d0 = 8 * (e % (DP / 8));
    const int klc = kl < rg.nk ? kl : rg.nk - 1, d0c = (FULLD || d0 < D) ? d0 : D - 8;
    const int64_t off = ((rg.kb + klc) * G + rg.g) * D + d0c;
    kw[i] = *reinterpret_cast<const uint4*>(k + off);
    vw[i] = *reinterpret_cast<const uint4*>(v + off);
  }
#pragma unroll
  for (int i = 0; i < KVI; ++i) {
    const int e = tid + kStatThreads * i;
    const int kl = e / (DP / 8), d0 = 8 * (e % (DP / 8));
    const bool ok = kl < rg.nk && (FULLD || d0 < D);
    *reinterpret_cast<uint4*>(sm.k + kl * KS + d0) = ok ? kw[i] : make_uint4(0u, 0u, 0u, 0u);
    *reinterpret_cast<uint4*>(sm.v + kl * KS + d0) = ok ? vw[i] : make_uint4(0u, 0u, 0u, 0u);
  }
  __syncthreads();

  const int ntiles = (nsel + kStatRowsPerTile - 1) / kStatRowsPerTile;
  for (int tile = 0; tile < ntiles; ++tile) {
    const int rbase = tile * kStatRowsPerTile + 16 * kStatRT * wid;
    if (rbase >= nsel) break;  // wave-uniform
    bf16x8 qf[kStatRT][NK], gf[kStatRT][NK];
    int lim[kStatRT];
    float lse2[kStatRT], cen[kStatRT];
#pragma unroll
    for (int rt = 0; rt < kStatRT; ++rt) {
      const int rho = rbase + 16 * rt + c;
      const bool ok = rho < nsel;
      const int64_t th = ok ? static_cast<int64_t>(t0) * Hq + sm.th[rho] : 0;
      const int64_t vis = ok ? static_cast<int64_t>(t0) + sm.th[rho] / Hq - rg.kb + 1 : 0;
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
    float psum[kStatRT], usum[kStatRT];
#pragma unroll
    for (int rt = 0; rt < kStatRT; ++rt) psum[rt] = usum[rt] = 0.f;
    // rows are in token order: when every row of the wave sees all 128 keys, no masks
    bool fl = true;
#pragma unroll
    for (int rt = 0; rt < kStatRT; ++rt) fl = fl && lim[rt] >= 128;
    const bool full = __all(fl);
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) {
      bf16x8 kf[NK], vf[NK];
#pragma unroll
      for (int kk = 0; kk < NK; ++kk) {
        kf[kk] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(sm.k + (16 * kt + c) * KS + 32 * kk + 8 * q4));
        vf[kk] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(sm.v + (16 * kt + c) * KS + 32 * kk + 8 * q4));
      }
#pragma unroll
      for (int rt = 0; rt < kStatRT; ++rt) {
        f32x4 sa = {0.f, 0.f, 0.f, 0.f}, da = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < NK; ++kk) {
          sa = mfma_t<DT>(kf[kk], qf[rt][kk], sa);
          da = mfma_t<DT>(vf[kk], gf[rt][kk], da);
        }
        if (full) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float p = __builtin_amdgcn_exp2f(sa[i] * scale2 - lse2[rt]);
            psum[rt] += p;
            usum[rt] = __builtin_fmaf(p, da[i] - cen[rt], usum[rt]);
          }
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const bool vis = 16 * kt + 4 * q4 + i < lim[rt];
            const float p = vis ? __builtin_amdgcn_exp2f(sa[i] * scale2 - lse2[rt]) : 0.f;
            psum[rt] += p;
            usum[rt] = __builtin_fmaf(p, da[i] - cen[rt], usum[rt]);
          }
        }
      }
    }
#pragma unroll
    for (int rt = 0; rt < kStatRT; ++rt) {
      float a = psum[rt], b = usum[rt];
      a += __shfl_xor(a, 16, kWave);
      b += __shfl_xor(b, 16, kWave);
      a += __shfl_xor(a, 32, kWave);
      b += __shfl_xor(b, 32, kWave);
      const int rho = rbase + 16 * rt + c;
      if (q4 == 0 && rho < nsel) spart[sm.rec[rho]] = make_float2(a, b);
    }
  }
}

// The main pass's per-row record (lse2, 1 / mass, c, w) in fp32, from the fp64 row state:
// p = 2^(x - lse2) / mass and dS = P ((dp - c) - w).
__device__ __forceinline__ float4 main_row_record(double lse2, double mass, double c, double w) {
  return make_float4(static_cast<float>(lse2), static_cast<float>(1.0 / fabs(mass)), static_cast<float>(c),
                     static_cast<float>(w));
}

// mass = sum_s A_s, delta = sum_s B_s / mass over the row's valid slots (FP64);
// 32 lanes per (token, head), slots lane-parallel then a fixed shuffle tree. Rows
// outside the pass (flat rows, unless all_rows) keep the forward's mass. The mass
// keeps the sign of the forward's mark, so a repeated backward selects the same rows.
// Every row of the chunk then gets the main pass's fp32 record in rowf. A 32-lane
// segment owns rps consecutive rows (32 when only the forward's peaked rows take the
// pass, 1 when all do): each lane settles its own row if it is outside the pass, then
// the segment takes its rows in the pass one after the other.
__global__ __launch_bounds__(256) void kv_bwd_stats_combine(const int32_t* __restrict__ indices,
                                                            const int32_t* __restrict__ cu, int nseq, int64_t t0,
                                                            int64_t t1, int Hq, int G, int K, int B, int all_rows,
                                                            int rps, const float2* __restrict__ spart,
                                                            double* __restrict__ row_state,
                                                            float4* __restrict__ rowf) {
  const int sub = threadIdx.x & 31;
  const int64_t base = t0 * Hq + (static_cast<int64_t>(blockIdx.x) * 8 + (threadIdx.x >> 5)) * rps;
  const int64_t end = t1 * Hq;
  bool in_pass = false;
  if (sub < rps && base + sub < end) {
    const int64_t th = base + sub;
    const double4 rs = *reinterpret_cast<const double4*>(row_state + th * 4);
    in_pass = all_rows || !(rs.y > 0.0);
    if (!in_pass) rowf[th] = main_row_record(rs.x, rs.y, rs.z, rs.w);
  }
  // this segment's rows in the pass (bits of its half of the wave)
  uint32_t todo = static_cast<uint32_t>(__ballot(in_pass) >> (threadIdx.x & 32));
  while (todo) {
    const int j = __builtin_ctz(todo);
    todo &= todo - 1;
    const int64_t th = base + j;
    const double mark = row_state[th * 4 + 1];
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
      const double mass = copysign(has ? a : 1.0, mark), delta = has ? b / a : 0.0;
      row_state[th * 4 + 1] = mass;
      row_state[th * 4 + 3] = delta;
      rowf[th] = main_row_record(row_state[th * 4], mass, row_state[th * 4 + 2], delta);
    }
  }
}

// One workgroup (8 waves) per work item: a key block row and <= kMainEdges of its
// edges, i.e. nrows = edges x (Hq / G) query rows, processed in tiles of 32 rows.
// Wave w owns keys 16w .. 16w + 15 of the block. Per tile:
//   S = Q K^T, dP = dO V^T     C[row 16 rt + 4 q4 + i][key c] (A: Q / dO rows from LDS,
//                              B: this wave's K / V fragments, in registers)
//   P = p / mass, dS           exact 3-way bf16 splits; A operands of dV / dK come
//                              straight from the C registers (rows permuted by pi)
//   dV += P^T dO, dK += dS^T Q B operands read transposed from the row tiles
//   dS planes -> LDS [key][row]; barrier
//   dQ^T = K^T dS^T            wave (rh, dq): rows 16 rh .. +15, dims 32 dq .. +31,
//                              K^T fragments in registers -> per-(row, block) partial
// Row tiles and dS planes are double-buffered, so one barrier per tile orders all
// LDS traffic; the next tile's rows are committed before it and the one after is
// loaded from memory during the current tile.
// PARTS selects the outputs: kPartAll (dK, dV and dQ) up to 128 dims; at 256 dims each
// 128-dim half takes a kPartKV launch, and dQ a kPartQ launch per half for fp16, one for
// both halves for bf16 (all three outputs in one launch exceed the registers of a wave
// there), each recomputing S and dP over every dim.
enum MainParts : int { kPartKV = 1, kPartQ = 2, kPartAll = 3 };
template <int DT, int NK, bool FULLD, int PARTS>
__global__ __launch_bounds__(kMainThreads, 1) void kv_bwd_main_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint16_t* __restrict__ dout, const double* __restrict__ row_state, const int32_t* __restrict__ cu,
    const int32_t* __restrict__ cu_blocks, const int32_t* __restrict__ qidx, const int32_t* __restrict__ sidx,
    const int32_t* __restrict__ e_hi, const int32_t* __restrict__ n_items, const int2* __restrict__ items,
    const int32_t* __restrict__ order, int nseq, int Hq, int G, int D, int K, int B, float scale2, int epi, int t0,
    uint32_t rmagic, int rshift, const float4* __restrict__ rowf, float* __restrict__ dqpart,
    float* __restrict__ kvpart, int dhalf) {
  // DP dims enter S and dP; the dK, dV and dQ outputs of one launch cover DPO dims from
  // dhalf (256 dims: launches for dhalf = 0 and 128)
  constexpr bool DO_KV = (PARTS & kPartKV) != 0, DO_Q = (PARTS & kPartQ) != 0;
  constexpr int DP = 32 * NK, DPO = NK == 8 ? 128 : DP, NDT = DPO / 16, KS = MainSmem<NK>::KS;
  if constexpr (NK != 8) dhalf = 0;  // (compile-time zero below 256 dims)
  constexpr int RV = DP / 8;             // 16-byte chunks per row
  constexpr int CPT = RV >= 8 ? RV / 8 : 1;  // chunks per staging thread (threads 0-255: Q, 256-511: dO)
  constexpr int TPR = RV / CPT;          // staging threads per row
  __shared__ MainSmem<NK> sm;
  if (static_cast<int>(blockIdx.x) >= *n_items) return;
  const int item = order[blockIdx.x];  // largest items first
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63, c = lane & 15, q4 = lane >> 4;
  const int2 it = items[item];
  const int row = it.x, e_begin = it.y;
  const RowGeom rg = row_geom(cu, cu_blocks, nseq, row, G, B);
  const int R = Hq / G;
  const int e_end = e_begin + epi < e_hi[row] ? e_begin + epi : e_hi[row];
  const int ne = e_end - e_begin;
  const int nrows = ne * R;
  const int ntiles = (nrows + 31) >> 5;
  if (nrows <= 0) return;  // (the plan emits no empty items; whole workgroup)

  // ---- item set-up: edges and the K block in LDS, V fragments of this wave's keys
  for (int e = tid; e < ne; e += kMainThreads) {
    sm.etok[e] = qidx[e_begin + e];
    sm.eslot[e] = sidx[e_begin + e];
  }
  {
    constexpr int KVI = (128 * RV + kMainThreads - 1) / kMainThreads;
    uint4 kw[KVI];
#pragma unroll
    for (int i = 0; i < KVI; ++i) {
      const int e = tid + kMainThreads * i;
      const int kl = (e < 128 * RV ? e : 0) / RV, d0 = 8 * (e % RV);
      const int klc = kl < rg.nk ? kl : rg.nk - 1, d0c = (FULLD || d0 < D) ? d0 : D - 8;
      kw[i] = *reinterpret_cast<const uint4*>(k + ((rg.kb + klc) * G + rg.g) * D + d0c);
    }
#pragma unroll
    for (int i = 0; i < KVI; ++i) {
      const int e = tid + kMainThreads * i;
      if ((128 * RV) % kMainThreads == 0 || e < 128 * RV) {
        const int kl = e / RV, d0 = 8 * (e % RV);
        const bool ok = kl < rg.nk && (FULLD || d0 < D);
        *reinterpret_cast<uint4*>(sm.k + kl * KS + d0) = ok ? kw[i] : make_uint4(0u, 0u, 0u, 0u);
      }
    }
  }
  // B operands of dP and S: V / K[key 16 w + c][dims 32 kk + 8 q4 + j], from memory (K at
  // 256 dims too: its LDS block is shared with the row tiles)
  bf16x8 vf[NK], kf[NK];
  const int kl_own = 16 * wid + c;
  const int64_t own_off = ((rg.kb + (kl_own < rg.nk ? kl_own : rg.nk - 1)) * G + rg.g) * D;
  auto load_own = [&](const uint16_t* base, bf16x8* f) __attribute__((always_inline)) {
    const uint16_t* p = base + own_off;
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) {
      const int d0 = 32 * kk + 8 * q4;
      const int d0c = (FULLD || d0 < D) ? d0 : D - 8;
      const bf16x8 x = load_frag(p + d0c);
      f[kk] = kl_own < rg.nk && (FULLD || d0 < D) ? x : zero_frag();
    }
  };
  load_own(v, vf);
  if constexpr (NK == 8) load_own(k, kf);
  __syncthreads();  // K block and edges visible

  if constexpr (NK != 8) {
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) kf[kk] = load_frag(sm.k + (16 * wid + c) * KS + 32 * kk + 8 * q4);
  }
  const int rh = wid >> 2, dq = wid & 3;
  const bool dq_active = 32 * dq < DPO;
  // dQ dims of this wave: NQ 16-dim tiles, qdim(dt2) + c. A bf16 dQ-only launch at 256 dims
  // covers both 128-dim halves (dims 32 dq .. + 31 of each), the others 32 dims of one.
  constexpr int NQ = (NK == 8 && PARTS == kPartQ && DT == kBF16) ? 4 : 2;
  auto qdim = [&](int dt2) { return dhalf + 128 * (dt2 >> 1) + 32 * dq + 16 * (dt2 & 1); };
  // A operand of dQ^T (a bf16 product, dS entering as bf16 planes for either input type):
  // K^T[dim qdim(dt2) + c][keys 32 kc + 8 q4 + j]; fp16 K as two exact bf16 terms (kt the
  // high terms, ktl the low ones).
  bf16x8 kt[NQ][4], ktl[NQ][4];
#pragma unroll
  for (int dt2 = 0; dt2 < (DO_Q ? NQ : 0); ++dt2)
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
      const bf16x8 x =
          dq_active ? frag_tr(sm.k, KS, 32 * kc + 8 * q4, 32 * kc + 8 * q4 + 4, qdim(dt2), c) : zero_frag();
      if constexpr (DT == kF16) {
        const uint4 w = __builtin_bit_cast(uint4, x);
        uint4 h, l;
        f16_pair_to_bf16_terms(w.x, h.x, l.x);
        f16_pair_to_bf16_terms(w.y, h.y, l.y);
        f16_pair_to_bf16_terms(w.z, h.z, l.z);
        f16_pair_to_bf16_terms(w.w, h.w, l.w);
        kt[dt2][kc] = __builtin_bit_cast(bf16x8, h);
        ktl[dt2][kc] = __builtin_bit_cast(bf16x8, l);
      } else {
        kt[dt2][kc] = x;
      }
    }

  // ---- row staging: a tile is 32 rows of Q (threads 0-255) and of dO (threads 256-511);
  // TPR threads per row, each CPT 16-byte chunks TPR apart (per load, the row's threads
  // cover contiguous bytes: the LDS writes are then free of bank conflicts, 0.18 -> 0.003
  // conflict cycles per LDS instruction of the kernel), so a thread forms one row
  // address per tile. The first thread of each Q row also fetches the row's fp32 record
  // (rowf), its visible keys and its dQ record (spread over waves 0-3).
  const int lt = tid & 255;
  const int srow = lt / TPR;  // tile row of this thread
  const bool stager = srow < 32;
  const int sc0 = lt % TPR;  // first chunk; then sc0 + TPR, ...
  const bool meta_thread = tid < 256 && stager && (lt % TPR) == 0;
  const uint16_t* src = tid < 256 ? q : dout;
  uint4 pf[CPT];
  float4 pst = make_float4(0.f, 1.f, 0.f, 0.f);
  int prec = -1, pvis = 0;
#define MSA_MAIN_ISSUE(R0)                                                                                  \
  if (stager) {                                                                                             \
    const int rho = (R0) + srow < nrows ? (R0) + srow : nrows - 1;                                          \
    const int eo = rshift >= 0 ? rho >> rshift : div_by_ratio(rho, rmagic);                                 \
    const int h = rg.g * R + (rho - eo * R);                                                                \
    const int tk = sm.etok[eo];                                                                             \
    const int64_t th = static_cast<int64_t>(tk) * Hq + h;                                                   \
    const uint16_t* rowp = src + th * D;                                                                    \
    _Pragma("unroll") for (int j = 0; j < CPT; ++j) {                                                       \
      const int d0 = 8 * (sc0 + TPR * j);                                                                   \
      pf[j] = *reinterpret_cast<const uint4*>(rowp + ((FULLD || d0 < D) ? d0 : D - 8));                     \
    }                                                                                                       \
    if (meta_thread) {                                                                                      \
      if ((R0) + srow < nrows) {                                                                            \
        pst = rowf[th];                                                                                     \
        prec = ((tk - t0) * Hq + h) * K + sm.eslot[eo];                                                     \
        const int64_t vk = static_cast<int64_t>(tk) - rg.kb + 1;                                            \
        pvis = vk < rg.nk ? static_cast<int>(vk) : rg.nk;                                                   \
      } else {                                                                                              \
        pst = make_float4(0.f, 1.f, 0.f, 0.f);                                                              \
        prec = -1;                                                                                          \
        pvis = 0;                                                                                           \
      }                                                                                                     \
    }                                                                                                       \
  }
#define MSA_MAIN_COMMIT(R0, BUF)                                                                            \
  if (stager) {                                                                                             \
    uint16_t* dstt = (tid < 256 ? sm.qs[BUF] : sm.gs[BUF]) + srow * KS;                                     \
    const bool rok = (R0) + srow < nrows;                                                                   \
    _Pragma("unroll") for (int j = 0; j < CPT; ++j) {                                                       \
      const int d0 = 8 * (sc0 + TPR * j);                                                                   \
      const bool ok = rok && (FULLD || d0 < D);                                                             \
      *reinterpret_cast<uint4*>(dstt + d0) = ok ? pf[j] : make_uint4(0u, 0u, 0u, 0u);                       \
    }                                                                                                       \
    if (meta_thread) {                                                                                      \
      sm.st[BUF][srow] = pst;                                                                               \
      sm.vis[BUF][srow] = pvis;                                                                             \
      sm.rec[BUF][srow] = prec;                                                                             \
    }                                                                                                       \
  }

  f32x4 dk[NDT], dv[NDT];  // C[key 16 w + 4 q4 + i][dim 16 dt + c]
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) dk[dt] = dv[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  // fp16: dS enters dK as fp16 terms of 2^ks dS, ks per key (this lane's key c) from the
  // running maximum kmax of |dS| over the item's tiles so far: 2^ks kmax < 2^15, so ks
  // only decreases (the key's accumulators are then rescaled, exactly). dk holds
  // 2^ks dK and dv 2^15 dV until the item's partial is stored.
  float kmax = 0.f;
  int ks = 15;

  MSA_MAIN_ISSUE(0)
  if constexpr (NK == 8) __syncthreads();  // the K block's LDS becomes the row tiles
  MSA_MAIN_COMMIT(0, 0)
  if (ntiles > 1) MSA_MAIN_ISSUE(32)
  __syncthreads();

  // dQ^T = K^T dS^T of the tile whose planes sit in buffer PB, into ACC[NQ]:
  // C[dim qdim(dt2) + 4 q4 + i][row 16 rh + c]
#define MSA_DQ_PRODUCTS(PB, ACC)                                                                          \
  _Pragma("unroll") for (int dt2 = 0; dt2 < NQ; ++dt2) ACC[dt2] = f32x4{0.f, 0.f, 0.f, 0.f};                \
  _Pragma("unroll") for (int kc = 0; kc < 4; ++kc) {                                                      \
    /* B[keys 32 kc + 8 q4 + j][tile rows 16 rh + c]: lane c reads key (.. + c / 4), piece 4 rh + c % 4 */  \
    const int ka = 32 * kc + 8 * q4 + (c >> 2), kb = ka + 4;                                              \
    const int oa = plane_offset(ka, 4 * rh + (c & 3)), ob = plane_offset(kb, 4 * rh + (c & 3));           \
    const bf16x8 bl = frag_tr_at(sm.ds[PB][2] + oa, sm.ds[PB][2] + ob);                                   \
    const bf16x8 bm = frag_tr_at(sm.ds[PB][1] + oa, sm.ds[PB][1] + ob);                                   \
    const bf16x8 bh = frag_tr_at(sm.ds[PB][0] + oa, sm.ds[PB][0] + ob);                                   \
    _Pragma("unroll") for (int dt2 = 0; dt2 < NQ; ++dt2) {                                                \
      if constexpr (DT == kF16) {                                                                         \
        /* (Kh + Kl)(Dh + Dm + Dl), the smaller products first; Kl Dl (|Kl| <= 2^-8 |K|, |Dl| <       \
           2^-14 |dS|) lies below 2^-22 of K dS, the order of the fp32 sums' own rounding, and is left \
           out (bit-identical dQ at the benchmark's c4 shape) */                                          \
        ACC[dt2] = mfma(ktl[dt2][kc], bm, ACC[dt2]);                                                      \
        ACC[dt2] = mfma(kt[dt2][kc], bl, ACC[dt2]);                                                       \
        ACC[dt2] = mfma(ktl[dt2][kc], bh, ACC[dt2]);                                                      \
      } else {                                                                                            \
        ACC[dt2] = mfma(kt[dt2][kc], bl, ACC[dt2]);                                                       \
      }                                                                                                   \
      ACC[dt2] = mfma(kt[dt2][kc], bm, ACC[dt2]);                                                         \
      ACC[dt2] = mfma(kt[dt2][kc], bh, ACC[dt2]);                                                         \
    }                                                                                                     \
  }
  auto dq_store = [&](int rec, const f32x4 (&acc)[NQ]) __attribute__((always_inline)) {
    if (rec >= 0) {
#pragma unroll
      for (int dt2 = 0; dt2 < NQ; ++dt2) {
        const int d0 = qdim(dt2) + 4 * q4;
        if (FULLD || d0 < D)
          __builtin_nontemporal_store(acc[dt2], reinterpret_cast<f32x4*>(dqpart + static_cast<uint32_t>(rec * D + d0)));
      }
    }
  };
  // LAG (bf16, 128 dims, all outputs): tile t - 1's dQ products are issued among tile t's
  // P / dS arithmetic (its planes stay in the other buffer until the barrier that ends tile
  // t), so that a wave's MFMA and VALU work overlap (main pass 6.02 -> 5.84 ms at c4); the
  // last tile's dQ follows the loop.
  constexpr bool LAG = DT == kBF16 && NK == 4 && PARTS == kPartAll;
  int myrec_prev = -1;
  const int key = 16 * wid + c;
  for (int t = 0; t < ntiles; ++t) {
    const int b = t & 1;
    // ---- S and dP: C[row 16 rt + 4 q4 + i][key c]
    f32x4 s[2], dp[2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      f32x4 a = {0.f, 0.f, 0.f, 0.f}, g = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < NK; ++kk) {
        const bf16x8 qa = load_frag(sm.qs[b] + (16 * rt + c) * KS + 32 * kk + 8 * q4);
        const bf16x8 ga = load_frag(sm.gs[b] + (16 * rt + c) * KS + 32 * kk + 8 * q4);
        a = mfma_t<DT>(qa, kf[kk], a);
        g = mfma_t<DT>(ga, vf[kk], g);
      }
      s[rt] = a;
      dp[rt] = g;
    }
    // ---- P and dS, split into three bf16 terms; element j = 4 rt + i is row pi(q4, j)
    const int myrec = sm.rec[b][16 * rh + c];  // read before the barrier: the buffer is refilled after it
    const bool full = 32 * t + 32 <= nrows && sm.vis[b][0] >= 16 * wid + 16;  // rows are in token order
    // bf16: P and dS as three bf16 terms (ph.., dh..); fp16: dS as bf16 terms for the dQ
    // planes, P and dS kept (Pv, Dv; element j = 4 rt + i) for their fp16 splits below
    uint32_t ph[8], pm[8], pl[8], dh[8], dm[8], dl[8];
    float Pv[8], Dv[8];
    // rows 16 rt + 4 q4 + i of this lane; FULL: every row sees the wave's 16 keys (no masks)
    auto pds_rows = [&](int rt, auto full_tag) __attribute__((always_inline)) {
      constexpr bool FULL = decltype(full_tag)::value;
      float4 stv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) stv[i] = sm.st[b][16 * rt + 4 * q4 + i];
      auto keep = [&](int i, float P, float d) __attribute__((always_inline)) {
        if constexpr (DT == kF16) {
          Pv[4 * rt + i] = P, Dv[4 * rt + i] = d;
        } else {
          if constexpr (DO_KV) split3_bits(P, ph[4 * rt + i], pm[4 * rt + i], pl[4 * rt + i]);
          split3_bits(d, dh[4 * rt + i], dm[4 * rt + i], dl[4 * rt + i]);
        }
      };
      if constexpr (FULL) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float P = __builtin_amdgcn_exp2f(s[rt][i] * scale2 - stv[i].x) * stv[i].y;
          keep(i, P, P * ((dp[rt][i] - stv[i].z) - stv[i].w));
        }
      } else {
        const int4 vis = *reinterpret_cast<const int4*>(&sm.vis[b][16 * rt + 4 * q4]);
        const int vv[4] = {vis.x, vis.y, vis.z, vis.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const bool ok = key < vv[i];
          const float P = ok ? __builtin_amdgcn_exp2f(s[rt][i] * scale2 - stv[i].x) * stv[i].y : 0.f;
          keep(i, P, ok ? P * ((dp[rt][i] - stv[i].z) - stv[i].w) : 0.f);
        }
      }
    };
    if constexpr (LAG) {
      // the previous tile's dQ products and this tile's P / dS arithmetic in one block
      f32x4 lacc[NQ];
      auto lagged = [&](auto full_tag) __attribute__((always_inline)) {
        MSA_DQ_PRODUCTS(b ^ 1, lacc)
        pds_rows(0, full_tag);
        pds_rows(1, full_tag);
      };
      if (full)
        lagged(std::true_type{});
      else
        lagged(std::false_type{});
      if (t > 0) dq_store(myrec_prev, lacc);
      myrec_prev = myrec;
    } else {
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        if (full)
          pds_rows(rt, std::true_type{});
        else
          pds_rows(rt, std::false_type{});
      }
    }
    if constexpr (DT == kF16) {
#pragma unroll
      for (int j = 0; j < 8; ++j) split3_bits(Dv[j], dh[j], dm[j], dl[j]);
    }
    bf16x8 ap[3], ad[3];  // [hi, mid, lo]
    {
      uint32_t w[3][4];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        w[0][jj] = pack_hi16(dh[2 * jj], dh[2 * jj + 1]);
        w[1][jj] = pack_hi16(dm[2 * jj], dm[2 * jj + 1]);
        w[2][jj] = pack_hi16(dl[2 * jj], dl[2 * jj + 1]);
      }
#pragma unroll
      for (int p3 = 0; p3 < 3; ++p3) {
        ad[p3] = __builtin_bit_cast(bf16x8, make_uint4(w[p3][0], w[p3][1], w[p3][2], w[p3][3]));
        // plane rows: key 16 w + c, columns (tile rows) 4 q4 .. +3 and 16 + 4 q4 .. +3
        if constexpr (DO_Q) {
          *reinterpret_cast<uint2*>(sm.ds[b][p3] + plane_offset(key, q4)) = make_uint2(w[p3][0], w[p3][1]);
          *reinterpret_cast<uint2*>(sm.ds[b][p3] + plane_offset(key, 4 + q4)) = make_uint2(w[p3][2], w[p3][3]);
        }
      }
      if constexpr (!DO_KV) {
      } else if constexpr (DT == kF16) {
        // P: fp16 terms of 2^15 P
        uint32_t wp[3][4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
          split3_pk_f16(Pv[2 * jj] * kPScaleF16, Pv[2 * jj + 1] * kPScaleF16, wp[0][jj], wp[1][jj], wp[2][jj]);
        // dS: the key's running maximum over this tile's 32 rows (the four lanes of key c)
        float mx = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) mx = fmaxf(mx, fabsf(Dv[j]));
        kmax = fmaxf(kmax, quad_max(mx));
        const int ks_new = 15 - __builtin_amdgcn_frexp_expf(kmax);  // kmax < 2^(15 - ks_new)
        const int dlt = ks_new - ks;  // < 0, or any value while the key's accumulators are all zero
        ks = ks_new;
        if (__ballot(dlt != 0) != 0) {  // wave-uniform
          // accumulator entry i of this lane is key 4 q4 + i: lane 4 q4 + i (c = 4 q4 + i) holds its shift
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int di = __shfl(dlt, 4 * q4 + i, kWave);
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) dk[dt][i] = __builtin_amdgcn_ldexpf(dk[dt][i], di);
          }
        }
        uint32_t wd[3][4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
          split3_pk_f16(__builtin_amdgcn_ldexpf(Dv[2 * jj], ks), __builtin_amdgcn_ldexpf(Dv[2 * jj + 1], ks), wd[0][jj],
                        wd[1][jj], wd[2][jj]);
#pragma unroll
        for (int p3 = 0; p3 < 3; ++p3) {
          ap[p3] = __builtin_bit_cast(bf16x8, make_uint4(wp[p3][0], wp[p3][1], wp[p3][2], wp[p3][3]));
          ad[p3] = __builtin_bit_cast(bf16x8, make_uint4(wd[p3][0], wd[p3][1], wd[p3][2], wd[p3][3]));
        }
      } else {
        ap[0] = __builtin_bit_cast(bf16x8, make_uint4(pack_hi16(ph[0], ph[1]), pack_hi16(ph[2], ph[3]),
                                                      pack_hi16(ph[4], ph[5]), pack_hi16(ph[6], ph[7])));
        ap[1] = __builtin_bit_cast(bf16x8, make_uint4(pack_hi16(pm[0], pm[1]), pack_hi16(pm[2], pm[3]),
                                                      pack_hi16(pm[4], pm[5]), pack_hi16(pm[6], pm[7])));
        ap[2] = __builtin_bit_cast(bf16x8, make_uint4(pack_hi16(pl[0], pl[1]), pack_hi16(pl[2], pl[3]),
                                                      pack_hi16(pl[4], pl[5]), pack_hi16(pl[6], pl[7])));
      }
    }
    // ---- dV += P^T dO, dK += dS^T Q: B = X[rows pi(q4, j)][dim 16 dt + c], read transposed
#pragma unroll
    for (int dt = 0; dt < (DO_KV ? NDT : 0); ++dt) {
      const bf16x8 gb = frag_tr(sm.gs[b], KS, 4 * q4, 16 + 4 * q4, dhalf + 16 * dt, c);
      const bf16x8 qb = frag_tr(sm.qs[b], KS, 4 * q4, 16 + 4 * q4, dhalf + 16 * dt, c);
      f32x4 x = dv[dt];
      x = mfma_t<DT>(ap[2], gb, x);
      x = mfma_t<DT>(ap[1], gb, x);
      dv[dt] = mfma_t<DT>(ap[0], gb, x);
      f32x4 y = dk[dt];
      y = mfma_t<DT>(ad[2], qb, y);
      y = mfma_t<DT>(ad[1], qb, y);
      dk[dt] = mfma_t<DT>(ad[0], qb, y);
    }
    // ---- stage the next tile, start loading the one after
    if (t + 1 < ntiles) {
      MSA_MAIN_COMMIT(32 * (t + 1), b ^ 1)
      if (t + 2 < ntiles) MSA_MAIN_ISSUE(32 * (t + 2))
    }
    __syncthreads();  // dS planes of this tile and rows of the next one complete
    // ---- dQ^T = K^T dS^T: C[dim qdim(dt2) + 4 q4 + i][row 16 rh + c]
    if (!LAG && DO_Q && dq_active) {
      f32x4 acc[NQ];
      MSA_DQ_PRODUCTS(b, acc)
      dq_store(myrec, acc);
    }
  }
  if constexpr (LAG) {  // the last tile's dQ (its planes are complete after the loop's last barrier)
    f32x4 acc[NQ];
    MSA_DQ_PRODUCTS((ntiles - 1) & 1, acc)
    dq_store(myrec_prev, acc);
  }
#undef MSA_MAIN_ISSUE
#undef MSA_MAIN_COMMIT
#undef MSA_DQ_PRODUCTS

  // ---- this item's dK / dV contribution, in accumulator-fragment order:
  // kvpart[item][0 = dK, 1 = dV][wave][dt][lane][i] holds key 16 wave + 4 q4 + i, dim 16 dt + c.
  if constexpr (!DO_KV) return;
  f32x4* base = reinterpret_cast<f32x4*>(kvpart + static_cast<int64_t>(item) * 2 * 128 * DP) + wid * (DP / 16) * 64 +
                (dhalf / 16) * 64 + lane;
  if constexpr (DT == kF16) {  // divide out the scales (powers of two: exact)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int si = __shfl(ks, 4 * q4 + i, kWave);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        dk[dt][i] = __builtin_amdgcn_ldexpf(dk[dt][i], -si);
        dv[dt][i] *= 1.f / kPScaleF16;
      }
    }
  }
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
    __builtin_nontemporal_store(dk[dt], base + dt * 64);
    __builtin_nontemporal_store(dv[dt], base + 32 * DP + dt * 64);
  }
}

// For chunk c: add each row's item partials (in item order) into the FP32 key
// accumulators acc[0 = dK, 1 = dV][key][group][dim]. Thread e owns fragment slot e
// of the partial layout (four keys, one dim). grid (rows, DP / 8). The first chunk
// stores its sums (every key of every row: no separate clearing pass), the last one
// writes the bf16 results dK = scale * acc[0], dV = acc[1] instead of acc; a single
// chunk does both and never touches acc. Per key the value is the same FP32 chain
// acc = ((s_0 + s_1) + ...) as with a cleared accumulator (0 + s_0 == s_0: the item
// sums start from +0, so s_0 is never -0).
template <int DT, int DP>
__global__ __launch_bounds__(256) void kv_bwd_accumulate(const int32_t* __restrict__ cu,
                                                         const int32_t* __restrict__ cu_blocks,
                                                         const int32_t* __restrict__ starts, int nseq, int G, int D,
                                                         int B, int64_t T, const float* __restrict__ kvpart,
                                                         float* __restrict__ acc, int first, int last, float scale,
                                                         uint16_t* __restrict__ dk, uint16_t* __restrict__ dv) {
  const int64_t row = blockIdx.x;
  const int i0 = starts[row], i1 = starts[row + 1];
  if (i0 == i1 && !first && !last) return;
  const RowGeom rg = row_geom(cu, cu_blocks, nseq, row, G, B);
  constexpr int NDT = DP / 16;
  const int e = blockIdx.y * 256 + threadIdx.x;  // fragment slot: (wave, dt, lane)
  const int w = e / (NDT * 64), dt = (e / 64) % NDT, ln = e % 64;
  const int kl0 = 16 * w + 4 * (ln >> 4), d = 16 * dt + (ln & 15);
  if (kl0 >= rg.nk || d >= D) return;
  f32x4 sk = {0.f, 0.f, 0.f, 0.f}, sv = {0.f, 0.f, 0.f, 0.f};
  for (int i = i0; i < i1; ++i) {
    const f32x4* p = reinterpret_cast<const f32x4*>(kvpart + static_cast<int64_t>(i) * 2 * 128 * DP) + e;
    sk += __builtin_nontemporal_load(p);
    sv += __builtin_nontemporal_load(p + 32 * DP);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (kl0 + i < rg.nk) {
      const int64_t off = ((rg.kb + kl0 + i) * G + rg.g) * D + d;
      float xk = sk[i], xv = sv[i];
      if (!first) {
        xk = acc[off] + xk;
        xv = acc[T * G * D + off] + xv;
      }
      if (last) {
        if (dk) store_from_f32<DT>(dk, off, xk * scale);
        if (dv) store_from_f32<DT>(dv, off, xv);
      } else {
        acc[off] = xk;
        acc[T * G * D + off] = xv;
      }
    }
  }
}

// dQ = scale * sum of the row's block partials over its valid slots (FP64, slot
// order); 32 lanes per row. Slots are taken 8 at a time with all of their
// partial loads issued first (every slot's record is in bounds; invalid slots
// are masked, never added).
// (token, head) rows per dQ-combine workgroup, one 32-lane segment each (measured at c4:
// 16 rows 1.47 ms, 8 rows 1.49, 4 rows 1.49, 32 rows 1.49).
constexpr int kDqCombineRows = 16;
template <int DT, int DC>
__global__ __launch_bounds__(32 * kDqCombineRows) void kv_bwd_dq_combine(const int32_t* __restrict__ indices,
                                                         const int32_t* __restrict__ cu, int nseq, int64_t t0,
                                                         int64_t t1, int Hq, int G, int D, int K, int B, double scale,
                                                         const float* __restrict__ dqpart,
                                                         uint16_t* __restrict__ dq) {
  constexpr int kBatch = 8;
  const int sub = threadIdx.x & 31;
  const int64_t th = t0 * Hq + static_cast<int64_t>(blockIdx.x) * kDqCombineRows + (threadIdx.x >> 5);
  if (th >= t1 * Hq) return;
  const int64_t t = th / Hq;
  const int h = static_cast<int>(th % Hq);
  const int g = h / (Hq / G);
  const int s = find_seq(cu, nseq, t);
  const int64_t qb = (t - cu[s]) / B;
  const int32_t* sel = indices + (t * G + g) * K;
  const int64_t rec0 = ((t - t0) * Hq + h) * static_cast<int64_t>(K);
#pragma unroll
  for (int hc = 0; hc < DC; ++hc) {  // 128-dim halves of the row (4 dims per lane in each)
  const int dc = 128 * hc + 4 * sub;
  if (dc >= D) return;
  double a0 = 0.0, a1 = 0.0, a2 = 0.0, a3 = 0.0;
  for (int s0 = 0; s0 < K; s0 += kBatch) {
    float4 x[kBatch];
    bool ok[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int slot = s0 + u < K ? s0 + u : K - 1;
      const int id = sel[slot];
      ok[u] = s0 + u < K && id >= 0 && id <= qb;
      const f32x4 y = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(dqpart + (rec0 + slot) * D + dc));
      x[u] = make_float4(y[0], y[1], y[2], y[3]);
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      if (ok[u]) {
        a0 += static_cast<double>(x[u].x);
        a1 += static_cast<double>(x[u].y);
        a2 += static_cast<double>(x[u].z);
        a3 += static_cast<double>(x[u].w);
      }
    }
  }
  *reinterpret_cast<uint2*>(dq + th * D + dc) = pack4_from_f64<DT>(a0 * scale, a1 * scale, a2 * scale, a3 * scale);
  }
}

static int nk_of_dim(int D) { return D <= 32 ? 1 : (D <= 64 ? 2 : (D <= 128 ? 4 : 8)); }

struct BwdLayout {
  KvPlan stat_plan, main_plan;
  int64_t stat_base, main_base, spart, dqpart, kvpart, acc, rowf, total;
};

static BwdLayout bwd_layout(int64_t T, int64_t Hq, int64_t G, int64_t D, int64_t K, int64_t total_blocks) {
  BwdLayout b;
  const int64_t rows = total_blocks * G;
  const int64_t R = Hq / (G > 0 ? G : 1);
  const int64_t DP = 32 * nk_of_dim(static_cast<int>(D));
  const int64_t tc = kv_chunk_tokens(T, Hq, K, D * 4 + 8, kv_chunk_budget(kPassBwd, int64_t(3) << 30));
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
  b.rowf = b.acc + align256(2 * T * G * D * 4);
  b.total = b.rowf + align256(T * Hq * 16);
  return b;
}

int64_t attn_bwd_kv_workspace_bytes(int64_t T, int64_t Hq, int64_t G, int64_t D, int64_t K, int64_t total_blocks) {
  return bwd_layout(T, Hq, G, D, K, total_blocks).total;
}

int attn_bwd_kv(int dt, const void* q, const void* k, const void* v, const void* out, const void* dout, double* rs,
                const int32_t* indices, const int32_t* cu, int nseq, int64_t T, int Hq, int G, int D, int K, int B,
                float scale, const int32_t* cu_blocks, int64_t total_blocks, const int32_t* row_ptr,
                const int32_t* qidx, const int32_t* sidx, void* dq, void* dk, void* dv, void* ws, int64_t ws_bytes,
                const float* o32, hipStream_t st) {
  if (dt != kBF16 && dt != kF16) return kErrInvalidArgument;
  const bool f16 = dt == kF16;
  const int64_t rows = total_blocks * G;
  const BwdLayout L = bwd_layout(T, Hq, G, D, K, total_blocks);
  if (ws_bytes < L.total) return kErrInvalidArgument;
  // dQ partial element offsets (record * D + dim) are 32-bit
  if (!kv_csr_fits(T, G, K, rows) || !kv_chunk_records_fit(L.main_plan.tc, Hq, K * D)) return kErrUnsupported;
  if (T == 0) return kOk;
  char* base = static_cast<char*>(ws);
  void* sbase = base + L.stat_base;
  void* mbase = base + L.main_base;
  float2* spart = reinterpret_cast<float2*>(base + L.spart);
  float* dqpart = reinterpret_cast<float*>(base + L.dqpart);
  float* kvpart = reinterpret_cast<float*>(base + L.kvpart);
  float* acc = reinterpret_cast<float*>(base + L.acc);
  float4* rowf = reinterpret_cast<float4*>(base + L.rowf);
  const auto* qb = static_cast<const uint16_t*>(q);
  const auto* kb = static_cast<const uint16_t*>(k);
  const auto* vb = static_cast<const uint16_t*>(v);
  const auto* ob = static_cast<const uint16_t*>(out);
  const auto* gb = static_cast<const uint16_t*>(dout);
  const float scale2 = scale * kLog2e;
  const int nk = nk_of_dim(D);
  const bool fd = D == 32 * nk;
  const bool need_kv = dk != nullptr || dv != nullptr;

  // With the forward's FP32 output, flat rows take delta = O . dO and the forward's
  // mass, and only the rows it marked peaked take the statistics pass; without it,
  // every row does.
  const int all_rows = o32 == nullptr;
  const uint32_t rmagic = ratio_magic(Hq / G);  // rows x ratio < 512 * 512^2 < 2^32
  const int ratio = Hq / G;
  const int rshift = (ratio & (ratio - 1)) == 0 ? __builtin_ctz(ratio) : -1;  // power-of-two ratios shift
  {
    ProfScope ps(kProfBwdCenter, st);
    const dim3 cgrid(grid_1d(T * Hq, 8 * kCenterRows));
    if (f16)
      hipLaunchKernelGGL((kv_bwd_center<kF16, kCenterRows>), cgrid, dim3(256), 0, st, ob, o32, gb, T * Hq, D, rs);
    else
      hipLaunchKernelGGL((kv_bwd_center<kBF16, kCenterRows>), cgrid, dim3(256), 0, st, ob, o32, gb, T * Hq, D, rs);
  }
  {
    ProfScope ps(kProfBwdPlan, st);
    kv_plan_launch(L.stat_plan, row_ptr, qidx, T, sbase, st, false);  // row order measured faster here
    kv_plan_launch(L.main_plan, row_ptr, qidx, T, mbase, st);
  }
  const KvPlan& sp = L.stat_plan;
  const KvPlan& mp = L.main_plan;
  for (int64_t c = 0; c < sp.nch; ++c) {
    const int64_t t0 = c * sp.tc, t1 = t0 + sp.tc < T ? t0 + sp.tc : T;
    const int it0 = static_cast<int>(t0);
    if (rows > 0) {
      ProfScope ps(kProfBwdStats, st);
      const int32_t* hi = kv_plan_hi(sp, sbase, c);
      const int32_t* nit = kv_plan_count(sp, sbase, c);
      const int2* its = kv_plan_items(sp, sbase, c);
      const int32_t* ord = nullptr;
      const int sepi = static_cast<int>(sp.epi);
      const dim3 grid(static_cast<unsigned>(sp.max_items)), block(kStatThreads);
#define MSA_BWD_STATS(DTV, NKV, FD) hipLaunchKernelGGL((kv_bwd_stats_kernel<DTV, NKV, FD>), grid, block, 0, st, qb, kb, vb, gb, rs, cu, cu_blocks, qidx, sidx, hi, nit, its, ord, nseq, Hq, G, D, K, B, scale2, sepi, it0, all_rows, spart)
#define MSA_BWD_STATS_NK(DTV)                                                                  \
  if (nk == 1) { if (fd) MSA_BWD_STATS(DTV, 1, true); else MSA_BWD_STATS(DTV, 1, false); }       \
  else if (nk == 2) { if (fd) MSA_BWD_STATS(DTV, 2, true); else MSA_BWD_STATS(DTV, 2, false); }  \
  else if (nk == 4) { if (fd) MSA_BWD_STATS(DTV, 4, true); else MSA_BWD_STATS(DTV, 4, false); }  \
  else { if (fd) MSA_BWD_STATS(DTV, 8, true); else MSA_BWD_STATS(DTV, 8, false); }
      if (f16) { MSA_BWD_STATS_NK(kF16) } else { MSA_BWD_STATS_NK(kBF16) }
#undef MSA_BWD_STATS_NK
#undef MSA_BWD_STATS
    }
    {
      ProfScope ps(kProfBwdStatsCombine, st);
      const int rps = all_rows ? 1 : 32;  // rows per 32-lane segment
      hipLaunchKernelGGL(kv_bwd_stats_combine, dim3(grid_1d((t1 - t0) * Hq, 8 * rps)), dim3(256), 0, st, indices, cu,
                         nseq, t0, t1, Hq, G, K, B, all_rows, rps, spart, rs, rowf);
    }
    if (rows > 0) {
      const int32_t* hi = kv_plan_hi(mp, mbase, c);
      const int32_t* nit = kv_plan_count(mp, mbase, c);
      const int2* its = kv_plan_items(mp, mbase, c);
      const int32_t* ord = kv_plan_order(mp, mbase, c);
      const int mepi = static_cast<int>(mp.epi);
      const dim3 grid(static_cast<unsigned>(mp.max_items)), block(kMainThreads);
      {
        ProfScope ps(kProfBwdMain, st);
#define MSA_BWD_MAIN(DTV, NKV, FD, PT, DH) hipLaunchKernelGGL((kv_bwd_main_kernel<DTV, NKV, FD, PT>), grid, block, 0, st, qb, kb, vb, gb, rs, cu, cu_blocks, qidx, sidx, hi, nit, its, ord, nseq, Hq, G, D, K, B, scale2, mepi, it0, rmagic, rshift, rowf, dqpart, kvpart, DH)
#define MSA_BWD_MAIN_NK(DTV)                                                                                     \
  if (nk == 1) { if (fd) MSA_BWD_MAIN(DTV, 1, true, kPartAll, 0); else MSA_BWD_MAIN(DTV, 1, false, kPartAll, 0); }       \
  else if (nk == 2) { if (fd) MSA_BWD_MAIN(DTV, 2, true, kPartAll, 0); else MSA_BWD_MAIN(DTV, 2, false, kPartAll, 0); }  \
  else if (nk == 4) { if (fd) MSA_BWD_MAIN(DTV, 4, true, kPartAll, 0); else MSA_BWD_MAIN(DTV, 4, false, kPartAll, 0); }  \
  else for (int dh = 0; dh < 256; dh += 128) {                                                                   \
    if (need_kv) { if (fd) MSA_BWD_MAIN(DTV, 8, true, kPartKV, dh); else MSA_BWD_MAIN(DTV, 8, false, kPartKV, dh); }   \
    /* bf16: one dQ launch covers both halves */                                                               \
    if (dq && (DTV == kF16 || dh == 0)) {                                                                      \
      if (fd) MSA_BWD_MAIN(DTV, 8, true, kPartQ, dh); else MSA_BWD_MAIN(DTV, 8, false, kPartQ, dh);             \
    }                                                                                                          \
  }
        if (f16) { MSA_BWD_MAIN_NK(kF16) } else { MSA_BWD_MAIN_NK(kBF16) }
#undef MSA_BWD_MAIN_NK
#undef MSA_BWD_MAIN
      }
      if (need_kv) {
        ProfScope ps(kProfBwdAccumulate, st);
        const int32_t* starts = kv_plan_starts(mp, mbase, c);
        const dim3 agrid(static_cast<unsigned>(rows), static_cast<unsigned>(32 * nk / 8));
        const int first = c == 0, last = c + 1 == sp.nch;
        auto* dkb = static_cast<uint16_t*>(dk);
        auto* dvb = static_cast<uint16_t*>(dv);
#define MSA_BWD_ACC(DTV, DPV) hipLaunchKernelGGL((kv_bwd_accumulate<DTV, DPV>), agrid, dim3(256), 0, st, cu, cu_blocks, starts, nseq, G, D, B, T, kvpart, acc, first, last, scale, dkb, dvb)
#define MSA_BWD_ACC_NK(DTV)                                                                           \
  if (nk == 1) MSA_BWD_ACC(DTV, 32); else if (nk == 2) MSA_BWD_ACC(DTV, 64); else if (nk == 4) MSA_BWD_ACC(DTV, 128); \
  else MSA_BWD_ACC(DTV, 256);
        if (f16) { MSA_BWD_ACC_NK(kF16) } else { MSA_BWD_ACC_NK(kBF16) }
#undef MSA_BWD_ACC_NK
#undef MSA_BWD_ACC
      }
    }
    if (dq) {
      ProfScope ps(kProfBwdDqCombine, st);
      const dim3 qgrid(grid_1d((t1 - t0) * Hq, kDqCombineRows)), qblock(32 * kDqCombineRows);
#define MSA_DQ_COMBINE(DTV, DCV)                                                                              \
  hipLaunchKernelGGL((kv_bwd_dq_combine<DTV, DCV>), qgrid, qblock, 0, st, indices, cu, nseq, t0, t1, Hq, G, D, K, B, \
                     static_cast<double>(scale), dqpart, static_cast<uint16_t*>(dq))
      if (f16) { if (D > 128) MSA_DQ_COMBINE(kF16, 2); else MSA_DQ_COMBINE(kF16, 1); }
      else { if (D > 128) MSA_DQ_COMBINE(kBF16, 2); else MSA_DQ_COMBINE(kBF16, 1); }
#undef MSA_DQ_COMBINE
    }
  }
  return status_from(hipGetLastError());
}

}  // namespace msa
