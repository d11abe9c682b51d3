// Indexer KL: the training branch that consumes the selection (bf16, gfx950 MFMA).
//
// Over the causal tokens of each (token t, group g)'s selected blocks:
//   student S_j = softmax_j(z), z_j = sigma_i * iq[t,g] . ik[j]      (index token logits)
//   teacher T_j = mean over the group's R heads of softmax_j(a_h),   a_hj = sigma_a * q[t,h] . k[j,g]
//   KL_tg = sum_j T_j (log T_j - log S_j),   loss = sum_tg KL_tg / (T * G)
// and, for index_q / index_k only, dLoss/dz_j = (S_j - T_j) / (T * G).
// The reference describes this branch (docs/msa_training_flow.md:92-138) but has no
// kernel for it (docs/implementation_plan.md:66-69).
//
// Both passes are KV-major over the k2q CSR like the attention kernels (one work
// item = a key block row and <= 512 of its edges):
//   pass 1 (kl_stats_kernel): per (edge, head) and per edge, the block's (max, sum)
//     of 2^x for the teacher and the student logits; merged per row in slot order
//     (kl_stats_combine) into base-2 log-normalisers.
//   pass 2 (kl_main_kernel): T, S, the KL terms and dz = S - T per (edge, key); the
//     per-(edge) KL and d_iq partials (merged per row in slot order, kl_row_combine)
//     and per-item d_ik partials (summed per key block in group and item order,
//     kl_accumulate). No floating-point atomics: results are deterministic.
#include <type_traits>

#include "attn_kv_common.hpp"
#include "msa_mi355x.h"

// Each logit and exponent argument is rounded as written (no fused multiply-adds):
// the statistics and main passes then form them identically, and the unmasked and
// masked code paths of a tile give the same bits.
#pragma clang fp contract(off)

namespace msa {

namespace {

constexpr int kKlThreads = 512;  // 8 waves
constexpr int kKlEdges = 512;    // edges per work item (both passes)
constexpr int kKlMaxRatio = 8;   // query heads per group staged by pass 2

template <int DP>
constexpr int kl_stride() { return DP + 16; }

typedef short v4i16 __attribute__((ext_vector_type(4)));

typedef _Float16 v4f16 __attribute__((ext_vector_type(4)));

// 16x16x16 MFMA of the input type (bf16 or fp16 operand words in v4i16 containers).
template <int DT>
__device__ __forceinline__ f32x4 mfma16(v4i16 a, v4i16 b, f32x4 c) {
  if constexpr (DT == kF16)
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(v4f16, a), __builtin_bit_cast(v4f16, b), c, 0,
                                                 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

template <int NK, int NKI>
struct KlStatSmem {
  static constexpr int KS = kl_stride<32 * NK>(), KSI = kl_stride<32 * NKI>();
  alignas(16) uint16_t k[128 * KS];    // K block [key][dim]
  alignas(16) uint16_t ik[128 * KSI];  // index_k block [key][dim]
  int32_t tok[kKlEdges];
  int32_t slot[kKlEdges];
};

// Base-2 (max, sum 2^(x - max)) over the 32 keys a lane holds (masked keys are -inf),
// reduced over the four lanes of the row.
__device__ __forceinline__ float2 lane_max_sum(float (&x)[8][4]) {
  float m = -__builtin_inff();
#pragma unroll
  for (int kt = 0; kt < 8; ++kt)
#pragma unroll
    for (int i = 0; i < 4; ++i) m = fmaxf(m, x[kt][i]);
  m = quad_max(m);
  const float base = m == -__builtin_inff() ? 0.f : m;
  float l = 0.f;
#pragma unroll
  for (int kt = 0; kt < 8; ++kt)
#pragma unroll
    for (int i = 0; i < 4; ++i) l += __builtin_amdgcn_exp2f(x[kt][i] - base);
  l += __shfl_xor(l, 16, kWave);
  l += __shfl_xor(l, 32, kWave);
  return make_float2(m, l);
}

}  // namespace

// Pass 1: waves own 16 edges each per tile (lane c = edge), all 128 keys of the
// block. Logits^T = K_block . rows^T (A = block rows from LDS, B = the edge's query
// row from memory): lane (c, q4) holds keys 16 kt + 4 q4 + i of edge c.
template <int DT, int NK, int NKI>
__global__ __launch_bounds__(kKlThreads, 2) void kl_stats_kernel(
    const uint16_t* __restrict__ iq, const uint16_t* __restrict__ ik, const uint16_t* __restrict__ q,
    const uint16_t* __restrict__ k, const int32_t* __restrict__ cu, const int32_t* __restrict__ cu_blocks,
    const int32_t* __restrict__ qidx, const int32_t* __restrict__ sidx, const int32_t* __restrict__ e_hi,
    const int32_t* __restrict__ n_items, const int2* __restrict__ items, const int32_t* __restrict__ order, int nseq, int Hq, int G, int K, int B,
    float zs2, float as2, int epi, int t0, int teacher, float2* __restrict__ tpart, float2* __restrict__ spart) {
  constexpr int D = 32 * NK, Di = 32 * NKI;
  constexpr int KS = KlStatSmem<NK, NKI>::KS, KSI = KlStatSmem<NK, NKI>::KSI;
  __shared__ KlStatSmem<NK, NKI> sm;
  if (static_cast<int>(blockIdx.x) >= *n_items) return;
  const int item = order[blockIdx.x];  // largest items first
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63, c = lane & 15, q4 = lane >> 4;
  const int2 it = items[item];
  const int row = it.x, e_begin = it.y;
  const RowGeom rg = row_geom(cu, cu_blocks, nseq, row, G, B);
  const int R = Hq / G;
  const int e_end = e_begin + epi < e_hi[row] ? e_begin + epi : e_hi[row];
  const int ne = e_end - e_begin;

  for (int e = tid; e < 128 * (D / 8); e += kKlThreads) {
    const int kl = e / (D / 8), d0 = 8 * (e % (D / 8));
    uint4 w = make_uint4(0u, 0u, 0u, 0u);
    if (kl < rg.nk) w = *reinterpret_cast<const uint4*>(k + ((rg.kb + kl) * G + rg.g) * D + d0);
    *reinterpret_cast<uint4*>(sm.k + kl * KS + d0) = w;
  }
  for (int e = tid; e < 128 * (Di / 8); e += kKlThreads) {
    const int kl = e / (Di / 8), d0 = 8 * (e % (Di / 8));
    uint4 w = make_uint4(0u, 0u, 0u, 0u);
    if (kl < rg.nk) w = *reinterpret_cast<const uint4*>(ik + (rg.kb + kl) * Di + d0);
    *reinterpret_cast<uint4*>(sm.ik + kl * KSI + d0) = w;
  }
  for (int e = tid; e < ne; e += kKlThreads) {
    sm.tok[e] = qidx[e_begin + e];
    sm.slot[e] = sidx[e_begin + e];
  }
  __syncthreads();

  const int ntiles = (ne + 127) / 128;
  for (int tile = 0; tile < ntiles; ++tile) {
    const int ebase = tile * 128 + 16 * wid;
    if (ebase >= ne) break;  // wave-uniform
    const int e = ebase + c;
    const bool ok = e < ne;
    const int tok = sm.tok[ok ? e : ebase];
    const int slot = ok ? sm.slot[e] : 0;
    const int64_t vk = static_cast<int64_t>(tok) - rg.kb + 1;
    const int lim = ok ? (vk < rg.nk ? static_cast<int>(vk) : rg.nk) : 0;
    // Wave-uniform: every edge of the wave sees all 128 keys (no masks), or not; the two
    // cases are separate code paths so the unmasked one carries no per-logit selects.
    const bool full = __ballot(lim < 128) == 0;
    auto body = [&](auto full_tag) __attribute__((always_inline)) {
    constexpr bool FULL = decltype(full_tag)::value;
    float x[8][4];
    // ---- student: z^T = ik_block . iq^T
    {
      bf16x8 bq[NKI];
#pragma unroll
      for (int kk = 0; kk < NKI; ++kk)
        bq[kk] = load_frag(iq + (static_cast<int64_t>(tok) * G + rg.g) * Di + 32 * kk + 8 * q4);
#pragma unroll
      for (int kt = 0; kt < 8; ++kt) {
        f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < NKI; ++kk) a = mfma_t<DT>(load_frag(sm.ik + (16 * kt + c) * KSI + 32 * kk + 8 * q4), bq[kk], a);
#pragma unroll
        for (int i = 0; i < 4; ++i) x[kt][i] = FULL || 16 * kt + 4 * q4 + i < lim ? a[i] * zs2 : -__builtin_inff();
      }
      const float2 ml = lane_max_sum(x);
      if (q4 == 0 && ok) spart[((static_cast<int64_t>(tok) - t0) * G + rg.g) * K + slot] = ml;
    }
    // ---- teacher, head by head: a^T = K_block . q_h^T (skipped when the caller supplies
    // the attention's lse, which is the teacher's normaliser)
    for (int h = 0; h < (teacher ? R : 0); ++h) {
      const int hq = rg.g * R + h;
      bf16x8 bq[NK];
#pragma unroll
      for (int kk = 0; kk < NK; ++kk)
        bq[kk] = load_frag(q + (static_cast<int64_t>(tok) * Hq + hq) * D + 32 * kk + 8 * q4);
#pragma unroll
      for (int kt = 0; kt < 8; ++kt) {
        f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < NK; ++kk) a = mfma_t<DT>(load_frag(sm.k + (16 * kt + c) * KS + 32 * kk + 8 * q4), bq[kk], a);
#pragma unroll
        for (int i = 0; i < 4; ++i) x[kt][i] = FULL || 16 * kt + 4 * q4 + i < lim ? a[i] * as2 : -__builtin_inff();
      }
      const float2 ml = lane_max_sum(x);
      if (q4 == 0 && ok) tpart[((static_cast<int64_t>(tok) - t0) * Hq + hq) * K + slot] = ml;
    }
    };
    if (full)
      body(std::true_type{});
    else
      body(std::false_type{});
  }
}

// Per row of the chunk (Hq teacher rows, then G student rows per token): merge the
// valid slots' (max, sum) in FP64 into lse2 = log2 sum_j 2^x_j, kept as
// (float(lse2), 2^(float(lse2) - lse2), float(lse2) - lse2): with them
// 2^(x - float(lse2)) * the second value is the normalised probability, and
// log2 p = (x - float(lse2)) + the third. 16 lanes per row (slots lane-parallel).
// With tlse (the attention's natural-log lse [T, Hq] for the same q, k, selection and
// scale), a teacher row takes (float(lse * log2 e), 1, 0) instead.
__global__ __launch_bounds__(256) void kl_stats_combine(const int32_t* __restrict__ indices,
                                                        const int32_t* __restrict__ cu, int nseq, int64_t t0,
                                                        int64_t t1, int Hq, int G, int K, int B,
                                                        const float2* __restrict__ tpart,
                                                        const float2* __restrict__ spart, const float* __restrict__ tlse,
                                                        float4* __restrict__ tstate, float4* __restrict__ sstate) {
  const int sub = threadIdx.x & 15;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 16 + (threadIdx.x >> 4);
  if (r >= (t1 - t0) * (Hq + G)) return;  // whole 16-lane segments exit together
  const int64_t tl = r / (Hq + G);
  const int j = static_cast<int>(r % (Hq + G));
  const int64_t t = t0 + tl;
  const bool student = j >= Hq;
  const int g = student ? j - Hq : j / (Hq / G);
  if (!student && tlse) {
    if (sub == 0) {
      const float l = tlse[t * Hq + j];
      tstate[t * Hq + j] = l == -__builtin_inff() ? make_float4(0.f, 0.f, 0.f, 0.f)
                                                  : make_float4(static_cast<float>(static_cast<double>(l) * 1.4426950408889634),
                                                                1.f, 0.f, 0.f);
    }
    return;
  }
  const float2* part = student ? spart + (tl * G + g) * K : tpart + (tl * Hq + j) * K;
  const int s = find_seq(cu, nseq, t);
  const int64_t qb = (t - cu[s]) / B;
  const int32_t* sel = indices + (t * G + g) * K;
  float M = -__builtin_inff();
  for (int slot = sub; slot < K; slot += 16) {
    const int id = sel[slot];
    if (id >= 0 && id <= qb) M = fmaxf(M, part[slot].x);
  }
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 16));
  double L = 0.0;
  if (M != -__builtin_inff()) {
    for (int slot = sub; slot < K; slot += 16) {
      const int id = sel[slot];
      if (id >= 0 && id <= qb) {
        const float2 ml = part[slot];
        L = fma(exp2(static_cast<double>(ml.x) - static_cast<double>(M)), static_cast<double>(ml.y), L);
      }
    }
  }
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) L += __shfl_xor(L, o, 16);
  if (sub == 0) {
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (L > 0.0) {
      const double lse2 = static_cast<double>(M) + log2(L);
      const float lf = static_cast<float>(lse2);
      const double res = static_cast<double>(lf) - lse2;
      v = make_float4(lf, static_cast<float>(exp2(res)), static_cast<float>(res), 0.f);
    }
    if (student)
      sstate[t * G + g] = v;
    else
      tstate[t * Hq + j] = v;
  }
}

namespace {

// dz planes [key][edge] are unpadded (32 bytes per key, so a row's 8 banks are set by its
// row index mod 8). Key k sits in row k ^ (4 ((k >> 3) & 1)) and its 8-byte piece p (edges
// 4p .. 4p + 3) at piece p ^ ((k >> 2) & 3). The transposed reads of 32 lanes take keys
// k0 .. k0 + 3 and k0 + 8 .. k0 + 11 (k0 a multiple of 8, or those plus 4), all four pieces:
// the row permutation puts the two key groups on different halves of the 64 banks, so the
// 32 reads of 8 bytes hit 64 distinct banks; the plane writes of 32 lanes (keys k0 .. k0 +
// 15, pieces 0 and 1) pair rows r and r ^ 12, whose piece swizzles differ in bit 1, so they
// are conflict-free too. SQ_LDS_BANK_CONFLICT over kl_main_kernel at c4: 0.47 conflict
// cycles per LDS instruction (the piece swizzle alone 0.82, unswizzled 1.08; the rest come
// from its other LDS accesses); the kernel's time is unchanged within run-to-run noise.
__device__ __forceinline__ int dz_offset(int key, int piece) {
  return (key ^ (((key >> 3) & 1) << 2)) * 16 + 4 * (piece ^ ((key >> 2) & 3));
}

template <int NK, int NKI>
struct KlMainSmem {
  static constexpr int KS = kl_stride<32 * NK>(), KSI = kl_stride<32 * NKI>();
  alignas(16) uint16_t qs[2][16 * kKlMaxRatio * KS];  // q rows of a tile [head * 16 + edge][dim]
  alignas(16) uint16_t iqs[2][16 * KSI];              // index_q rows of a tile [edge][dim]
  alignas(16) uint16_t ikb[128 * KSI];                // the index_k block [key][dim]
  alignas(16) uint16_t dz[2][3][128 * 16];            // dz split planes (hi, mid, lo) [key][edge]
  alignas(16) float2 tst[2][16 * kKlMaxRatio];        // teacher (lse2, 1 / mass) per tile row
  alignas(16) float4 sst[2][16];                      // student normalisers per tile edge
  alignas(16) int32_t vis[2][16];                     // visible keys per tile edge (0 past the end)
  alignas(16) int32_t rec[2][16];                     // (token, group, slot) record per tile edge (-1 past the end)
  float red[2][8][16];                                // per-wave KL sums per tile edge
  int32_t etok[kKlEdges];
  int32_t eslot[kKlEdges];
};

}  // namespace

// Pass 2: one workgroup per work item, 8 waves x 16 keys (wave w owns keys 16 w ..
// 16 w + 15 of the block), tiles of 16 edges. Per tile:
//   teacher  a_h = q_h K^T per head: C[edge 4 q4 + i][key c] (A: q rows from LDS,
//            B: the wave's K fragments in registers); T = mean_h 2^(x - lse2_h)
//   student  z = iq ik^T, S = 2^(x - lse2); KL terms T (log2 T - log2 S) summed
//            over the wave's keys, then over the 8 waves in order
//   dz = S - T split into three bf16 terms:
//     d_ik += dz^T iq   (16x16x16 MFMAs: A = dz straight from the C registers,
//                        B = iq rows read transposed)
//     dz planes -> LDS [key][edge]; barrier
//     d_iq^T = ik^T dz^T  wave w: dims 16 w .. 16 w + 15, all 16 edges, all 128 keys
// Row tiles, planes and the KL scratch are double-buffered: one barrier per tile.
template <int DT, int NK, int NKI>
__global__ __launch_bounds__(kKlThreads, 1) void kl_main_kernel(
    const uint16_t* __restrict__ iq, const uint16_t* __restrict__ ik, const uint16_t* __restrict__ q,
    const uint16_t* __restrict__ k, const float4* __restrict__ tstate, const float4* __restrict__ sstate,
    const int32_t* __restrict__ cu, const int32_t* __restrict__ cu_blocks, const int32_t* __restrict__ qidx,
    const int32_t* __restrict__ sidx, const int32_t* __restrict__ e_hi, const int32_t* __restrict__ n_items,
    const int2* __restrict__ items, const int32_t* __restrict__ order, int nseq, int Hq, int G, int K, int B, float zs2, float as2, int epi, int t0,
    int need_diq, int need_dik, float* __restrict__ klpart, float* __restrict__ diqpart,
    float* __restrict__ ikpart) {
  constexpr int D = 32 * NK, Di = 32 * NKI, NDTI = Di / 16;
  constexpr int KS = KlMainSmem<NK, NKI>::KS, KSI = KlMainSmem<NK, NKI>::KSI;
  constexpr int QV = D / 8, IV = Di / 8;                               // 16-byte chunks per row
  constexpr int QI = (16 * kKlMaxRatio * QV + kKlThreads - 1) / kKlThreads;  // q chunks per staging thread
  __shared__ KlMainSmem<NK, NKI> sm;
  if (static_cast<int>(blockIdx.x) >= *n_items) return;
  const int item = order[blockIdx.x];  // largest items first
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63, c = lane & 15, q4 = lane >> 4;
  const int2 it = items[item];
  const int row = it.x, e_begin = it.y;
  const RowGeom rg = row_geom(cu, cu_blocks, nseq, row, G, B);
  const int R = Hq / G;
  const int e_end = e_begin + epi < e_hi[row] ? e_begin + epi : e_hi[row];
  const int ne = e_end - e_begin;
  if (ne <= 0) return;  // (the plan emits no empty items; whole workgroup)
  const int ntiles = (ne + 15) >> 4;
  const float inv_r = 1.f / static_cast<float>(R);

  // ---- item set-up: edges, the index_k block, this wave's K / index_k fragments
  for (int e = tid; e < ne; e += kKlThreads) {
    sm.etok[e] = qidx[e_begin + e];
    sm.eslot[e] = sidx[e_begin + e];
  }
  for (int e = tid; e < 128 * IV; e += kKlThreads) {
    const int kl = e / IV, d0 = 8 * (e % IV);
    uint4 w = make_uint4(0u, 0u, 0u, 0u);
    if (kl < rg.nk) w = *reinterpret_cast<const uint4*>(ik + (rg.kb + kl) * Di + d0);
    *reinterpret_cast<uint4*>(sm.ikb + kl * KSI + d0) = w;
  }
  const int key = 16 * wid + c;
  bf16x8 kf[NK], ikf[NKI];  // B operands: K[key][dims 32 kk + 8 q4 + j], index_k likewise
  {
    const int kc = key < rg.nk ? key : rg.nk - 1;
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) {
      const bf16x8 x = load_frag(k + ((rg.kb + kc) * G + rg.g) * D + 32 * kk + 8 * q4);
      kf[kk] = key < rg.nk ? x : zero_frag();
    }
#pragma unroll
    for (int kk = 0; kk < NKI; ++kk) {
      const bf16x8 x = load_frag(ik + (rg.kb + kc) * Di + 32 * kk + 8 * q4);
      ikf[kk] = key < rg.nk ? x : zero_frag();
    }
  }
  __syncthreads();  // edges and the index_k block visible
  const bool diq_wave = need_diq && 16 * wid < Di;
  bf16x8 ikt[4];  // A operand of d_iq^T: ik^T[dim 16 w + c][keys 32 kc + 8 q4 + j]
#pragma unroll
  for (int kc = 0; kc < 4; ++kc)
    ikt[kc] = diq_wave ? frag_tr(sm.ikb, KSI, 32 * kc + 8 * q4, 32 * kc + 8 * q4 + 4, 16 * wid, c) : zero_frag();

  // ---- row staging (16 edges per tile): q rows (edge * R + head) and index_q rows,
  // per-row normalisers, visible keys and records. Two register stages: tile j is
  // loaded into stage j % 2 two tiles ahead of its use and committed to LDS one tile
  // ahead (measured: with the rows of every tile cache-hot the KL runs 14 % faster,
  // so its row gathers are worth hiding).
  struct Stage {
    uint4 pf[QI], pfi;
    float4 pst;
    int pvis, prec;
  };
  Stage st0, st1;
  st0.pfi = st1.pfi = make_uint4(0u, 0u, 0u, 0u);
  st0.pst = st1.pst = make_float4(0.f, 0.f, 0.f, 0.f);
  st0.pvis = st1.pvis = 0;
  st0.prec = st1.prec = -1;
  // the thread -> (tile edge, head, dims) split of the q rows is the same for every tile
  int qel[QI], qsrc[QI], qdst[QI];
#pragma unroll
  for (int i = 0; i < QI; ++i) {
    const int idx = tid + kKlThreads * i;
    const int rr = idx / QV, d0 = 8 * (idx % QV);
    const int el = rr / R, h = rr - el * R;
    qel[i] = idx < 16 * R * QV ? el : -1;  // -1: no chunk for this thread
    qsrc[i] = (rg.g * R + h) * D + d0;
    qdst[i] = (h * 16 + el) * KS + d0;
  }
  const int64_t qrow = static_cast<int64_t>(Hq) * D;
  auto issue = [&](int e0, Stage& S) {
    uint4(&pf)[QI] = S.pf;
    uint4& pfi = S.pfi;
    float4& pst = S.pst;
    int &pvis = S.pvis, &prec = S.prec;
#pragma unroll
    for (int i = 0; i < QI; ++i) {
      if (qel[i] >= 0) {
        const int e = e0 + qel[i] < ne ? e0 + qel[i] : ne - 1;
        pf[i] = *reinterpret_cast<const uint4*>(q + sm.etok[e] * qrow + qsrc[i]);
      }
    }
    if (tid < 16 * IV) {
      const int el = tid / IV, d0 = 8 * (tid % IV);
      const int e = e0 + el < ne ? e0 + el : ne - 1;
      pfi = *reinterpret_cast<const uint4*>(iq + (static_cast<int64_t>(sm.etok[e]) * G + rg.g) * Di + d0);
    }
    if (tid < 16 * R) {
      const int el = tid / R, h = tid - el * R;
      const int e = e0 + el < ne ? e0 + el : ne - 1;
      pst = tstate[static_cast<int64_t>(sm.etok[e]) * Hq + rg.g * R + h];
    } else if (tid >= 256 && tid < 256 + 16) {
      const int el = tid - 256;
      const int e = e0 + el;
      if (e < ne) {
        const int tk = sm.etok[e];
        pst = sstate[static_cast<int64_t>(tk) * G + rg.g];
        const int64_t vk = static_cast<int64_t>(tk) - rg.kb + 1;
        pvis = vk < rg.nk ? static_cast<int>(vk) : rg.nk;
        prec = ((tk - t0) * G + rg.g) * K + sm.eslot[e];
      } else {
        pst = make_float4(0.f, 0.f, 0.f, 0.f);
        pvis = 0;
        prec = -1;
      }
    }
  };
  auto commit = [&](int e0, int buf, const Stage& S) {
    const uint4(&pf)[QI] = S.pf;
    const uint4& pfi = S.pfi;
    const float4& pst = S.pst;
    const int pvis = S.pvis, prec = S.prec;
#pragma unroll
    for (int i = 0; i < QI; ++i) {
      // head-major rows: the A-operand reads of one head (lane c -> edge c) hit
      // consecutive rows, conflict-free with the padded stride
      if (qel[i] >= 0)
        *reinterpret_cast<uint4*>(sm.qs[buf] + qdst[i]) = e0 + qel[i] < ne ? pf[i] : make_uint4(0u, 0u, 0u, 0u);
    }
    if (tid < 16 * IV) {
      const int el = tid / IV, d0 = 8 * (tid % IV);
      *reinterpret_cast<uint4*>(sm.iqs[buf] + el * KSI + d0) = e0 + el < ne ? pfi : make_uint4(0u, 0u, 0u, 0u);
    }
    if (tid < 16 * R) {
      sm.tst[buf][tid] = make_float2(pst.x, pst.y);
    } else if (tid >= 256 && tid < 256 + 16) {
      sm.sst[buf][tid - 256] = pst;
      sm.vis[buf][tid - 256] = pvis;
      sm.rec[buf][tid - 256] = prec;
    }
  };

  f32x4 dik[NDTI];  // C[key 16 w + 4 q4 + i][dim 16 dt + c]
#pragma unroll
  for (int dt = 0; dt < NDTI; ++dt) dik[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  issue(0, st0);
  commit(0, 0, st0);
  if (ntiles > 1) issue(16, st1);
  if (ntiles > 2) issue(32, st0);
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int b = t & 1;
    // visible keys of the lane's edges 4 q4 + i
    const int4 vis4 = *reinterpret_cast<const int4*>(&sm.vis[b][4 * q4]);
    const int vv[4] = {vis4.x, vis4.y, vis4.z, vis4.w};
    // Wave-uniform: all 16 edges of the tile see all of the wave's keys (edges are in
    // token order, so edge 0 sees the fewest), or not; separate code paths keep the
    // per-element selects out of the unmasked one.
    const bool full = 16 * t + 16 <= ne && sm.vis[b][0] >= key - c + 16;
    float dz[4], klv[4];
    auto teacher_student = [&](auto full_tag) __attribute__((always_inline)) {
    constexpr bool FULL = decltype(full_tag)::value;
    // ---- teacher: T[edge 4 q4 + i][key] = mean_h 2^(a_h * as2 - lse2_h) / mass_h
    float tsum[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int h = 0; h < kKlMaxRatio; ++h) {
      if (h < R) {  // wave-uniform; unrolled so that heads interleave
        f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < NK; ++kk) a = mfma_t<DT>(load_frag(sm.qs[b] + (h * 16 + c) * KS + 32 * kk + 8 * q4), kf[kk], a);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float2 st = sm.tst[b][(4 * q4 + i) * R + h];
          const float p = __builtin_amdgcn_exp2f(a[i] * as2 - st.x) * st.y;
          tsum[i] += FULL || key < vv[i] ? p : 0.f;
        }
      }
    }
    // ---- student, KL terms and dz
    f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < NKI; ++kk) z = mfma_t<DT>(load_frag(sm.iqs[b] + c * KSI + 32 * kk + 8 * q4), ikf[kk], z);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 st = sm.sst[b][4 * q4 + i];
      const bool vis = FULL || key < vv[i];
      const float y = z[i] * zs2 - st.x;  // log2 S - st.z
      const float S = vis ? __builtin_amdgcn_exp2f(y) * st.y : 0.f;
      const float T = vis ? tsum[i] * inv_r : 0.f;
      dz[i] = S - T;
      // base-2 logs (v_log_f32); terms below 2^-100 are dropped
      klv[i] = T > 0x1p-100f ? T * (__builtin_amdgcn_logf(T) - (y + st.z)) : 0.f;
    }
    };
    if (full)
      teacher_student(std::true_type{});
    else
      teacher_student(std::false_type{});
    // KL: sum over the wave's 16 keys (lanes c of the quad group), then over waves
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = klv[i];
      v += __shfl_xor(v, 1, 16);
      v += __shfl_xor(v, 2, 16);
      v += __shfl_xor(v, 4, 16);
      v += __shfl_xor(v, 8, 16);
      klv[i] = v;
    }
    if (c == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) sm.red[b][wid][4 * q4 + i] = klv[i];
    }
    // ---- dz split: words of edges (4 q4, 4 q4 + 1) and (4 q4 + 2, 4 q4 + 3) per term
    // (fp16: terms of 2^15 dz, |dz| <= 1; the d_ik and d_iq partials carry the factor until stored)
    uint32_t w[3][2];
    if constexpr (DT == kF16) {
      split3_pk_f16(dz[0] * kPScaleF16, dz[1] * kPScaleF16, w[0][0], w[1][0], w[2][0]);
      split3_pk_f16(dz[2] * kPScaleF16, dz[3] * kPScaleF16, w[0][1], w[1][1], w[2][1]);
    } else {
      split3_pk(dz[0], dz[1], w[0][0], w[1][0], w[2][0]);
      split3_pk(dz[2], dz[3], w[0][1], w[1][1], w[2][1]);
    }
    if (need_dik) {
      // d_ik[key][dim 16 dt + c'] += dz^T[key][edges] iq[edges][dim]: A = dz (lane c = key,
      // edges 4 q4 + j), B[edges 4 q4 + j][dim 16 dt + c] read transposed from the iq rows
      const v4i16 al = __builtin_bit_cast(v4i16, make_uint2(w[2][0], w[2][1]));
      const v4i16 am = __builtin_bit_cast(v4i16, make_uint2(w[1][0], w[1][1]));
      const v4i16 ah = __builtin_bit_cast(v4i16, make_uint2(w[0][0], w[0][1]));
#pragma unroll
      for (int dt = 0; dt < NDTI; ++dt) {
        const uint2 raw = lds_read_tr16(sm.iqs[b] + (4 * q4 + (c >> 2)) * KSI + 16 * dt + 4 * (c & 3));
        const v4i16 bq = __builtin_bit_cast(v4i16, raw);
        f32x4 x = dik[dt];
        x = mfma16<DT>(al, bq, x);
        x = mfma16<DT>(am, bq, x);
        dik[dt] = mfma16<DT>(ah, bq, x);
      }
    }
    if (need_diq) {
      // planes [key][edge]: key 16 w + c, edges 4 q4 .. 4 q4 + 3
#pragma unroll
      for (int p3 = 0; p3 < 3; ++p3)
        *reinterpret_cast<uint2*>(sm.dz[b][p3] + dz_offset(key, q4)) = make_uint2(w[p3][0], w[p3][1]);
    }
    // records read before the barrier: buffer b is refilled (tile t + 2) before the next one
    const int myrec = sm.rec[b][c];
    const int krec = tid < 16 ? sm.rec[b][tid] : -1;
    // ---- stage the next tile (from register stage (t + 1) % 2), then load tile t + 3 into that stage
    if (t + 1 < ntiles) {
      if ((t + 1) & 1) {
        commit(16 * (t + 1), b ^ 1, st1);
        if (t + 3 < ntiles) issue(16 * (t + 3), st1);
      } else {
        commit(16 * (t + 1), b ^ 1, st0);
        if (t + 3 < ntiles) issue(16 * (t + 3), st0);
      }
    }
    __syncthreads();  // planes, KL sums of this tile and rows of the next one complete
    if (krec >= 0) {  // threads 0-15: edge tid of the tile
      float s = 0.f;
#pragma unroll
      for (int ww = 0; ww < 8; ++ww) s += sm.red[b][ww][tid];
      klpart[krec] = s;
    }
    // ---- d_iq^T = ik^T dz^T: C[dim 16 w + 4 q4 + i][edge c]
    if (diq_wave) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kc = 0; kc < 4; ++kc) {
        // lane c reads keys ka + c / 4 and ka + 4 + c / 4, piece c % 4
        const int ka = 32 * kc + 8 * q4 + (c >> 2);
        const int oa = dz_offset(ka, c & 3), ob = dz_offset(ka + 4, c & 3);
        const bf16x8 bl = frag_tr_at(sm.dz[b][2] + oa, sm.dz[b][2] + ob);
        const bf16x8 bm = frag_tr_at(sm.dz[b][1] + oa, sm.dz[b][1] + ob);
        const bf16x8 bh = frag_tr_at(sm.dz[b][0] + oa, sm.dz[b][0] + ob);
        acc = mfma_t<DT>(ikt[kc], bl, acc);
        acc = mfma_t<DT>(ikt[kc], bm, acc);
        acc = mfma_t<DT>(ikt[kc], bh, acc);
      }
      if constexpr (DT == kF16) acc *= 1.f / kPScaleF16;
      if (myrec >= 0)
        __builtin_nontemporal_store(acc, reinterpret_cast<f32x4*>(diqpart + static_cast<int64_t>(myrec) * Di + 16 * wid + 4 * q4));
    }
  }

  // ---- this item's d_ik contribution in accumulator-fragment order:
  // ikpart[item][wave][dt][lane][i] holds key 16 wave + 4 q4 + i, dim 16 dt + c.
  if (need_dik) {
    f32x4* base = reinterpret_cast<f32x4*>(ikpart + static_cast<int64_t>(item) * 128 * Di) + wid * NDTI * 64 + lane;
#pragma unroll
    for (int dt = 0; dt < NDTI; ++dt) {
      if constexpr (DT == kF16) dik[dt] *= 1.f / kPScaleF16;
      __builtin_nontemporal_store(dik[dt], base + dt * 64);
    }
  }
}

// Per (token, group) of the chunk: KL = ln 2 * sum of the valid slots' partials and,
// when wanted, d_iq = gscale * sum of the slots' d_iq partials (FP64, slot order).
// 32 lanes per row, Di <= 128 (4 dims per lane).
__global__ __launch_bounds__(256) void kl_row_combine(const int32_t* __restrict__ indices,
                                                      const int32_t* __restrict__ cu, int nseq, int64_t t0, int64_t t1,
                                                      int G, int K, int B, int Di, double gscale,
                                                      const float* __restrict__ klpart,
                                                      const float* __restrict__ diqpart,
                                                      double* __restrict__ rowkl, float* __restrict__ row_kl,
                                                      float* __restrict__ diq) {
  const int sub = threadIdx.x & 31;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 8 + (threadIdx.x >> 5);
  if (r >= (t1 - t0) * G) return;
  const int64_t tl = r / G;
  const int g = static_cast<int>(r % G);
  const int64_t t = t0 + tl;
  const int s = find_seq(cu, nseq, t);
  const int64_t qb = (t - cu[s]) / B;
  const int32_t* sel = indices + (t * G + g) * K;
  const int64_t rec0 = (tl * G + g) * K;
  double kl = 0.0;
  for (int slot = sub; slot < K; slot += 32) {
    const int id = sel[slot];
    if (id >= 0 && id <= qb) kl += static_cast<double>(klpart[rec0 + slot]);
  }
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) kl += __shfl_xor(kl, o, 32);
  if (sub == 0) {
    rowkl[t * G + g] = kl * kLn2;
    if (row_kl) row_kl[t * G + g] = static_cast<float>(kl * kLn2);
  }
  if (diq && 4 * sub < Di) {
    // slots 8 at a time, all of their loads issued first (every slot's record is in
    // bounds; invalid slots are masked, never added)
    constexpr int kBatch = 8;
    double acc[4] = {0.0, 0.0, 0.0, 0.0};
    for (int s0 = 0; s0 < K; s0 += kBatch) {
      f32x4 x[kBatch];
      bool ok[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int slot = s0 + u < K ? s0 + u : K - 1;
        const int id = sel[slot];
        ok[u] = s0 + u < K && id >= 0 && id <= qb;
        x[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(diqpart + (rec0 + slot) * Di + 4 * sub));
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        if (ok[u]) {
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[i] += static_cast<double>(x[u][i]);
        }
      }
    }
    *reinterpret_cast<float4*>(diq + (t * G + g) * Di + 4 * sub) =
        make_float4(static_cast<float>(acc[0] * gscale), static_cast<float>(acc[1] * gscale),
                    static_cast<float>(acc[2] * gscale), static_cast<float>(acc[3] * gscale));
  }
}

// For chunk c: add the item partials of every group row of key block gb (groups in
// order, items in order) into the FP32 accumulator acc[key][dim]. Thread e owns
// fragment slot e (four keys, one dim). grid (total blocks, 128 * Di / 4 / 256).
template <int Di>
__global__ __launch_bounds__(256) void kl_accumulate(const int32_t* __restrict__ cu,
                                                     const int32_t* __restrict__ cu_blocks,
                                                     const int32_t* __restrict__ starts, int nseq, int G, int B,
                                                     const float* __restrict__ ikpart, float* __restrict__ acc) {
  constexpr int NDTI = Di / 16;
  const int64_t gb = blockIdx.x;
  const RowGeom rg = row_geom(cu, cu_blocks, nseq, gb * G, G, B);
  const int e = blockIdx.y * 256 + threadIdx.x;  // fragment slot: (wave, dt, lane)
  if (e >= 8 * NDTI * 64) return;
  const int w = e / (NDTI * 64), dt = (e / 64) % NDTI, ln = e % 64;
  const int kl0 = 16 * w + 4 * (ln >> 4), d = 16 * dt + (ln & 15);
  if (kl0 >= rg.nk) return;
  float s[4] = {0.f, 0.f, 0.f, 0.f};
  bool any = false;
  for (int g = 0; g < G; ++g) {
    const int64_t row = gb * G + g;
    const int i0 = starts[row], i1 = starts[row + 1];
    for (int i = i0; i < i1; ++i) {
      const f32x4 x = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(ikpart + static_cast<int64_t>(i) * 128 * Di) + e);
#pragma unroll
      for (int j = 0; j < 4; ++j) s[j] += x[j];
      any = true;
    }
  }
  if (!any) return;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (kl0 + j < rg.nk) acc[(rg.kb + kl0 + j) * Di + d] += s[j];
}

// One workgroup: loss = sum of the row KLs (fixed order, FP64) / rows.
__global__ __launch_bounds__(1024) void kl_loss(const double* __restrict__ rowkl, int64_t n, double inv_rows,
                                                float* __restrict__ loss) {
  __shared__ double part[1024];
  double s = 0.0;
  for (int64_t i = threadIdx.x; i < n; i += 1024) s += rowkl[i];
  part[threadIdx.x] = s;
  __syncthreads();
  for (int o = 512; o > 0; o >>= 1) {
    if (static_cast<int>(threadIdx.x) < o) part[threadIdx.x] += part[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) loss[0] = static_cast<float>(part[0] * inv_rows);
}

__global__ __launch_bounds__(256) void kl_scale(const float* __restrict__ acc, int64_t n, float s,
                                                float* __restrict__ out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) out[i] = acc[i] * s;
}

__global__ __launch_bounds__(256) void kl_zero(float* __restrict__ p, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) p[i] = 0.f;
}

// ---------------------------------------------------------------------------- host side

namespace {

struct KlLayout {
  KvPlan plan;
  int64_t tpart, spart, tstate, sstate, klpart, diqpart, ikpart, acc, rowkl, total;
};

int kl_nk(int64_t dim) { return dim == 32 ? 1 : dim == 64 ? 2 : dim == 128 ? 4 : 0; }

bool kl_supported(int64_t Hq, int64_t G, int64_t D, int64_t Di, int64_t B) {
  return G > 0 && Hq % G == 0 && Hq / G <= kKlMaxRatio && kl_nk(D) && kl_nk(Di) && B > 0 && B <= 128;
}

KlLayout kl_layout(int64_t T, int64_t Hq, int64_t G, int64_t Di, int64_t K, int64_t total_blocks) {
  KlLayout L;
  const int64_t rows = total_blocks * G;
  // per (token, slot): teacher (m, l) per head, student (m, l), KL and d_iq per group
  const int64_t rec = Hq * 8 + G * (8 + 4 + 4 * Di);
  const int64_t tc = kv_chunk_tokens(T, 1, K, rec, kv_chunk_budget(kPassKl, int64_t(1) << 30));
  L.plan = kv_plan_layout(T, rows, G, K, tc, kKlEdges);
  int64_t off = align256(L.plan.bytes);
  L.tpart = off;   off += align256(tc * Hq * K * 8);
  L.spart = off;   off += align256(tc * G * K * 8);
  L.tstate = off;  off += align256(T * Hq * 16);
  L.sstate = off;  off += align256(T * G * 16);
  L.klpart = off;  off += align256(tc * G * K * 4);
  L.diqpart = off; off += align256(tc * G * K * Di * 4);
  L.ikpart = off;  off += align256(L.plan.max_items * 128 * Di * 4);
  L.acc = off;     off += align256(T * Di * 4);
  L.rowkl = off;   off += align256(T * G * 8);
  L.total = off;
  return L;
}

}  // namespace

}  // namespace msa

using namespace msa;

extern "C" int64_t msa_indexer_kl_workspace_bytes(int32_t dtype, int64_t total_tokens, int64_t q_heads,
                                                  int64_t kv_groups, int64_t head_dim, int64_t index_dim,
                                                  int64_t topk_slots, int64_t total_blocks, int64_t block_size) {
  if ((dtype != kBF16 && dtype != kF16) || total_tokens <= 0 || topk_slots < 0 || total_blocks < 0) return 0;
  if (!kl_supported(q_heads, kv_groups, head_dim, index_dim, block_size)) return 0;
  return kl_layout(total_tokens, q_heads, kv_groups, index_dim, topk_slots, total_blocks).total;
}

extern "C" int msa_indexer_kl(const void* index_q, const void* index_k, const void* q, const void* k, int32_t dtype,
                              const int32_t* indices, const int32_t* cu_seqlens, int64_t num_seqs,
                              int64_t total_tokens, int64_t q_heads, int64_t kv_groups, int64_t head_dim,
                              int64_t index_dim, int64_t topk_slots, int64_t block_size, double index_scale,
                              double scale, const int32_t* cu_block_lens, int64_t total_blocks,
                              const int32_t* row_ptr, const int32_t* query_indices, const int32_t* slot_indices,
                              const float* teacher_lse, float* loss, float* row_kl, float* grad_index_q,
                              float* grad_index_k, void* workspace, int64_t workspace_bytes, void* stream) {
  if (num_seqs <= 0 || total_tokens < 0 || topk_slots < 0 || total_blocks < 0 || !loss || q_heads <= 0 ||
      kv_groups <= 0 || q_heads % kv_groups)
    return kErrInvalidArgument;
  if ((dtype != kBF16 && dtype != kF16) || !kl_supported(q_heads, kv_groups, head_dim, index_dim, block_size))
    return kErrUnsupported;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t T = total_tokens, Hq = q_heads, G = kv_groups, D = head_dim, Di = index_dim, K = topk_slots;
  if (T == 0) {
    hipLaunchKernelGGL(kl_zero, dim3(1), dim3(256), 0, st, loss, 1);
    return status_from(hipGetLastError());
  }
  if (!kv_csr_fits(T, G, K, total_blocks * G)) return kErrUnsupported;
  if (!cu_block_lens || !row_ptr || !workspace || !indices || !cu_seqlens || (K > 0 && (!query_indices || !slot_indices)))
    return kErrInvalidArgument;
  const KlLayout L = kl_layout(T, Hq, G, Di, K, total_blocks);
  if (workspace_bytes < L.total) return kErrInvalidArgument;
  if (!kv_chunk_records_fit(L.plan.tc, Hq, K)) return kErrUnsupported;
  char* base = static_cast<char*>(workspace);
  auto* tpart = reinterpret_cast<float2*>(base + L.tpart);
  auto* spart = reinterpret_cast<float2*>(base + L.spart);
  auto* tstate = reinterpret_cast<float4*>(base + L.tstate);
  auto* sstate = reinterpret_cast<float4*>(base + L.sstate);
  auto* klpart = reinterpret_cast<float*>(base + L.klpart);
  auto* diqpart = reinterpret_cast<float*>(base + L.diqpart);
  auto* ikpart = reinterpret_cast<float*>(base + L.ikpart);
  auto* acc = reinterpret_cast<float*>(base + L.acc);
  auto* rowkl = reinterpret_cast<double*>(base + L.rowkl);
  const auto* iqb = static_cast<const uint16_t*>(index_q);
  const auto* ikb = static_cast<const uint16_t*>(index_k);
  const auto* qb = static_cast<const uint16_t*>(q);
  const auto* kb = static_cast<const uint16_t*>(k);
  const int nseq = static_cast<int>(num_seqs), iHq = static_cast<int>(Hq), iG = static_cast<int>(G);
  const int iK = static_cast<int>(K), iB = static_cast<int>(block_size), iDi = static_cast<int>(Di);
  const float zs2 = static_cast<float>(index_scale) * kLog2e, as2 = static_cast<float>(scale) * kLog2e;
  const double rows_tg = static_cast<double>(T * G);
  const double gscale = index_scale / rows_tg;
  const int64_t rows = total_blocks * G;
  const KvPlan& pl = L.plan;
  const int nk = kl_nk(D), nki = kl_nk(Di);
  const int need_diq = grad_index_q != nullptr, need_dik = grad_index_k != nullptr;

  if (need_dik) hipLaunchKernelGGL(kl_zero, dim3(grid_1d(T * Di, 256)), dim3(256), 0, st, acc, T * Di);
  kv_plan_launch(pl, row_ptr, query_indices, T, base, st);
  for (int64_t ch = 0; ch < pl.nch; ++ch) {
    const int64_t t0 = ch * pl.tc, t1 = t0 + pl.tc < T ? t0 + pl.tc : T;
    const int it0 = static_cast<int>(t0);
    const int32_t* hi = kv_plan_hi(pl, base, ch);
    const int32_t* nit = kv_plan_count(pl, base, ch);
    const int2* its = kv_plan_items(pl, base, ch);
    const int32_t* ord = kv_plan_order(pl, base, ch);
    const int epi = static_cast<int>(pl.epi);
    const dim3 grid(static_cast<unsigned>(pl.max_items > 0 ? pl.max_items : 1)), block(kKlThreads);
    if (rows > 0 && pl.max_items > 0) {
#define MSA_KL_STATS(DTV, A, C) hipLaunchKernelGGL((kl_stats_kernel<DTV, A, C>), grid, block, 0, st, iqb, ikb, qb, kb, cu_seqlens, cu_block_lens, query_indices, slot_indices, hi, nit, its, ord, nseq, iHq, iG, iK, iB, zs2, as2, epi, it0, teacher_lse ? 0 : 1, tpart, spart)
#define MSA_KL_DISPATCH_DT(M, DTV)                                                         \
  if (nk == 1) { if (nki == 1) M(DTV, 1, 1); else if (nki == 2) M(DTV, 1, 2); else M(DTV, 1, 4); }       \
  else if (nk == 2) { if (nki == 1) M(DTV, 2, 1); else if (nki == 2) M(DTV, 2, 2); else M(DTV, 2, 4); }  \
  else { if (nki == 1) M(DTV, 4, 1); else if (nki == 2) M(DTV, 4, 2); else M(DTV, 4, 4); }
#define MSA_KL_DISPATCH(M) \
  if (dtype == kF16) { MSA_KL_DISPATCH_DT(M, kF16) } else { MSA_KL_DISPATCH_DT(M, kBF16) }
      MSA_KL_DISPATCH(MSA_KL_STATS)
#undef MSA_KL_STATS
    }
    hipLaunchKernelGGL(kl_stats_combine, dim3(grid_1d((t1 - t0) * (Hq + G), 16)), dim3(256), 0, st, indices,
                       cu_seqlens, nseq, t0, t1, iHq, iG, iK, iB, tpart, spart, teacher_lse, tstate, sstate);
    if (rows > 0 && pl.max_items > 0) {
#define MSA_KL_MAIN(DTV, A, C) hipLaunchKernelGGL((kl_main_kernel<DTV, A, C>), grid, block, 0, st, iqb, ikb, qb, kb, tstate, sstate, cu_seqlens, cu_block_lens, query_indices, slot_indices, hi, nit, its, ord, nseq, iHq, iG, iK, iB, zs2, as2, epi, it0, need_diq, need_dik, klpart, diqpart, ikpart)
      MSA_KL_DISPATCH(MSA_KL_MAIN)
#undef MSA_KL_MAIN
#undef MSA_KL_DISPATCH
#undef MSA_KL_DISPATCH_DT
    }
    hipLaunchKernelGGL(kl_row_combine, dim3(grid_1d((t1 - t0) * G, 8)), dim3(256), 0, st, indices, cu_seqlens, nseq,
                       t0, t1, iG, iK, iB, iDi, gscale, klpart, diqpart, rowkl, row_kl, grad_index_q);
    if (need_dik && rows > 0 && pl.max_items > 0) {
      const int32_t* starts = kv_plan_starts(pl, base, ch);
      const dim3 agrid(static_cast<unsigned>(total_blocks), static_cast<unsigned>((8 * (Di / 16) * 64 + 255) / 256));
      if (nki == 1) hipLaunchKernelGGL(kl_accumulate<32>, agrid, dim3(256), 0, st, cu_seqlens, cu_block_lens, starts, nseq, iG, iB, ikpart, acc);
      else if (nki == 2) hipLaunchKernelGGL(kl_accumulate<64>, agrid, dim3(256), 0, st, cu_seqlens, cu_block_lens, starts, nseq, iG, iB, ikpart, acc);
      else hipLaunchKernelGGL(kl_accumulate<128>, agrid, dim3(256), 0, st, cu_seqlens, cu_block_lens, starts, nseq, iG, iB, ikpart, acc);
    }
  }
  hipLaunchKernelGGL(kl_loss, dim3(1), dim3(1024), 0, st, rowkl, T * G, 1.0 / rows_tg, loss);
  if (need_dik)
    hipLaunchKernelGGL(kl_scale, dim3(grid_1d(T * Di, 256)), dim3(256), 0, st, acc, T * Di, static_cast<float>(gscale),
                       grad_index_k);
  return status_from(hipGetLastError());
}
