// Stage 3 forward, KV-major (bf16 and fp16 inputs).
//
// Query-major attention streams each token's selected K/V blocks (K/V bytes
// gathered per token = #slots x block x D x 4: ~137 GB at 32K tokens). Here the
// k2q CSR (built from the indices) drives the work instead: a workgroup owns a
// (key block, group) row -- its K and V blocks sit in LDS, row-major -- and streams the row's edges, i.e. the (query token, slot) pairs
// that selected the block, 128 (edge, head) rows per tile. Each (edge, head)
// row yields a partial softmax over the block in base 2:
//   m = max_j s_j, l = sum_j 2^(s_j - m), O = sum_j 2^(s_j - m) v_j   (fp32),
// with s_j = fl(q.k_j * scale * log2(e)), stored per (token, slot, head): the heads
// of one edge are adjacent, so an edge's rows write one contiguous run. A
// combine kernel then merges the <= K partials of each (token, head) in slot
// order in FP64:
//   M = max m_s, L = sum 2^(m_s - M) l_s, out = sum 2^(m_s - M) O_s / L,
//   lse = (M + log2 L) ln 2.
// Query tokens are processed in chunks so the partial buffer stays bounded;
// inside each CSR row the edges of a chunk form a contiguous range because rows
// are ordered by query token.
//
// Partial records are written and read once each, with non-temporal (streaming)
// stores and loads: the partial pass is bound by their write traffic.
//
// The logits use the K row fragment and the Q row fragment over the same dims
// in the same k order as the backward kernels. P.V is computed exactly in its
// products: P is split into three terms of the input type (hi + mid + lo == P); fp16
// splits 2^15 P (fp16's exponent range ends at 2^-24), and the partial O carries that
// factor until the combine divides it out.
#include <atomic>
#include <type_traits>

#include "attn_kv_common.hpp"
#include "profile.hpp"

// Logits are x = fl(acc * scale2) with their own rounding, and exponent arguments
// x - m with another: no fused multiply-adds, so a row's maximum gets p == 1 exactly.
#pragma clang fp contract(off)

namespace msa {

namespace {

constexpr int kRowsPerTile = 128;  // (edge, head) rows per tile
constexpr int kTilesPerItem = 4;   // tiles per work item
constexpr int kItemRows = kRowsPerTile * kTilesPerItem;

// Workgroup shape of the partial pass: 4 waves x 32 rows (two 16-row operands per wave)
// up to 128 dims; 8 waves x 16 rows at 256 dims, whose query fragments, logits and
// output accumulators of 16 rows fill what 32 rows take at 128 dims (the K and V blocks,
// 136 KiB of LDS there, leave one workgroup per CU: two waves per SIMD).
template <int NK>
struct FwdShape {
  static constexpr int kWaves = NK == 8 ? 8 : 4;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kRT = kRowsPerTile / (16 * kWaves);  // 16-row operands per wave
};

template <int NK>
struct FwdSmem {
  static constexpr int DP = 32 * NK;
  // Row stride of the K and V blocks (bf16): DP + 16 halves (288 bytes at DP = 128) puts
  // both the row-fragment reads of K (ds_read_b128, lane c -> row c) and the transposed
  // reads of V (ds_read_b64_tr_b16, four rows x 32 bytes per 16 lanes) on distinct banks;
  // DP + 8 leaves both 2-way conflicted.
  static constexpr int KS = DP + 16;
  alignas(16) uint16_t k[128 * KS];
  alignas(16) uint16_t v[128 * KS];
  int32_t th[kItemRows];   // (token - t0) * Hq + head (chunk-local)
  int32_t tok[kItemRows];  // query token
  int32_t rec[kItemRows];  // partial record kv_record(token - t0, head, slot)
};

}  // namespace

// Per row, the first edge whose query token is >= c * tc, for c = 0..nch
// (bounds[c * rows + row]); bound nch is the row end. One wavefront per row, one
// lane per chunk boundary (independent binary searches over the row's edges).
__global__ __launch_bounds__(256) void kv_chunk_bounds(const int32_t* __restrict__ row_ptr,
                                                       const int32_t* __restrict__ qidx, int64_t rows, int64_t T,
                                                       int64_t tc, int nch, int32_t* __restrict__ bounds) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int32_t a = row_ptr[r], b = row_ptr[r + 1];
  for (int c = threadIdx.x & 63; c <= nch; c += kWave) {
    const int64_t t = c * tc < T ? c * tc : T;
    int32_t lo = a, hi = b;
    while (lo < hi) {
      const int32_t mid = lo + ((hi - lo) >> 1);  // lo + hi may exceed INT32_MAX
      if (qidx[mid] < t) lo = mid + 1; else hi = mid;
    }
    bounds[c * rows + r] = (c == nch) ? b : lo;
  }
}

// For chunk blockIdx.x: the exclusive prefix over rows of ceil(edges / epi) work
// items, item_start[c * (rows + 1) + row], with the chunk total at index rows,
// and the item table items[c * max_items + i] = (row, first edge of the item).
__global__ __launch_bounds__(1024) void kv_item_scan(const int32_t* __restrict__ bounds, int64_t rows, int epi,
                                                      int64_t max_items, int32_t* __restrict__ item_start,
                                                      int2* __restrict__ items) {
  __shared__ int32_t wsum[16];
  __shared__ int32_t carry_s;
  const int64_t c = blockIdx.x;
  const int32_t* lo_b = bounds + c * rows;
  const int32_t* hi_b = bounds + (c + 1) * rows;
  int32_t* out = item_start + c * (rows + 1);
  if (threadIdx.x == 0) carry_s = 0;
  __syncthreads();
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  for (int64_t base = 0; base < rows; base += 1024) {
    const int64_t r = base + threadIdx.x;
    const int32_t n = r < rows ? (hi_b[r] - lo_b[r] + epi - 1) / epi : 0;
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
    if (r < rows) {
      const int32_t first = carry + (wid > 0 ? wsum[wid - 1] : 0) + x - n;
      out[r] = first;
      int2* dst = items + c * max_items + first;  // first + n <= chunk total <= max_items
      for (int32_t j = 0; j < n; ++j) dst[j] = make_int2(static_cast<int32_t>(r), lo_b[r] + j * epi);
    }
    __syncthreads();
    if (threadIdx.x == 0) carry_s = carry + wsum[15];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[rows] = carry_s;
}

// For chunk blockIdx.x: order[slot] = the chunk's work items by decreasing edge count
// (a counting sort on epi - edges, clamped to kOrderBuckets - 1). Launched in this
// order, the short items (row tails) are the last to start, so the workgroups of a
// launch finish closer together. Items of equal size take their slots in no fixed
// order (integer atomics); no result depends on it, as each item writes only its own
// outputs, indexed by item.
constexpr int kOrderBuckets = 1024;
__global__ __launch_bounds__(1024) void kv_item_order(const int32_t* __restrict__ bounds, int64_t rows, int epi,
                                                       int64_t max_items, const int32_t* __restrict__ item_start,
                                                       const int2* __restrict__ items, int32_t* __restrict__ order,
                                                       int row_order) {
  __shared__ int32_t cnt[kOrderBuckets];
  __shared__ int32_t wsum[16];
  const int64_t c = blockIdx.x;
  const int32_t* hi_b = bounds + (c + 1) * rows;
  const int2* its = items + c * max_items;
  int32_t* out = order + c * max_items;
  const int32_t n = item_start[c * (rows + 1) + rows];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  if (row_order) {  // the identity (testing hook)
    for (int32_t i = tid; i < n; i += 1024) out[i] = i;
    return;
  }
  auto bucket = [&](int32_t i) {
    const int2 it = its[i];
    const int32_t left = hi_b[it.x] - it.y;  // edges from the item's first to the row's end
    const int32_t b = epi - (left < epi ? left : epi);
    return b < kOrderBuckets ? b : kOrderBuckets - 1;
  };
  // Most items are full (bucket 0): those take one LDS atomic per wave, ranked by ballot.
  cnt[tid] = 0;
  __syncthreads();
  for (int32_t i0 = 0; i0 < n; i0 += 1024) {  // whole waves iterate together (ballots)
    const int32_t i = i0 + tid;
    const int32_t b = i < n ? bucket(i) : -1;
    const uint64_t full = __ballot(b == 0);
    if (full != 0 && lane == static_cast<int>(__ffsll(static_cast<long long>(full)) - 1))
      atomicAdd(&cnt[0], __popcll(full));
    if (b > 0) atomicAdd(&cnt[b], 1);
  }
  __syncthreads();
  // exclusive prefix over the buckets (thread tid owns bucket tid)
  const int32_t own = cnt[tid];
  int32_t x = own;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int32_t y = __shfl_up(x, o, kWave);
    if (lane >= o) x += y;
  }
  if (lane == 63) wsum[wid] = x;
  __syncthreads();
  if (tid < 16) {
    int32_t w = wsum[tid];
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
      const int32_t y = __shfl_up(w, o, 16);
      if (tid >= o) w += y;
    }
    wsum[tid] = w;
  }
  __syncthreads();
  cnt[tid] = (wid > 0 ? wsum[wid - 1] : 0) + x - own;
  __syncthreads();
  for (int32_t i0 = 0; i0 < n; i0 += 1024) {
    const int32_t i = i0 + tid;
    const int32_t b = i < n ? bucket(i) : -1;
    const uint64_t full = __ballot(b == 0);
    const int lead = full != 0 ? static_cast<int>(__ffsll(static_cast<long long>(full))) - 1 : 0;
    int32_t base = 0;
    if (full != 0 && lane == lead) base = atomicAdd(&cnt[0], __popcll(full));
    base = __shfl(base, lead, kWave);
    if (b == 0) out[base + __popcll(full & ((uint64_t(1) << lane) - 1))] = i;
    else if (b > 0) out[atomicAdd(&cnt[b], 1)] = i;
  }
}

template <int DT, int NK, bool FULLD>
__global__ __launch_bounds__(FwdShape<NK>::kThreads, NK == 8 ? 1 : 2) void attn_fwd_partial_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const int32_t* __restrict__ cu, const int32_t* __restrict__ cu_blocks, const int32_t* __restrict__ qidx,
    const int32_t* __restrict__ sidx, const int32_t* __restrict__ e_hi, const int32_t* __restrict__ n_items,
    const int2* __restrict__ items, const int32_t* __restrict__ order, int nseq, int Hq, int G, int D, int K, int B, float scale2, int epi, int t0,
    float* __restrict__ opart, float2* __restrict__ mlpart) {
  constexpr int DP = 32 * NK, NDT = DP / 16, KS = FwdSmem<NK>::KS;
  constexpr int NT = FwdShape<NK>::kThreads, RT = FwdShape<NK>::kRT;
  __shared__ FwdSmem<NK> sm;
  if (static_cast<int>(blockIdx.x) >= *n_items) return;
  const int item = order[blockIdx.x];  // largest items first
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63, c = lane & 15, q4 = lane >> 4;
  const int2 it = items[item];
  const int row = it.x, e_begin = it.y;
  const RowGeom rg = row_geom(cu, cu_blocks, nseq, row, G, B);
  const int R = Hq / G;
  const int e_end = e_begin + epi < e_hi[row] ? e_begin + epi : e_hi[row];
  const int nrows = (e_end - e_begin) * R;  // <= kItemRows

  // ---- stage the K and V blocks (row-major) and the item's row metadata in LDS.
  // All global loads are issued before any LDS store.
  constexpr int KVI = 128 * (DP / 8) / NT;  // 16-byte K (and V) loads per thread
  uint4 kw[KVI], vw[KVI];
#pragma unroll
  for (int it = 0; it < KVI; ++it) {
    const int e = tid + NT * it;
    const int kl = e / (DP / 8), d0 = 8 * (e % (DP / 8));  // lanes along dims
    // unconditional loads from clamped (in-bounds) addresses; out-of-range lanes are zeroed at the store
    const int klc = kl < rg.nk ? kl : rg.nk - 1, d0c = (FULLD || d0 < D) ? d0 : D - 8;
    const int64_t off = ((rg.kb + klc) * G + rg.g) * D + d0c;
    kw[it] = *reinterpret_cast<const uint4*>(k + off);
    vw[it] = *reinterpret_cast<const uint4*>(v + off);
  }
  constexpr int MI = kItemRows / NT;
  int32_t mtok[MI], mslot[MI];
#pragma unroll
  for (int j = 0; j < MI; ++j) {
    const int rho = tid + NT * j;
    const int eo = (rho < nrows ? rho : nrows - 1) / R;  // nrows >= 1
    mtok[j] = qidx[e_begin + eo];
    mslot[j] = sidx[e_begin + eo];
  }
#pragma unroll
  for (int it = 0; it < KVI; ++it) {
    const int e = tid + NT * it;
    const int kl = e / (DP / 8), d0 = 8 * (e % (DP / 8));
    const bool ok = kl < rg.nk && (FULLD || d0 < D);
    *reinterpret_cast<uint4*>(sm.k + kl * KS + d0) = ok ? kw[it] : make_uint4(0u, 0u, 0u, 0u);
    *reinterpret_cast<uint4*>(sm.v + kl * KS + d0) = ok ? vw[it] : make_uint4(0u, 0u, 0u, 0u);
  }
#pragma unroll
  for (int j = 0; j < MI; ++j) {
    const int rho = tid + NT * j;
    if (rho < nrows) {
      const int eo = rho / R;
      const int h = rg.g * R + (rho - eo * R);
      sm.th[rho] = (mtok[j] - t0) * Hq + h;  // < tc * Hq: chunk records fit in int32 (checked on the host)
      sm.tok[rho] = mtok[j];
      sm.rec[rho] = kv_record(mtok[j] - t0, h, mslot[j], Hq, K);
    }
  }
  __syncthreads();

  // Waves are independent from here on. Wave wid owns rows r0 + 16*RT*wid + 16*rt + c of each tile.
  const int ntiles = (nrows + kRowsPerTile - 1) / kRowsPerTile;
  bf16x8 qf[RT][NK];
  auto load_q = [&](int r0) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int rho = r0 + 16 * RT * wid + 16 * rt + c;
      const bool ok = rho < nrows;
      const int64_t th = ok ? static_cast<int64_t>(t0) * Hq + sm.th[rho] : 0;
#pragma unroll
      for (int kk = 0; kk < NK; ++kk) {
        const int d0 = 32 * kk + 8 * q4;
        qf[rt][kk] = (ok && (FULLD || d0 < D)) ? load_frag(q + th * D + d0) : zero_frag();
      }
    }
  };
  load_q(0);
  for (int tile = 0; tile < ntiles; ++tile) {
    const int r0 = tile * kRowsPerTile;
    const int rbase = r0 + 16 * RT * wid;
    if (rbase >= nrows) break;  // wave-uniform: no rows of this wave are left
    int lim[RT];  // visible keys of the lane's rows
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int rho = rbase + 16 * rt + c;
      const int64_t vis = rho < nrows ? static_cast<int64_t>(sm.tok[rho]) - rg.kb + 1 : 0;
      lim[rt] = vis < rg.nk ? static_cast<int>(vis) : rg.nk;
    }
    // ---- logits S^T = K Q^T: lane holds S[row 16*rt + c][key 16*kt + 4*q4 + i]
    f32x4 s[RT][8];
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) {
      bf16x8 kf[NK];
#pragma unroll
      for (int kk = 0; kk < NK; ++kk)
        kf[kk] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(sm.k + (16 * kt + c) * KS + 32 * kk + 8 * q4));
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < NK; ++kk) a = mfma_t<DT>(kf[kk], qf[rt][kk], a);
        s[rt][kt] = a;
      }
    }
    // Q fragments are dead: prefetch the next tile's rows.
    if (tile + 1 < ntiles) load_q(r0 + kRowsPerTile);
    // ---- base-2 partial softmax per row (rows of the lane's quad share c):
    // x = fl(acc * scale2), m = max x, p = 2^(x - m) (exactly 1 at the maximum).
    // Wave-uniform: every row of the wave sees all 128 keys (no masks), or not. The two
    // cases are separate code paths so the unmasked one carries no per-logit selects.
    bool part = false;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) part = part || lim[rt] < 128;
    const bool full = __ballot(part) == 0;
    float mrow[RT], lrow[RT];
    f32x4 o[RT][NDT];
    auto softmax_pv = [&](auto full_tag) __attribute__((always_inline)) {
      constexpr bool FULL = decltype(full_tag)::value;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        float m = -__builtin_inff();
#pragma unroll
        for (int kt = 0; kt < 8; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float x = s[rt][kt][i] * scale2;
            if constexpr (!FULL) x = (16 * kt + 4 * q4 + i < lim[rt]) ? x : -__builtin_inff();
            s[rt][kt][i] = x;
            m = fmaxf(m, x);
          }
        m = quad_max(m);
        const float base = m == -__builtin_inff() ? 0.f : m;
        float l = 0.f;
#pragma unroll
        for (int kt = 0; kt < 8; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float p = __builtin_amdgcn_exp2f(s[rt][kt][i] - base);
            s[rt][kt][i] = p;
            l += p;
          }
        l += __shfl_xor(l, 16, kWave);
        l += __shfl_xor(l, 32, kWave);
        mrow[rt] = m;
        lrow[rt] = l;
      }
      // ---- O^T = V^T P^T over 4 chunks of 32 keys: A = V^T[dim c][keys pi], B = P^T[keys pi][row c]
#pragma unroll
      for (int kc = 0; kc < 4; ++kc) {
        bf16x8 ph[RT], pm[RT], pl[RT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          uint32_t wh[4], wm[4], wl[4];
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            // elements j = 2*jj, 2*jj + 1 -> C tile 2*kc + j/4, entry j%4
            const int j0 = 2 * jj, j1 = 2 * jj + 1;
            const float x0 = s[rt][2 * kc + j0 / 4][j0 % 4], x1 = s[rt][2 * kc + j1 / 4][j1 % 4];
            if constexpr (DT == kF16)
              split3_pk_f16(x0 * kPScaleF16, x1 * kPScaleF16, wh[jj], wm[jj], wl[jj]);
            else
              split3_pk(x0, x1, wh[jj], wm[jj], wl[jj]);
          }
          ph[rt] = __builtin_bit_cast(bf16x8, make_uint4(wh[0], wh[1], wh[2], wh[3]));
          pm[rt] = __builtin_bit_cast(bf16x8, make_uint4(wm[0], wm[1], wm[2], wm[3]));
          pl[rt] = __builtin_bit_cast(bf16x8, make_uint4(wl[0], wl[1], wl[2], wl[3]));
        }
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          // V^T[dim 16*dt + c][keys pi(q4, j)] read transposed from the row-major V block
          const bf16x8 vb = frag_tr(sm.v, KS, 32 * kc + 4 * q4, 32 * kc + 16 + 4 * q4, 16 * dt, c);
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) {
            f32x4 acc = kc == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : o[rt][dt];
            acc = mfma_t<DT>(vb, pl[rt], acc);
            acc = mfma_t<DT>(vb, pm[rt], acc);
            o[rt][dt] = mfma_t<DT>(vb, ph[rt], acc);
          }
        }
      }
    };
    if (full)
      softmax_pv(std::true_type{});
    else
      softmax_pv(std::false_type{});
    // ---- store partials: o lane holds O[row 16*rt + c][dims 16*dt + 4*q4 + 0..3]
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int rho = rbase + 16 * rt + c;
      if (rho < nrows) {
        float* dst = opart + static_cast<int64_t>(sm.rec[rho]) * D + 4 * q4;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
          if (FULLD || 16 * dt + 4 * q4 < D) __builtin_nontemporal_store(o[rt][dt], reinterpret_cast<f32x4*>(dst + 16 * dt));
      }
      if (q4 == 0 && rho < nrows) mlpart[sm.rec[rho]] = make_float2(mrow[rt], lrow[rt]);
    }
  }
}

// 32 lanes per (token, head) of the chunk, 4 dims in each of DC 128-dim halves (D <= 128 DC): merge the
// valid slots' partials in slot order in FP64. Slots are taken 8 at a time with
// all of their partial loads issued before any arithmetic (records are in bounds
// for every slot, valid or not; invalid slots are masked, never multiplied).
constexpr int kCombineBatch = 8;
// A row is flat when sum_j 2^(x_j - max x) >= kFlatRowMass, i.e. no key has probability
// above 5 %; then sum_j p_j^2 <= 0.05 and the delta = O . dO shortcut's extra dQ / dK
// error term (~ sqrt(sum p^2) times the statistics pass's error) stays below ~22 % of
// it, ~2.5 % in quadrature. Measured: the same count of one-ulp bf16 flips against the
// FP64 oracle as the statistics pass for every row, at logit scales 0.3x to 16x.
constexpr double kFlatRowMass = 20.0;

template <int DT, int DC>
__global__ __launch_bounds__(256) void attn_fwd_combine(const int32_t* __restrict__ indices,
                                                        const int32_t* __restrict__ cu, int nseq, int64_t t0,
                                                        int64_t t1, int Hq, int G, int D, int K, int B,
                                                        const float* __restrict__ opart,
                                                        const float2* __restrict__ mlpart, uint16_t* __restrict__ out,
                                                        float* __restrict__ lse, double* __restrict__ row_state,
                                                        float* __restrict__ o32) {
  const int sub = threadIdx.x & 31;
  const int64_t th = t0 * Hq + static_cast<int64_t>(blockIdx.x) * 8 + (threadIdx.x >> 5);
  if (th >= t1 * Hq) return;  // whole 32-lane segments exit together
  const int64_t t = th / Hq;
  const int h = static_cast<int>(th % Hq);
  const int g = h / (Hq / G);
  const int s = find_seq(cu, nseq, t);
  const int64_t qb = (t - cu[s]) / B;
  const int32_t* sel = indices + (t * G + g) * K;
  const int64_t rec0 = kv_record(t - t0, h, 0, Hq, K);  // slot j: rec0 + j * Hq

  // slot sub (and sub + 32, ...) of this row: validity and (m, l)
  float M = -__builtin_inff();
  for (int s0 = 0; s0 < K; s0 += 32) {
    const int slot = s0 + sub;
    if (slot < K) {
      const int id = sel[slot];
      if (id >= 0 && id <= qb) M = fmaxf(M, mlpart[rec0 + slot * Hq].x);
    }
  }
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 32));

  double L = 0.0;
  double acc[DC][4];
  bool has_dims[DC];
  int dcol[DC];
#pragma unroll
  for (int hc = 0; hc < DC; ++hc) {
    acc[hc][0] = acc[hc][1] = acc[hc][2] = acc[hc][3] = 0.0;
    has_dims[hc] = 128 * hc + 4 * sub < D;
    dcol[hc] = has_dims[hc] ? 128 * hc + 4 * sub : 0;  // lanes without dims read (and ignore) dims 0..3
  }
  if (M != -__builtin_inff()) {
    for (int s0 = 0; s0 < K; s0 += 32) {
      const int slot = s0 + sub;
      double w = 0.0;
      if (slot < K) {
        const int id = sel[slot];
        if (id >= 0 && id <= qb) {
          const float2 ml = mlpart[rec0 + slot * Hq];
          w = exp2(static_cast<double>(ml.x) - static_cast<double>(M));
          L = fma(w, static_cast<double>(ml.y), L);
        }
      }
      const int n = K - s0 < 32 ? K - s0 : 32;
      // the two 32-lane halves of the wave hold two rows: slot j's weight comes from
      // lane j of this half (wave-uniform readlanes of both halves, then a select)
      const bool upper = (threadIdx.x & 32) != 0;
      const uint64_t wbits = __double_as_longlong(w);
      const uint32_t wlo = static_cast<uint32_t>(wbits), whi = static_cast<uint32_t>(wbits >> 32);
      for (int j0 = 0; j0 < n; j0 += kCombineBatch) {
        float4 op[kCombineBatch][DC];
#pragma unroll
        for (int u = 0; u < kCombineBatch; ++u) {
          const int j = j0 + u < n ? j0 + u : n - 1;
#pragma unroll
          for (int hc = 0; hc < DC; ++hc) {
            const f32x4 x = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(opart + (rec0 + static_cast<int64_t>(s0 + j) * Hq) * D + dcol[hc]));
            op[u][hc] = make_float4(x[0], x[1], x[2], x[3]);
          }
        }
#pragma unroll
        for (int u = 0; u < kCombineBatch; ++u) {
          const int j = j0 + u < n ? j0 + u : 0;
          const uint32_t alo = __builtin_amdgcn_readlane(wlo, j), ahi = __builtin_amdgcn_readlane(whi, j);
          const uint32_t blo = __builtin_amdgcn_readlane(wlo, 32 + j), bhi = __builtin_amdgcn_readlane(whi, 32 + j);
          const double wj = __longlong_as_double(static_cast<long long>(
              (static_cast<uint64_t>(upper ? bhi : ahi) << 32) | (upper ? blo : alo)));
          if (j0 + u < n && wj != 0.0) {  // invalid slot (or a weight that underflowed to zero)
#pragma unroll
            for (int hc = 0; hc < DC; ++hc) {
              acc[hc][0] = fma(wj, static_cast<double>(op[u][hc].x), acc[hc][0]);
              acc[hc][1] = fma(wj, static_cast<double>(op[u][hc].y), acc[hc][1]);
              acc[hc][2] = fma(wj, static_cast<double>(op[u][hc].z), acc[hc][2]);
              acc[hc][3] = fma(wj, static_cast<double>(op[u][hc].w), acc[hc][3]);
            }
          }
        }
      }
    }
  }
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) L += __shfl_xor(L, o, 32);
  const bool has = L > 0.0;
#pragma unroll
  for (int hc = 0; hc < DC; ++hc) {
    if (has_dims[hc]) {
      double x[4];  // the partials carry the P scale of the input type (a power of two)
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = has ? acc[hc][i] / L * (1.0 / p_scale<DT>()) : 0.0;
      *reinterpret_cast<uint2*>(out + th * D + dcol[hc]) = pack4_from_f64<DT>(x[0], x[1], x[2], x[3]);
      if (o32)
        *reinterpret_cast<float4*>(o32 + th * D + dcol[hc]) =
            make_float4(static_cast<float>(x[0]), static_cast<float>(x[1]), static_cast<float>(x[2]),
                        static_cast<float>(x[3]));
    }
  }
  if (sub == 0) {
    // row_state keeps the base-2 lse (the backward's p = 2^(x - lse2) is then exactly
    // 1 for a row whose only visible key attains it); the public lse is natural.
    const double lse2 = has ? static_cast<double>(M) + log2(L) : -__builtin_inf();
    lse[th] = static_cast<float>(lse2 * kLn2);
    if (row_state) {
      // slot 1: the mass sum_j 2^(x_j - float(lse2)) in closed form, 2^(lse2 - float(lse2)),
      // so that the backward's p = 2^(x - float(lse2)) / mass is normalised exactly; its
      // sign marks the row: negative when its largest probability 1 / L exceeds
      // 1 / kFlatRowMass (peaked). The backward takes delta = O . dO (FP32 output) for the
      // positive (flat) rows; the peaked ones take the reference's centred statistics
      // pass, whose delta shares the rounding of the dP values of dS (the error of the
      // dominant key's dP then cancels in dS).
      row_state[th * 4] = lse2;
      const double mass = has ? exp2(lse2 - static_cast<double>(static_cast<float>(lse2))) : 1.0;
      row_state[th * 4 + 1] = has && L < kFlatRowMass ? -mass : mass;
    }
  }
}

// ---------------------------------------------------------------------------- host side

bool attn_mfma_supported(int64_t ratio, int64_t head_dim, int64_t block_size) {
  return ratio >= 1 && ratio <= kItemRows && head_dim >= 8 && head_dim <= 256 && head_dim % 8 == 0 &&
         block_size >= 1 && block_size <= 128;
}

static int nk_of_dim(int D) { return D <= 32 ? 1 : (D <= 64 ? 2 : (D <= 128 ? 4 : 8)); }

static int64_t fwd_epi(int64_t R) {
  const int64_t e = static_cast<int64_t>(kRowsPerTile) * kTilesPerItem / R;
  return e < 1 ? 1 : e;
}

namespace {
std::atomic<int64_t> g_chunk_budget[3] = {{0}, {0}, {0}};
std::atomic<int> g_item_order{1};
}  // namespace

int64_t kv_chunk_budget(KvPass pass, int64_t dflt) {
  const int64_t b = g_chunk_budget[pass].load(std::memory_order_relaxed);
  return b > 0 ? b : dflt;
}

int64_t kv_chunk_tokens(int64_t T, int64_t Hq, int64_t K, int64_t record_bytes, int64_t budget) {
  const int64_t per_token = Hq * (K > 0 ? K : 1) * record_bytes;
  int64_t tc = budget / (per_token > 0 ? per_token : 1);
  if (tc < 64) tc = 64;
  if (T <= tc) return T > 0 ? T : 1;
  const int64_t nch = (T + tc - 1) / tc;  // balanced chunks
  return (T + nch - 1) / nch;
}

KvPlan kv_plan_layout(int64_t T, int64_t rows, int64_t G, int64_t K, int64_t tc, int64_t epi) {
  KvPlan p;
  p.rows = rows;
  p.tc = tc;
  p.nch = (T + tc - 1) / tc;
  p.epi = epi;
  // one item per row plus one per epi edges of the chunk (a chunk holds <= tc * G * K edges)
  p.max_items = rows + (tc * G * K) / epi + 1;
  p.bounds = 0;
  p.starts = align256((p.nch + 1) * rows * 4);
  p.items = p.starts + align256(p.nch * (rows + 1) * 4);
  p.order = p.items + align256(p.nch * p.max_items * 8);
  p.bytes = p.order + align256(p.nch * p.max_items * 4);
  return p;
}

void kv_plan_launch(const KvPlan& p, const int32_t* row_ptr, const int32_t* qidx, int64_t T, void* base,
                    hipStream_t st, bool ordered) {
  if (p.rows <= 0) return;
  char* b = static_cast<char*>(base);
  int32_t* bounds = reinterpret_cast<int32_t*>(b + p.bounds);
  hipLaunchKernelGGL(kv_chunk_bounds, dim3(grid_1d(p.rows, 4)), dim3(256), 0, st, row_ptr, qidx, p.rows, T, p.tc,
                     static_cast<int>(p.nch), bounds);
  hipLaunchKernelGGL(kv_item_scan, dim3(static_cast<unsigned>(p.nch)), dim3(1024), 0, st, bounds, p.rows,
                     static_cast<int>(p.epi), p.max_items, reinterpret_cast<int32_t*>(b + p.starts),
                     reinterpret_cast<int2*>(b + p.items));
  if (ordered)
    hipLaunchKernelGGL(kv_item_order, dim3(static_cast<unsigned>(p.nch)), dim3(1024), 0, st, bounds, p.rows,
                       static_cast<int>(p.epi), p.max_items, reinterpret_cast<const int32_t*>(b + p.starts),
                       reinterpret_cast<const int2*>(b + p.items), reinterpret_cast<int32_t*>(b + p.order),
                       g_item_order.load(std::memory_order_relaxed) ? 0 : 1);
}

struct FwdLayout {
  KvPlan plan;
  int64_t opart, ml, total;
};

static FwdLayout fwd_layout(int64_t T, int64_t Hq, int64_t G, int64_t D, int64_t K, int64_t total_blocks) {
  FwdLayout f;
  const int64_t tc = kv_chunk_tokens(T, Hq, K, (D + 2) * 4, kv_chunk_budget(kPassFwd, int64_t(2) << 30));
  f.plan = kv_plan_layout(T, total_blocks * G, G, K, tc, fwd_epi(Hq / (G > 0 ? G : 1)));
  f.opart = f.plan.bytes;
  f.ml = f.opart + align256(tc * Hq * K * D * 4);
  f.total = f.ml + align256(tc * Hq * K * 8);
  return f;
}

int64_t attn_fwd_kv_workspace_bytes(int64_t T, int64_t Hq, int64_t G, int64_t D, int64_t K, int64_t total_blocks) {
  return fwd_layout(T, Hq, G, D, K, total_blocks).total;
}

int attn_fwd_kv(int dt, const void* q, const void* k, const void* v, const int32_t* indices, const int32_t* cu,
                int nseq, int64_t T, int Hq, int G, int D, int K, int B, float scale, const int32_t* cu_blocks,
                int64_t total_blocks, const int32_t* row_ptr, const int32_t* qidx, const int32_t* sidx, void* ws,
                int64_t ws_bytes, void* out, float* lse, double* rs, float* o32, hipStream_t st) {
  if (dt != kBF16 && dt != kF16) return kErrInvalidArgument;
  const int64_t rows = total_blocks * G;
  const FwdLayout f = fwd_layout(T, Hq, G, D, K, total_blocks);
  if (ws_bytes < f.total) return kErrInvalidArgument;
  if (!kv_csr_fits(T, G, K, rows) || !kv_chunk_records_fit(f.plan.tc, Hq, K)) return kErrUnsupported;
  if (T == 0) return kOk;
  char* base = static_cast<char*>(ws);
  float* opart = reinterpret_cast<float*>(base + f.opart);
  float2* ml = reinterpret_cast<float2*>(base + f.ml);
  const KvPlan& pl = f.plan;
  const int epi = static_cast<int>(pl.epi);
  const float scale2 = scale * kLog2e;
  const auto* qb = static_cast<const uint16_t*>(q);
  const auto* kb = static_cast<const uint16_t*>(k);
  const auto* vb = static_cast<const uint16_t*>(v);
  auto* ob = static_cast<uint16_t*>(out);
  {
    ProfScope ps(kProfFwdPlan, st);
    kv_plan_launch(pl, row_ptr, qidx, T, base, st);
  }
  for (int64_t c = 0; c < pl.nch; ++c) {
    const int64_t t0 = c * pl.tc, t1 = t0 + pl.tc < T ? t0 + pl.tc : T;
    if (rows > 0) {
      ProfScope ps(kProfFwdPartial, st);
      const dim3 grid(static_cast<unsigned>(pl.max_items));
      const int32_t* hi = kv_plan_hi(pl, base, c);
      const int32_t* nit = kv_plan_count(pl, base, c);
      const int2* its = kv_plan_items(pl, base, c);
      const int32_t* ord = kv_plan_order(pl, base, c);
      const int it0 = static_cast<int>(t0);
#define MSA_FWD_PARTIAL(DTV, NKV, FD) hipLaunchKernelGGL((attn_fwd_partial_kernel<DTV, NKV, FD>), grid, dim3(FwdShape<NKV>::kThreads), 0, st, qb, kb, vb, cu, cu_blocks, qidx, sidx, hi, nit, its, ord, nseq, Hq, G, D, K, B, scale2, epi, it0, opart, ml)
#define MSA_FWD_PARTIAL_NK(DTV)                                                                   \
  if (nk == 1) { if (fd) MSA_FWD_PARTIAL(DTV, 1, true); else MSA_FWD_PARTIAL(DTV, 1, false); }       \
  else if (nk == 2) { if (fd) MSA_FWD_PARTIAL(DTV, 2, true); else MSA_FWD_PARTIAL(DTV, 2, false); }  \
  else if (nk == 4) { if (fd) MSA_FWD_PARTIAL(DTV, 4, true); else MSA_FWD_PARTIAL(DTV, 4, false); }  \
  else { if (fd) MSA_FWD_PARTIAL(DTV, 8, true); else MSA_FWD_PARTIAL(DTV, 8, false); }
      const int nk = nk_of_dim(D);
      const bool fd = D == 32 * nk;
      if (dt == kF16) { MSA_FWD_PARTIAL_NK(kF16) } else { MSA_FWD_PARTIAL_NK(kBF16) }
#undef MSA_FWD_PARTIAL_NK
#undef MSA_FWD_PARTIAL
    }
    ProfScope ps(kProfFwdCombine, st);
    const dim3 cgrid(grid_1d((t1 - t0) * Hq, 8));
#define MSA_FWD_COMBINE(DTV, DCV)                                                                               \
  hipLaunchKernelGGL((attn_fwd_combine<DTV, DCV>), cgrid, dim3(256), 0, st, indices, cu, nseq, t0, t1, Hq, G, D, K, B, \
                     opart, ml, ob, lse, rs, o32)
    if (dt == kF16) { if (D > 128) MSA_FWD_COMBINE(kF16, 2); else MSA_FWD_COMBINE(kF16, 1); }
    else { if (D > 128) MSA_FWD_COMBINE(kBF16, 2); else MSA_FWD_COMBINE(kBF16, 1); }
#undef MSA_FWD_COMBINE
  }
  return status_from(hipGetLastError());
}

}  // namespace msa

extern "C" int msa_set_item_order(int enabled) {
  msa::g_item_order.store(enabled != 0 ? 1 : 0, std::memory_order_relaxed);
  return msa::kOk;
}

extern "C" int msa_set_chunk_budgets(int64_t fwd_bytes, int64_t bwd_bytes, int64_t kl_bytes) {
  msa::g_chunk_budget[msa::kPassFwd].store(fwd_bytes > 0 ? fwd_bytes : 0, std::memory_order_relaxed);
  msa::g_chunk_budget[msa::kPassBwd].store(bwd_bytes > 0 ? bwd_bytes : 0, std::memory_order_relaxed);
  msa::g_chunk_budget[msa::kPassKl].store(kl_bytes > 0 ? kl_bytes : 0, std::memory_order_relaxed);
  return msa::kOk;
}
