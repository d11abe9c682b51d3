// Causal top-k selection of one (token, group) row, by sixteen lanes (one DPP row)
// or by a whole wavefront, and the host launch that picks between them.
//
// Semantics follow triton/topk.py:31-46 (eager twin eager/ops.py:94-129): blocks
// b > qb(t) are masked to -inf, blocks in (qb-L, qb] are forced to +inf, the
// min(K, NB) largest are returned in descending order, -inf picks become -1, and
// the row is right-padded with -1 up to K slots. NaN scores rank above +inf (as in
// torch.topk). Ties (equal values, e.g. several +inf local blocks, or NaNs) are
// emitted in ascending block order.
#pragma once
#include "common.hpp"

namespace msa {

// Monotone map of float bits onto uint32 (+0 and -0 collapse to the same key). NaN of
// either sign ranks above +inf, as in torch.topk (the reference's selection,
// triton/topk.py:44-45); 0xfffffffe keeps the 64-bit key of block 0 below the scan's
// initial bound ~0.
__device__ __forceinline__ uint32_t ordered_key(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0xfffffffeu;
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

constexpr uint32_t kKeyNegInf = 0x007fffffu;  // ordered_key(-inf)
constexpr uint32_t kKeyPosInf = 0xff800000u;  // ordered_key(+inf)

// 64-bit max over the 16 lanes of a DPP row (every lane of the row receives it):
// quad butterflies, then half-row and row mirrors pair disjoint groups.
__device__ __forceinline__ uint64_t row16_max_u64(uint64_t v) {
#define MSA_DPP_MAX(CTRL)                                                                         \
  {                                                                                               \
    const uint32_t lo = static_cast<uint32_t>(v), hi = static_cast<uint32_t>(v >> 32);            \
    const uint32_t olo = __builtin_amdgcn_update_dpp(0u, lo, CTRL, 0xF, 0xF, false);              \
    const uint32_t ohi = __builtin_amdgcn_update_dpp(0u, hi, CTRL, 0xF, 0xF, false);              \
    const uint64_t o = (static_cast<uint64_t>(ohi) << 32) | olo;                                  \
    v = o > v ? o : v;                                                                            \
  }
  MSA_DPP_MAX(0xB1)   // quad_perm [1, 0, 3, 2]
  MSA_DPP_MAX(0x4E)   // quad_perm [2, 3, 0, 1]
  MSA_DPP_MAX(0x141)  // row_half_mirror
  MSA_DPP_MAX(0x140)  // row_mirror
#undef MSA_DPP_MAX
  return v;
}

// A lane's sorted cache of its N largest keys below a bound (0 = empty slot):
// c[0] > c[1] > ... > c[N - 1]. Keys are unique (the block id is in the low word).
template <int N>
struct TopN {
  uint64_t c[N];
  __device__ __forceinline__ void insert(uint64_t x) {
    // x enters at the bottom when it beats the smallest entry, then bubbles up
    if (x > c[N - 1]) c[N - 1] = x;
#pragma unroll
    for (int i = N - 1; i > 0; --i) {
      const uint64_t hi = c[i] > c[i - 1] ? c[i] : c[i - 1];
      const uint64_t lo = c[i] > c[i - 1] ? c[i - 1] : c[i];
      c[i - 1] = hi;
      c[i] = lo;
    }
  }
  template <int VPL>
  __device__ __forceinline__ void fill(const uint64_t (&key)[VPL], uint64_t below) {
#pragma unroll
    for (int i = 0; i < N; ++i) c[i] = 0;
#pragma unroll
    for (int v = 0; v < VPL; ++v)
      if (key[v] < below) insert(key[v]);
  }
  __device__ __forceinline__ void pop() {
#pragma unroll
    for (int i = 0; i + 1 < N; ++i) c[i] = c[i + 1];
    c[N - 1] = 0;
  }
};

// Sixteen lanes (one DPP row) per (token, group) row, four rows per wavefront: lane
// j of a row holds blocks j, j + 16, ... (VPL values). Each pick is a 16-lane DPP
// max of the lanes' best remaining keys. A lane keeps its largest remaining keys
// sorted (TopN: 4 for up to 16 values per lane, 8 above, where a lane more often
// holds several winners); the owner of a pick pops it and refills from its values below the
// popped key only once its cache is empty. The picks are those of a full rescan
// after every pick: the cache always holds the lane's largest keys below its last
// popped one.
// Every lane of the wavefront must call it (row >= rows: no output, but the lanes
// still take part in the DPP and shuffle steps). The selection key is the ordered
// float bits << 32 | ~block, so one 64-bit comparison implements "larger value,
// then smaller block id".
template <int VPL>
__device__ __forceinline__ void topk_row16(const float* __restrict__ scores, const int32_t* __restrict__ cu,
                                           int nseq, int64_t rows, int G, int NB, int B, int K, int L,
                                           int32_t* __restrict__ out, int64_t row, int sub) {
  const bool live = row < rows;
  const int64_t rr = live ? row : rows - 1;
  const int64_t t = rr / G;
  const int s = find_seq(cu, nseq, t);
  const int64_t qb = (t - cu[s]) / B;
  const int n = static_cast<int>(qb + 1 < NB ? qb + 1 : NB);
  const int count = K < NB ? K : NB;
  const int sel = live ? (count < n ? count : n) : 0;
  const float* src = scores + rr * NB;
  int32_t* dst = out + rr * K;

  uint64_t key[VPL];
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    const int b = v * 16 + sub;
    uint32_t k = 0u;  // below every real key: never selected
    if (b < n) {
      k = (L > 0 && b > qb - L) ? kKeyPosInf : ordered_key(src[b]);
    }
    key[v] = (static_cast<uint64_t>(k) << 32) | static_cast<uint32_t>(~static_cast<uint32_t>(b));
  }
  TopN<(VPL > 16 ? 8 : 4)> top;
  top.fill(key, ~uint64_t(0));

  // every row of the wave runs the same number of picks (the wave maximum)
  int sel_w = sel;
#pragma unroll
  for (int o = 16; o < 64; o <<= 1) sel_w = max(sel_w, __shfl_xor(sel_w, o, kWave));
  for (int it = 0; it < sel_w; ++it) {
    const uint64_t win = row16_max_u64(top.c[0]);
    const int b = static_cast<int>(~static_cast<uint32_t>(win));
    const uint32_t k = static_cast<uint32_t>(win >> 32);
    if (sub == 0 && it < sel) dst[it] = (k == kKeyNegInf) ? -1 : b;
    if ((b & 15) == sub && it < sel) {  // win == top.c[0] of this lane
      top.pop();
      if (top.c[0] == 0) top.fill(key, win);
    }
  }
  if (live)
    for (int it = sel + sub; it < K; it += 16) dst[it] = -1;
}

// Host launch of the stand-alone selection (topk.hip): 16-lane rows up to 1024
// blocks, one wavefront per row with the row in registers up to 4096, streamed above.
int topk_launch(const float* scores, const int32_t* cu_seqlens, int nseq, int64_t rows, int G, int NB, int B, int K,
                int L, int32_t* indices, hipStream_t st);

// One wavefront per row: lane j holds blocks j, j + 64, ... (VPL values); each pick
// is a 64-lane max. All lanes of the wavefront call it for the same row.
template <int VPL>
__device__ __forceinline__ void topk_row64(const float* __restrict__ scores, const int32_t* __restrict__ cu,
                                           int nseq, int G, int NB, int B, int K, int L,
                                           int32_t* __restrict__ out, int64_t row, int lane) {
  const int64_t t = row / G;
  const int s = find_seq(cu, nseq, t);
  const int64_t qb = (t - cu[s]) / B;
  const int n = static_cast<int>(qb + 1 < NB ? qb + 1 : NB);
  const int count = K < NB ? K : NB;
  const int sel = count < n ? count : n;
  const float* src = scores + row * NB;
  int32_t* dst = out + row * K;
  uint64_t key[VPL];
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    const int b = v * kWave + lane;
    uint32_t k = 0u;
    if (b < n) k = (L > 0 && b > qb - L) ? kKeyPosInf : ordered_key(src[b]);
    key[v] = (static_cast<uint64_t>(k) << 32) | static_cast<uint32_t>(~static_cast<uint32_t>(b));
  }
  uint64_t best = 0;
#pragma unroll
  for (int v = 0; v < VPL; ++v) best = key[v] > best ? key[v] : best;
  for (int it = 0; it < sel; ++it) {
    const uint64_t win = wave_max_u64(best);
    const int b = static_cast<int>(~static_cast<uint32_t>(win));
    const uint32_t k = static_cast<uint32_t>(win >> 32);
    if (lane == 0) dst[it] = (k == kKeyNegInf) ? -1 : b;
    if ((b & 63) == lane) {
      best = 0;
#pragma unroll
      for (int v = 0; v < VPL; ++v) {
        if (key[v] == win) key[v] = 0;
        best = key[v] > best ? key[v] : best;
      }
    }
  }
  for (int it = sel + lane; it < K; it += kWave) dst[it] = -1;
}

// One wavefront per row with the row left in memory, for any number of blocks (used
// above 4096): lane j scans blocks j, j + 64, ... and keeps its eight largest keys
// below its last pick (TopN<8>); it rescans its blocks only when that cache runs empty,
// so a row is read about once. Picks, order and padding are those of topk_row64.
__device__ __forceinline__ void topk_row_stream(const float* __restrict__ scores, const int32_t* __restrict__ cu,
                                                int nseq, int G, int NB, int B, int K, int L,
                                                int32_t* __restrict__ out, int64_t row, int lane) {
  const int64_t t = row / G;
  const int s = find_seq(cu, nseq, t);
  const int64_t qb = (t - cu[s]) / B;
  const int n = static_cast<int>(qb + 1 < NB ? qb + 1 : NB);
  const int count = K < NB ? K : NB;
  const int sel = count < n ? count : n;
  const float* src = scores + row * NB;
  int32_t* dst = out + row * static_cast<int64_t>(K);
  TopN<8> top;
  auto fill = [&](uint64_t below) {
#pragma unroll
    for (int i = 0; i < 8; ++i) top.c[i] = 0;
    for (int b = lane; b < n; b += kWave) {
      const uint32_t k = (L > 0 && b > qb - L) ? kKeyPosInf : ordered_key(src[b]);
      const uint64_t x = (static_cast<uint64_t>(k) << 32) | static_cast<uint32_t>(~static_cast<uint32_t>(b));
      if (x < below) top.insert(x);
    }
  };
  fill(~uint64_t(0));
  for (int it = 0; it < sel; ++it) {
    const uint64_t win = wave_max_u64(top.c[0]);
    const int b = static_cast<int>(~static_cast<uint32_t>(win));
    const uint32_t k = static_cast<uint32_t>(win >> 32);
    if (lane == 0) dst[it] = (k == kKeyNegInf) ? -1 : b;
    if ((b & 63) == lane) {  // win == top.c[0] of this lane
      top.pop();
      if (top.c[0] == 0) fill(win);
    }
  }
  for (int it = sel + lane; it < K; it += kWave) dst[it] = -1;
}

}  // namespace msa
