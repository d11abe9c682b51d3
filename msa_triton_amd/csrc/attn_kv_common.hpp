// Shared pieces of the KV-major stage-3 kernels (bf16 and fp16 MFMA paths).
//
// The k2q CSR has one row per (key block, group); its edges are the (query
// token, slot) pairs that selected the block, ordered by query token. KV-major
// passes walk the edges of a row with the row's K/V block resident on chip.
// Query tokens are cut into chunks of tc tokens so that per-(token, head, slot)
// partial buffers stay bounded; within a row, the edges of one chunk form a
// contiguous range. A plan lists, per chunk, work items (row, first edge) of at
// most `epi` edges each.
#pragma once
#include "attn_mfma.hpp"
#include "mfma_util.hpp"

namespace msa {

constexpr float kLog2e = 1.4426950408889634f;
constexpr double kLn2 = 0.6931471805599453;

// fp16 kernels split probabilities P <= 1 into fp16 terms after scaling them by 2^15 (the
// top binade of fp16, so that the split is exact down to P = 2^-16 and within 2^-40 of P
// below); the products they feed carry the factor, which is divided out exactly later.
constexpr float kPScaleF16 = 32768.f;
template <int DT>
constexpr double p_scale() { return DT == kF16 ? 32768.0 : 1.0; }

// Two 8-byte reads of tile[row][base + pi(q4, j)] where pi(q4, j) = 16*(j/4) + 4*q4 + j%4.
__device__ __forceinline__ bf16x8 read_keys_pi(const uint16_t* tile, int stride, int row, int base, int q4) {
  const uint16_t* p = tile + row * stride + base + 4 * q4;
  const uint2 a = *reinterpret_cast<const uint2*>(p);
  const uint2 b = *reinterpret_cast<const uint2*>(p + 16);
  return __builtin_bit_cast(bf16x8, make_uint4(a.x, a.y, b.x, b.y));
}

struct RowGeom {
  int64_t kb;  // first key of the block
  int nk;      // keys in the block
  int g;
};

// Geometry of CSR row (global block gb = row / G, group row % G).
__device__ __forceinline__ RowGeom row_geom(const int32_t* __restrict__ cu, const int32_t* __restrict__ cu_blocks,
                                            int nseq, int64_t row, int G, int B) {
  const int64_t gb = row / G;
  int s = upper_index(cu_blocks, nseq + 1, gb);
  while (s < nseq && cu_blocks[s + 1] <= gb) ++s;
  RowGeom r;
  r.g = static_cast<int>(row % G);
  r.kb = cu[s] + (gb - cu_blocks[s]) * B;
  const int64_t end = cu[s + 1];
  r.nk = static_cast<int>(end - r.kb < B ? end - r.kb : B);
  return r;
}

inline int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

// x / r for 0 <= x with x * r < 2^32 (the row -> edge split inside a work item) as a
// multiply-high by magic = ceil(2^32 / r): with 2^32 = magic * r - e, 0 <= e < r, the
// error term x * e / (r * 2^32) stays below 1 / r, so the floor is exact. r == 1 is
// passed as magic 0.
__device__ __forceinline__ int div_by_ratio(int x, uint32_t magic) {
  return magic ? static_cast<int>(__umulhi(static_cast<uint32_t>(x), magic)) : x;
}
inline uint32_t ratio_magic(int64_t r) {
  return r <= 1 ? 0u : static_cast<uint32_t>(((int64_t(1) << 32) + r - 1) / r);
}

// Query tokens per chunk: per-(token, head, slot) records of `record_bytes` each
// within `budget` bytes, chunks of equal size. Measured at c4 (T = 32768): the forward
// partial pass runs best with ~2 GiB chunks (5 chunks; 1 GiB: +1.5 %), the backward with
// ~6 GiB (2 chunks; 4 GiB: +2 %, fewer per-chunk key-block reloads and item tails); the
// backward's 32-bit dQ record offsets bound its budget below 8 GiB.
int64_t kv_chunk_tokens(int64_t T, int64_t Hq, int64_t K, int64_t record_bytes, int64_t budget);

// Chunk budgets of the KV-major passes: `dflt` unless msa_set_chunk_budgets set one.
enum KvPass { kPassFwd = 0, kPassBwd = 1, kPassKl = 2 };
int64_t kv_chunk_budget(KvPass pass, int64_t dflt);

// Chunk-local record index of (token t0 + tl, head, slot): ((tl * K + slot) * heads + head).
// The heads of one (token, slot) are adjacent, so the rows of one CSR edge (the heads
// of its group) write one contiguous run of records and of (m, l) pairs.
__device__ __forceinline__ int64_t kv_record(int64_t tl, int head, int slot, int heads, int K) {
  return (tl * K + slot) * heads + head;
}

// Chunk-local record indices are int32: a chunk may hold at most 2^31 - 1 records
// (with the default budgets it holds far fewer).
inline bool kv_chunk_records_fit(int64_t tc, int64_t heads, int64_t K) {
  return tc * heads * (K > 0 ? K : 1) < (int64_t(1) << 31);
}

// The capacity limit of the KV-major kernels is the k2q CSR's (triton/k2q.py:65-69):
// T * G * K edges and the (block, group) rows must fit in int32. Token ids, token-head
// indices and element offsets are formed in int64.
inline bool kv_csr_fits(int64_t T, int64_t G, int64_t K, int64_t rows) {
  return T * G * (K > 0 ? K : 1) < (int64_t(1) << 31) && rows < (int64_t(1) << 31);
}

struct KvPlan {
  int64_t rows, tc, nch, epi, max_items;         // max_items: per-chunk upper bound on work items
  int64_t bounds, starts, items, order, bytes;  // byte offsets of the arrays inside the plan area, total size
};

KvPlan kv_plan_layout(int64_t T, int64_t rows, int64_t G, int64_t K, int64_t tc, int64_t epi);

// Fills bounds[(nch + 1) x rows], starts[nch x (rows + 1)] and items[nch x max_items]
// (int2: row, first edge) in the plan area at `base`, and with `ordered` also
// order[nch x max_items] (per chunk, the item indices largest first: the dispatch order
// of the KV-major kernels; a kernel given no order takes the items in row order).
void kv_plan_launch(const KvPlan& p, const int32_t* row_ptr, const int32_t* qidx, int64_t T, void* base,
                    hipStream_t st, bool ordered = true);

// Per chunk views of a launched plan.
inline const int32_t* kv_plan_hi(const KvPlan& p, const void* base, int64_t c) {
  return reinterpret_cast<const int32_t*>(static_cast<const char*>(base) + p.bounds) + (c + 1) * p.rows;
}
inline const int32_t* kv_plan_lo(const KvPlan& p, const void* base, int64_t c) {
  return reinterpret_cast<const int32_t*>(static_cast<const char*>(base) + p.bounds) + c * p.rows;
}
inline const int32_t* kv_plan_count(const KvPlan& p, const void* base, int64_t c) {
  return reinterpret_cast<const int32_t*>(static_cast<const char*>(base) + p.starts) + c * (p.rows + 1) + p.rows;
}
inline const int32_t* kv_plan_starts(const KvPlan& p, const void* base, int64_t c) {
  return reinterpret_cast<const int32_t*>(static_cast<const char*>(base) + p.starts) + c * (p.rows + 1);
}
inline const int2* kv_plan_items(const KvPlan& p, const void* base, int64_t c) {
  return reinterpret_cast<const int2*>(static_cast<const char*>(base) + p.items) + c * p.max_items;
}
inline const int32_t* kv_plan_order(const KvPlan& p, const void* base, int64_t c) {
  return reinterpret_cast<const int32_t*>(static_cast<const char*>(base) + p.order) + c * p.max_items;
}

}  // namespace msa
