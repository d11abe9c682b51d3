// Deterministic block->query CSR ("k2q") for the KV-owned backward.
//
// Semantics follow triton/k2q.py:94-128 (K2QCSR at :20-36):
//   edge (t, g, s) with id = indices[t,g,s] is valid iff 0 <= id < nb(seq) and
//   id <= qb(t); its row is (cu_block_lens[seq] + id) * G + g; row_ptr is the
//   exclusive prefix of the row counts; inside a row edges are ordered by
//   (query token, slot) ascending; unused tail entries are -1.
//
// Instead of the reference's argsort over int64 keys this is a stable counting
// sort whose tiles are the query blocks themselves: every token of query block
// qb can only reach rows with block id <= qb, so tile (seq, qb) owns a compact
// counter range of (qb+1)*G entries.
//   1. k2q_count   : per-tile histogram of its edges (integer atomics -> exact),
//                    in LDS when the tile's counters fit.
//   2. k2q_rowscan : per row, exclusive prefix of the counts over the tiles
//                    qb >= b (in qb order), giving the tile's start inside the row;
//                    one wavefront per row, 64 tiles per step.
//   3. k2q_ptrscan : exclusive scan of row totals -> row_ptr (one workgroup).
//   4. k2q_scatter_par : per (tile, group), a stable counting sort of the tile's
//                    edges on their block id places each edge at row_ptr[row] +
//                    tile offset + its rank among the tile's edges of that row.
//   5. k2q_tail    : entries at or beyond row_ptr[rows] become -1.
#include <algorithm>
#include <mutex>

#include "common.hpp"
#include "msa_mi355x.h"

namespace msa {

struct TileInfo {
  int seq;
  int qb;
  int64_t tok_begin;
  int64_t tok_end;
  int64_t counter_base;  // offset of this tile's (qb+1)*G counters
};

// tri_prefix[s] = G * sum_{s'<s} nb(s') * (nb(s') + 1) / 2, computed on the host.
__device__ __forceinline__ TileInfo tile_info(int64_t tile, const int32_t* __restrict__ cu,
                                              const int32_t* __restrict__ cu_blocks,
                                              const int64_t* __restrict__ tri_prefix, int nseq, int G,
                                              int B) {
  TileInfo ti;
  ti.seq = upper_index(cu_blocks, nseq + 1, tile);
  // Skip empty sequences that share the same block boundary.
  while (ti.seq < nseq && cu_blocks[ti.seq + 1] <= tile) ++ti.seq;
  ti.qb = static_cast<int>(tile - cu_blocks[ti.seq]);
  const int64_t start = cu[ti.seq];
  const int64_t end = cu[ti.seq + 1];
  ti.tok_begin = start + static_cast<int64_t>(ti.qb) * B;
  ti.tok_end = ti.tok_begin + B < end ? ti.tok_begin + B : end;
  ti.counter_base = tri_prefix[ti.seq] + static_cast<int64_t>(G) * ti.qb * (ti.qb + 1) / 2;
  return ti;
}

// Tiles with at most this many counters ((qb + 1) * G) count in LDS.
constexpr int kCountLds = 8192;

__global__ __launch_bounds__(256) void k2q_count(const int32_t* __restrict__ indices,
                                                 const int32_t* __restrict__ cu,
                                                 const int32_t* __restrict__ cu_blocks,
                                                 const int64_t* __restrict__ tri_prefix, int nseq,
                                                 int G, int K, int B, int32_t* __restrict__ counters) {
  __shared__ int32_t hist[kCountLds];
  const TileInfo ti = tile_info(blockIdx.x, cu, cu_blocks, tri_prefix, nseq, G, B);
  const int64_t ncnt = static_cast<int64_t>(ti.qb + 1) * G;
  const bool in_lds = ncnt <= kCountLds;  // uniform over the workgroup
  int32_t* cnt = counters + ti.counter_base;
  int32_t* h = in_lds ? hist : cnt;
  for (int64_t i = threadIdx.x; i < ncnt; i += blockDim.x) h[i] = 0;
  __syncthreads();
  const int nb = cu_blocks[ti.seq + 1] - cu_blocks[ti.seq];
  // a tile holds at most B tokens: its edge count fits in 32 bits (B * G * K < 2^31 checked on the host)
  const int edges = static_cast<int>((ti.tok_end - ti.tok_begin) * G * K);
  const int32_t* src = indices + ti.tok_begin * G * K;
  for (int e = threadIdx.x; e < edges; e += blockDim.x) {
    const int id = src[e];
    const int g = (e / K) % G;
    if (id >= 0 && id < nb && id <= ti.qb) {
      if (in_lds)
        atomicAdd(&hist[id * G + g], 1);
      else
        atomicAdd(&cnt[static_cast<int64_t>(id) * G + g], 1);
    }
  }
  if (in_lds) {
    __syncthreads();
    for (int i = threadIdx.x; i < static_cast<int>(ncnt); i += blockDim.x) cnt[i] = hist[i];
  }
}

// One wavefront per row: rewrite the row's per-tile counts into exclusive offsets
// (in tile order, 64 tiles per step with a wave prefix sum) and emit the row total.
__global__ __launch_bounds__(256) void k2q_rowscan(const int32_t* __restrict__ cu_blocks,
                                                   const int64_t* __restrict__ tri_prefix, int nseq,
                                                   int G, int64_t rows, int32_t* __restrict__ counters,
                                                   int32_t* __restrict__ totals) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;  // whole wavefronts
  const int64_t gb = r / G;
  const int g = static_cast<int>(r % G);
  int s = upper_index(cu_blocks, nseq + 1, gb);
  while (s < nseq && cu_blocks[s + 1] <= gb) ++s;
  const int b = static_cast<int>(gb - cu_blocks[s]);
  const int nb = cu_blocks[s + 1] - cu_blocks[s];
  int32_t carry = 0;
  for (int q0 = b; q0 < nb; q0 += kWave) {  // trip count uniform over the wavefront
    const int qb = q0 + lane;
    int64_t idx = 0;
    int32_t c = 0;
    if (qb < nb) {
      idx = tri_prefix[s] + static_cast<int64_t>(G) * qb * (qb + 1) / 2 + static_cast<int64_t>(b) * G + g;
      c = counters[idx];
    }
    int32_t x = c;  // inclusive prefix over the lanes
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const int32_t y = __shfl_up(x, o, kWave);
      if (lane >= o) x += y;
    }
    if (qb < nb) counters[idx] = carry + x - c;
    carry += __shfl(x, kWave - 1, kWave);
  }
  if (lane == 0) totals[r] = carry;
}

// Exclusive scan of totals[0..rows) into row_ptr[0..rows], one workgroup of 1024.
__global__ __launch_bounds__(1024) void k2q_ptrscan(const int32_t* __restrict__ totals, int64_t rows,
                                                    int32_t* __restrict__ row_ptr) {
  __shared__ int32_t warp_sums[16];
  __shared__ int32_t carry_s;
  if (threadIdx.x == 0) carry_s = 0;
  __syncthreads();
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  for (int64_t base = 0; base < rows; base += 1024) {
    const int64_t i = base + threadIdx.x;
    const int32_t v = i < rows ? totals[i] : 0;
    // inclusive wave scan
    int32_t x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int32_t y = __shfl_up(x, o, kWave);
      if (lane >= o) x += y;
    }
    if (lane == 63) warp_sums[wid] = x;
    __syncthreads();
    if (threadIdx.x < 16) {
      int32_t w = warp_sums[threadIdx.x];
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) {
        const int32_t y = __shfl_up(w, o, 16);
        if (static_cast<int>(threadIdx.x) >= o) w += y;
      }
      warp_sums[threadIdx.x] = w;  // inclusive over waves
    }
    __syncthreads();
    const int32_t carry = carry_s;
    const int32_t wave_off = wid > 0 ? warp_sums[wid - 1] : 0;
    if (i < rows) row_ptr[i] = carry + wave_off + x - v;
    __syncthreads();
    if (threadIdx.x == 0) carry_s = carry + warp_sums[15];
    __syncthreads();
  }
  if (threadIdx.x == 0) row_ptr[rows] = carry_s;
}

// Parallel scatter. One workgroup per (tile, group) for tiles with at most
// kParIds ids (query blocks below kParIds; later tiles of longer sequences walk
// their edges serially): the tile's edges of that group, taken in (token, slot) order 256
// per step, are placed by a stable counting sort on the block id. Inside a 64-lane
// wave the rank among equal ids comes from one ballot per id bit; waves are merged
// in order through per-wave id counts, and a running count per id carries the
// order across steps. The position is row_ptr[row] + the tile's offset in the row
// (from k2q_rowscan) + that rank, i.e. the same (query, slot) order as the
// sequential scatter, duplicates included. The first two terms are staged in LDS per
// id once, and each step's indices are loaded one step ahead.
constexpr int kParIds = 1024;
constexpr int kParIdBits = 10;

__global__ __launch_bounds__(256) void k2q_scatter_par(const int32_t* __restrict__ indices,
                                                       const int32_t* __restrict__ cu,
                                                       const int32_t* __restrict__ cu_blocks,
                                                       const int64_t* __restrict__ tri_prefix, int nseq, int G,
                                                       int K, int B, const int32_t* __restrict__ row_ptr,
                                                       int32_t* __restrict__ counters,
                                                       int32_t* __restrict__ query_idx,
                                                       int32_t* __restrict__ slot_idx) {
  __shared__ int32_t running[kParIds];
  __shared__ int32_t wcnt[4][kParIds];
  __shared__ int32_t rbase[kParIds];  // row_ptr[row of id] + the tile's offset inside that row
  const TileInfo ti = tile_info(blockIdx.x, cu, cu_blocks, tri_prefix, nseq, G, B);
  const int g = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int nb = cu_blocks[ti.seq + 1] - cu_blocks[ti.seq];
  const int nid = ti.qb + 1;  // ids of this tile: 0 .. qb
  int32_t* cntw = counters + ti.counter_base;
  if (nid > kParIds) {
    // more ids than the LDS counters hold: one thread walks the edges in (token, slot)
    // order, advancing the tile's offsets of this group's rows in place
    if (tid == 0) {
      const int64_t rb = static_cast<int64_t>(cu_blocks[ti.seq]) * G;
      for (int64_t t = ti.tok_begin; t < ti.tok_end; ++t)
        for (int slot = 0; slot < K; ++slot) {
          const int v = indices[(t * G + g) * K + slot];
          if (v < 0 || v >= nb || v > ti.qb) continue;
          const int64_t lr = static_cast<int64_t>(v) * G + g;
          const int64_t pos = static_cast<int64_t>(row_ptr[rb + lr]) + cntw[lr]++;
          query_idx[pos] = static_cast<int32_t>(t);
          slot_idx[pos] = slot;
        }
    }
    return;
  }
  const int32_t* cnt = counters + ti.counter_base;  // the tile's offset inside each row
  const int64_t row_base = static_cast<int64_t>(cu_blocks[ti.seq]) * G;
  for (int i = tid; i < nid; i += 256) {
    running[i] = 0;
    wcnt[0][i] = wcnt[1][i] = wcnt[2][i] = wcnt[3][i] = 0;
    const int64_t lr = static_cast<int64_t>(i) * G + g;
    rbase[i] = row_ptr[row_base + lr] + cnt[lr];
  }
  __syncthreads();
  // a tile holds at most B tokens: B * K < 2^31 edges (checked on the host)
  const int nedge = static_cast<int>((ti.tok_end - ti.tok_begin) * K);
  const uint64_t lt = (uint64_t(1) << lane) - 1;
  auto load_id = [&](int e) {
    int v = -1;
    if (e < nedge) v = indices[((ti.tok_begin + e / K) * G + g) * K + e % K];
    return v;
  };
  int vnext = load_id(tid);
  for (int base = 0; base < nedge; base += 256) {
    const int e = base + tid;
    const int v = vnext;
    vnext = load_id(e + 256);  // next step's index, in flight during this one
    const int64_t t = ti.tok_begin + e / K;
    const int slot = e % K;
    const int id = (e < nedge && v >= 0 && v < nb && v <= ti.qb) ? v : -1;
    const bool on = id >= 0;
    uint64_t match = __ballot(on);
#pragma unroll
    for (int bit = 0; bit < kParIdBits; ++bit) {
      const uint64_t m = __ballot(on && ((id >> bit) & 1));
      match &= ((id >> bit) & 1) ? m : ~m;
    }
    const int rank = __popcll(match & lt);
    const int total = __popcll(match);
    if (on && rank == total - 1) wcnt[wid][id] = total;
    __syncthreads();
    if (on) {
      int before = running[id] + rank;
      for (int w2 = 0; w2 < wid; ++w2) before += wcnt[w2][id];
      const int64_t pos = static_cast<int64_t>(rbase[id]) + before;
      query_idx[pos] = static_cast<int32_t>(t);
      slot_idx[pos] = slot;
    }
    __syncthreads();
    for (int i = tid; i < nid; i += 256) {
      running[i] += wcnt[0][i] + wcnt[1][i] + wcnt[2][i] + wcnt[3][i];
      wcnt[0][i] = wcnt[1][i] = wcnt[2][i] = wcnt[3][i] = 0;
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(256) void k2q_tail(const int32_t* __restrict__ row_ptr, int64_t rows,
                                                int64_t capacity, int32_t* __restrict__ query_idx,
                                                int32_t* __restrict__ slot_idx) {
  const int64_t used = row_ptr[rows];
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x + used; i < capacity;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    query_idx[i] = -1;
    slot_idx[i] = -1;
  }
}

__global__ __launch_bounds__(256) void fill_i32(int32_t* __restrict__ dst, int64_t n, int32_t value) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    dst[i] = value;
}

inline unsigned capped_grid(int64_t n) {
  unsigned g = grid_1d(n, 256);
  return g > 65535u * 16u ? 65535u * 16u : g;
}

}  // namespace msa

using namespace msa;

// Number of int32 counters the tile histogram needs: G * sum_s nb_s (nb_s + 1) / 2.
extern "C" int64_t msa_k2q_counter_elems(int64_t num_seqs, const int32_t* host_cu_block_lens,
                                         int64_t groups) {
  int64_t counters = 0;
  for (int64_t s = 0; s < num_seqs; ++s) {
    const int64_t nb = host_cu_block_lens[s + 1] - host_cu_block_lens[s];
    counters += groups * nb * (nb + 1) / 2;
  }
  return counters;
}

namespace msa {

namespace {

// The five launches of the build over a caller-provided int32 workspace of
// counter_elems + total_blocks * groups entries (the tile histograms are cleared by
// k2q_count itself and the row totals are written before they are read, so the
// workspace may hold anything on entry).
int k2q_build_launch(const int32_t* indices, const int32_t* cu_seqlens, const int32_t* cu_block_lens,
                     const int64_t* tri_prefix, int64_t num_seqs, int64_t total_tokens, int64_t groups,
                     int64_t topk_slots, int64_t block_size, int64_t total_blocks, int64_t counter_elems,
                     int32_t* row_ptr, int32_t* query_indices, int32_t* slot_indices, int32_t* workspace,
                     hipStream_t st) {
  const int64_t rows = total_blocks * groups;
  const int64_t capacity = total_tokens * groups * topk_slots;
  if (capacity == 0 || rows == 0) {
    hipLaunchKernelGGL(fill_i32, dim3(capped_grid(rows + 1)), dim3(256), 0, st, row_ptr, rows + 1, 0);
    return status_from(hipGetLastError());
  }
  int32_t* counters = workspace;
  int32_t* totals = workspace + counter_elems;
  const int nseq = static_cast<int>(num_seqs), G = static_cast<int>(groups);
  const int K = static_cast<int>(topk_slots), B = static_cast<int>(block_size);
  hipLaunchKernelGGL(k2q_count, dim3(static_cast<unsigned>(total_blocks)), dim3(256), 0, st, indices,
                     cu_seqlens, cu_block_lens, tri_prefix, nseq, G, K, B, counters);
  hipLaunchKernelGGL(k2q_rowscan, dim3(grid_1d(rows, 4)), dim3(256), 0, st, cu_block_lens, tri_prefix,
                     nseq, G, rows, counters, totals);
  hipLaunchKernelGGL(k2q_ptrscan, dim3(1), dim3(1024), 0, st, totals, rows, row_ptr);
  hipLaunchKernelGGL(k2q_scatter_par, dim3(static_cast<unsigned>(total_blocks), static_cast<unsigned>(G)),
                     dim3(256), 0, st, indices, cu_seqlens, cu_block_lens, tri_prefix, nseq, G, K, B, row_ptr,
                     counters, query_indices, slot_indices);
  hipLaunchKernelGGL(k2q_tail, dim3(capped_grid(capacity)), dim3(256), 0, st, row_ptr, rows, capacity,
                     query_indices, slot_indices);
  return status_from(hipGetLastError());
}

bool k2q_args_valid(int64_t num_seqs, int64_t total_tokens, int64_t groups, int64_t topk_slots, int64_t block_size,
                    int64_t total_blocks, int64_t counter_elems) {
  return num_seqs > 0 && total_tokens >= 0 && groups > 0 && topk_slots >= 0 && block_size > 0 &&
         total_blocks >= 0 && counter_elems >= 0;
}

// Workspace of msa_k2q_build_noalloc: a fixed device array, one copy per GPU (the
// module is loaded on every device the library runs on). Host code never uses the
// symbol's name as an address: each device's address is looked up once, with that
// device current, and kept in scratch_addr.
constexpr int64_t kNoAllocElems = MSA_K2Q_NOALLOC_MAX_ELEMS;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) int32_t scratch[kNoAllocElems];
std::mutex g_scratch_mu;
int32_t* g_scratch_addr[kMaxDevices] = {};

// The current device's copy of `scratch`, or nullptr (status in *rc) when it cannot be found.
int32_t* scratch_addr(int* rc) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    *rc = kErrUnsupported;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_addr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      *rc = kErrLaunch;
      return nullptr;
    }
    g_scratch_addr[dev] = static_cast<int32_t*>(p);
  }
  *rc = kOk;
  return g_scratch_addr[dev];
}

}  // namespace

}  // namespace msa

// workspace: int32 [counter_elems + total_blocks * groups].
// tri_prefix: int64 [num_seqs + 1], tri_prefix[s] = G * sum_{s'<s} nb(nb+1)/2.
extern "C" int msa_k2q_build(const int32_t* indices, const int32_t* cu_seqlens,
                             const int32_t* cu_block_lens, const int64_t* tri_prefix,
                             int64_t num_seqs, int64_t total_tokens, int64_t groups, int64_t topk_slots,
                             int64_t block_size, int64_t total_blocks, int64_t counter_elems,
                             int32_t* row_ptr, int32_t* query_indices, int32_t* slot_indices,
                             int32_t* workspace, void* stream) {
  if (!k2q_args_valid(num_seqs, total_tokens, groups, topk_slots, block_size, total_blocks, counter_elems))
    return kErrInvalidArgument;
  if (block_size * groups * topk_slots >= (int64_t(1) << 31)) return kErrUnsupported;  // edges per tile in int32
  return k2q_build_launch(indices, cu_seqlens, cu_block_lens, tri_prefix, num_seqs, total_tokens, groups,
                          topk_slots, block_size, total_blocks, counter_elems, row_ptr, query_indices, slot_indices,
                          workspace, static_cast<hipStream_t>(stream));
}

// msa_k2q_build with the library's fixed per-GPU scratch array as the workspace.
extern "C" int msa_k2q_build_noalloc(const int32_t* indices, const int32_t* cu_seqlens,
                                     const int32_t* cu_block_lens, const int64_t* tri_prefix, int64_t num_seqs,
                                     int64_t total_tokens, int64_t groups, int64_t topk_slots, int64_t block_size,
                                     int64_t total_blocks, int64_t counter_elems, int32_t* row_ptr,
                                     int32_t* query_indices, int32_t* slot_indices, void* stream) {
  if (!k2q_args_valid(num_seqs, total_tokens, groups, topk_slots, block_size, total_blocks, counter_elems))
    return kErrInvalidArgument;
  if (block_size * groups * topk_slots >= (int64_t(1) << 31)) return kErrUnsupported;  // edges per tile in int32
  if (counter_elems + total_blocks * groups > kNoAllocElems) return kErrUnsupported;  // beyond the scratch array
  int rc = kOk;
  int32_t* ws = scratch_addr(&rc);
  if (!ws) return rc;
  return k2q_build_launch(indices, cu_seqlens, cu_block_lens, tri_prefix, num_seqs, total_tokens, groups,
                          topk_slots, block_size, total_blocks, counter_elems, row_ptr, query_indices, slot_indices,
                          ws, static_cast<hipStream_t>(stream));
}

namespace msa {
namespace {

// out[r, s f + i] = f indices[r, s] + i (i < f), or -1 where indices[r, s] is negative or
// f indices[r, s] + i would pass INT32_MAX (no sequence has that many sub-blocks, so such
// an id selects nothing either way). Grid-stride over the n f outputs.
__global__ __launch_bounds__(256) void split_blocks_kernel(const int32_t* __restrict__ indices, int64_t n, int f,
                                                           int32_t* __restrict__ out) {
  const int32_t limit = (INT32_MAX - (f - 1)) / f;
  const int64_t total = n * f;
  for (int64_t o = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; o < total;
       o += static_cast<int64_t>(gridDim.x) * 256) {
    const int32_t b = indices[o / f];
    out[o] = (b >= 0 && b <= limit) ? b * f + static_cast<int32_t>(o % f) : -1;
  }
}

}  // namespace
}  // namespace msa

extern "C" int msa_split_block_indices(const int32_t* indices, int64_t rows, int64_t slots, int32_t factor,
                                       int32_t* out, void* stream) {
  if (rows < 0 || slots < 0 || factor <= 0 || (rows > 0 && slots > 0 && (!indices || !out)))
    return kErrInvalidArgument;
  if (slots > (int64_t(1) << 31) / factor) return kErrUnsupported;  // sub-block slots per row in int32
  const int64_t n = rows * slots;
  if (n == 0) return kOk;
  const int64_t blocks = std::min<int64_t>((n * factor + 255) / 256, 65536);
  hipLaunchKernelGGL(split_blocks_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), indices, n, static_cast<int>(factor), out);
  return status_from(hipGetLastError());
}
