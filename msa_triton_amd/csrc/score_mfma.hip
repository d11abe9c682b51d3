// Stage 1 on MFMA (bf16 inputs): block maxima of the indexer logits with a
// certified exact winner.
//
// Work unit: a tile of 128 consecutive (t, g) rows of the flattened [T*G] row
// space, 4 waves x 32 rows. A wave keeps its rows' query fragments in
// registers and, for every key block reachable by the tile, evaluates its
// 32 x 128 logits on v_mfma_f32_16x16x32_bf16 (exact bf16 products, fp32
// accumulation) against the block held in LDS. Key blocks are double-buffered:
// the next block is fetched from memory while the current one is used, so one
// barrier per block orders all LDS traffic. With the index dim a multiple of 32
// the blocks go from memory straight to LDS (global_load_lds_dwordx4: 16 bytes
// per lane, no staging registers) into unpadded rows whose 16-byte chunks are
// XOR-swizzled by row, so the fragment reads stay bank-conflict free. Tiles are
// issued heaviest first (the last rows of a sequence see the most blocks).
// Squared key norms (for the error bound below) are computed once per key by a
// pre-pass (score_key_norms), and each key block's largest norm and safety once per
// block by a second (score_block_norms), instead of per tile.
//
// Exactness (the public score is the reference's FP32 form of the exact winning dot,
// public_score, and the winner set must be the exact one, index_score.py:121-136): with
//   E = (Di_pad + 8) * 2^-22 * ||q|| * max_k ||k||  >=  |s_mfma - s_exact|,
// every key whose approximate directed logit is below (max_approx - 2E) is
// certainly beaten by the approximate winner. The running maximum and runner-up
// are tracked on logits whose 7 low mantissa bits are replaced by the key's
// position (4 kt + i, an inline constant of the and-or; the quarter q4 is
// recovered after the cross-lane merge and the key is 16 kt + 4 q4 + i),
// which moves each by < 2^-16 of its magnitude: the test therefore also allows
// 2^-15 max(|max|, |runner-up|) plus the smallest normal float. If exactly one key
// survives, it is the unique exact winner and only its dot is evaluated in FP64: a lane
// pair owns the row, each lane runs one half of exact_dot's fixed order (two
// sequential chains over the halves of the index dim) from the query half it keeps in
// registers and the key row in LDS, and the halves are added in that order. Each
// bf16 x bf16 product comes from v_dot2_f32_bf16 against a key word with the other
// half masked to zero: exact in fp32 when every nonzero element of the query row and
// the key block lies in [2^-60, 2^55) ("safe": products then are normal fp32 numbers,
// and no MFMA sum can overflow), and adding that exact product in FP64 gives the bits
// of exact_dot's fused multiply-add. Pairs of an unsafe row or block go to the resolve
// kernel below.
// Otherwise the (row, block) pair is marked in a bitmap that a second
// kernel (score_fwd_resolve) settles after the main pass: one wave re-evaluates
// every visible key of the block in FP64 (same order) and takes max / tie count /
// first winner exactly. Deferring keeps the rare ambiguous rows (a few per
// thousand on random data) from holding the other waves of a workgroup at the
// next block barrier.
// A negative scale flips the query signs once (exact), so every comparison is
// on the directed dot.
#include <type_traits>

#include "mfma_util.hpp"
#include "score_mfma.hpp"

namespace msa {

namespace {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

constexpr int kTileRows = 128;  // 4 waves x 32 rows
constexpr int kThreads = 256;

// Workspace: squared key norms (fp32 per key), the key blocks' norms (fp32, at each
// block's first key), then the ambiguous-pair bitmap, block-major: bit
// block * rows_pad + row of 32-bit words, rows_pad = rows rounded up to a whole number
// of resolve chunks.
constexpr int kResolveRows = 8192;  // rows per resolve workgroup
int64_t align256(int64_t x) { return (x + 255) & ~int64_t{255}; }
int64_t ws_bnorm_offset(int64_t T) { return align256(4 * (T > 0 ? T : 1)); }
int64_t ws_bitmap_offset(int64_t T) { return 2 * ws_bnorm_offset(T); }
int64_t rows_padded(int64_t rows) { return (rows + kResolveRows - 1) / kResolveRows * kResolveRows; }
int64_t bitmap_words(int64_t rows, int64_t NB) { return rows_padded(rows) / 32 * NB; }

template <int NK>
struct ScoreSmem {
  static constexpr int DP = 32 * NK;
  static constexpr int RS = DP + 8;  // row stride (bf16) of a padded key block (index dim below DP)
  alignas(16) uint16_t k[2][128 * RS];  // full-width blocks use the first 128 * DP entries (swizzled rows)
};

// Offset (bf16 elements) of dims [d, d + 8) of key `row` in a buffered block (d a
// multiple of 8). Full width: rows DP apart, 16-byte chunk c at c ^ swz(row), with
// swz chosen so the 16 rows one fragment read touches land on 16 distinct bank
// groups. Otherwise: rows DP + 8 apart, unswizzled.
template <int NK, bool FULLD>
__device__ __forceinline__ int key_off(int row, int d) {
  constexpr int DP = 32 * NK, CPK = DP / 8;
  if constexpr (FULLD) {
    constexpr int SH = NK == 4 ? 0 : (NK == 2 ? 1 : 2);  // rows sharing a bank base: 16 / CPK apart
    return row * DP + 8 * ((d >> 3) ^ ((row >> SH) & (CPK - 1)));
  } else {
    return row * (DP + 8) + d;
  }
}

// Logit bits with the key position in the 7 low mantissa bits (see the header comment).
__device__ __forceinline__ float pack_key(float v, uint32_t pos) {
  return __uint_as_float((__float_as_uint(v) & 0xffffff80u) | pos);
}
constexpr float kMaskedLogit = -3.0e38f;  // a finite stand-in for masked keys (packing keeps it finite)

// v_max3_f32 on finite values. Written out because the optimiser, given fmaxf, adds a
// canonicalisation of every operand whose bits it cannot trace to an FP operation.
__device__ __forceinline__ float max3(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

__device__ __forceinline__ float min2(float a, float b) {
  float r;
  asm("v_min_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

// The value of this lane and that of lane ^ 32 (or ^ 16), in an order that depends on
// the lane: v_permlane32_swap (v_permlane16_swap) of x with itself. For a symmetric
// combination (max, min, a sum of two) the order does not matter.
struct LanePair {
  uint32_t a, b;
};
__device__ __forceinline__ LanePair pair_xor32(uint32_t x) {
  const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  return LanePair{r[0], r[1]};
}
__device__ __forceinline__ LanePair pair_xor16(uint32_t x) {
  const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
  return LanePair{r[0], r[1]};
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Both bf16 of a word zero or of magnitude in [2^-60, 2^55) (biased exponent 67 .. 181):
// the product of two such values is zero or a normal fp32 number below 2^110, and a
// sum of up to 128 of them stays below 2^117.
__device__ __forceinline__ bool bf16_safe(uint32_t x16) {
  const uint32_t e = (x16 >> 7) & 0xffu;
  return (x16 & 0x7fffu) == 0u || (e >= 67u && e <= 181u);
}
__device__ __forceinline__ bool word_safe(uint32_t w) { return bf16_safe(w & 0xffffu) && bf16_safe(w >> 16); }

// fp32 product of the low (lo) or high bf16 of a and of b, exact when both are safe.
__device__ __forceinline__ float prod_lo(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b & 0xffffu),
                                         0.0f, false);
}
__device__ __forceinline__ float prod_hi(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b & 0xffff0000u), 0.0f, false);
}

// Iteration space of a tile: (sequence, block) pairs for every sequence overlapping
// the tile rows [r0, r0 + nr), blocks 0 .. the last row's query block.
struct BlockCursor {
  int s;       // sequence
  int b;       // sequence-local block
  int b_last;  // last block of this sequence the tile needs
};

__device__ __forceinline__ int last_block_of(const int32_t* __restrict__ cu, int s, int64_t r0, int nr, int G,
                                             int B) {
  const int64_t start = cu[s], end = cu[s + 1];
  const int64_t t_last = (r0 + nr - 1) / G;
  const int64_t t = t_last < end - 1 ? t_last : end - 1;
  return static_cast<int>((t - start) / B);
}

// Next (s, b) after c; s == nseq when the tile has no more blocks.
__device__ __forceinline__ BlockCursor next_block(const int32_t* __restrict__ cu, int nseq, BlockCursor c,
                                                  int64_t r0, int nr, int G, int B) {
  if (c.b < c.b_last) {
    ++c.b;
    return c;
  }
  const int64_t t_last = (r0 + nr - 1) / G;
  for (int s = c.s + 1; s < nseq && cu[s] <= t_last; ++s) {
    if (cu[s + 1] > cu[s]) return BlockCursor{s, 0, last_block_of(cu, s, r0, nr, G, B)};
  }
  return BlockCursor{nseq, 0, -1};
}

}  // namespace

// Squared norm of every index key, rounded up by 1.0001 (bounds the fp32 rounding of
// the sum): the max over a key block enters the MFMA logits' error bound. The sign bit
// is set for a key that is not safe (a nonzero element outside [2^-60, 2^55)).
// Also clears the ambiguous-pair bitmap the main pass marks.
__global__ __launch_bounds__(256) void score_key_norms(const uint16_t* __restrict__ ik, int64_t T, int Di,
                                                       float* __restrict__ knorm2, uint32_t* __restrict__ amb,
                                                       int64_t amb_words) {
  const int64_t j = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (j < amb_words) amb[j] = 0u;
  if (j >= T) return;
  float n2 = 0.f;
  bool safe = true;
  for (int d = 0; d < Di; d += 8) {
    const uint4 w = *reinterpret_cast<const uint4*>(ik + j * Di + d);
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      n2 = fmaf(bf16_lo(ws[u]), bf16_lo(ws[u]), n2);
      n2 = fmaf(bf16_hi(ws[u]), bf16_hi(ws[u]), n2);
      safe = safe && word_safe(ws[u]);
    }
  }
  knorm2[j] = safe ? n2 * 1.0001f : -(n2 * 1.0001f) - 1.0f;  // unsafe: negative
}

// Per key block, stored at the block's first key: the largest key norm of the block,
// sqrt(max |knorm2|), negated when a key of the block is not safe (or not a number).
// Safety is read from the sign bit: a block whose only unsafe key is NaN (fmaxf skips
// its NaN entry) and whose other keys are zero stores -0.
__global__ __launch_bounds__(256) void score_block_norms(const float* __restrict__ knorm2,
                                                         const int32_t* __restrict__ cu, int nseq, int64_t T, int B,
                                                         float* __restrict__ bnorm) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (t >= T) return;
  const int s = find_seq(cu, nseq, t);
  const int64_t start = cu[s], end = cu[s + 1];
  if ((t - start) % B != 0) return;
  const int64_t e = t + B < end ? t + B : end;
  float m = 0.f;
  bool safe = true;
  for (int64_t j = t; j < e; ++j) {
    const float v = knorm2[j];
    m = fmaxf(m, fabsf(v));
    safe = safe && v >= 0.f;
  }
  const float r = sqrtf(m);
  bnorm[t] = safe ? r : -r;
}

// Two workgroups per CU; one for the widest partial-width variant (index dim 72..120),
// whose register staging of the next block does not fit beside two.
template <int NK, bool FULLD>
__global__ __launch_bounds__(kThreads, NK == 4 && !FULLD ? 1 : 2) void score_fwd_mfma_kernel(const uint16_t* __restrict__ iq,
                                                                     const uint16_t* __restrict__ ik,
                                                                     const int32_t* __restrict__ cu, int nseq,
                                                                     int64_t rows, int G, int Di, int NB, int B,
                                                                     double scale, const float* __restrict__ bnorm,
                                                                     uint32_t* __restrict__ amb, int64_t rows_pad,
                                                                     float* __restrict__ scores,
                                                                     int32_t* __restrict__ tie) {
  constexpr int DP = 32 * NK;
  constexpr int CPK = DP / 8;                 // 16-byte chunks per key row
  constexpr int KCH = 128 * CPK / kThreads;   // chunks per thread per key block
  constexpr int HF = DP / 2;                  // max dims of a query half (Di / 2 <= DP / 2)
  __shared__ ScoreSmem<NK> sm;
  const int tid = threadIdx.x, lane = tid & 63, c = lane & 15, q4 = lane >> 4;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar) index
  const int64_t r0 = static_cast<int64_t>(gridDim.x - 1 - blockIdx.x) * kTileRows;  // heaviest tiles first
  const int nr = static_cast<int>(rows - r0 < kTileRows ? rows - r0 : kTileRows);
  const bool neg = scale < 0.0;
  const float fscale = static_cast<float>(fabs(scale));  // the reference's FP32 |scale|
  const uint32_t flip = neg ? 0x80008000u : 0u;
  const float cerr = static_cast<float>(DP + 8) * 0x1p-22f;
  // exact_dot's split point (Di % 8 == 0, so h % 4 == 0); compile-time for Di == DP
  const int h = FULLD ? DP / 2 : Di / 2;

  // ---- this wave's rows: MFMA B fragments (rows 16 rt + c) ...
  const int wr0 = 32 * wid;  // first tile row of the wave
  bf16x8 qf[2][NK];
  int64_t mtok[2];
  bool min_tile[2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const int rr = wr0 + 16 * rt + c;
    min_tile[rt] = rr < nr;
    mtok[rt] = min_tile[rt] ? (r0 + rr) / G : -1;
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) {
      const int d0 = 32 * kk + 8 * q4;
      uint4 w = make_uint4(0u, 0u, 0u, 0u);
      if (min_tile[rt] && d0 < Di) w = *reinterpret_cast<const uint4*>(iq + (r0 + rr) * Di + d0);
      w.x ^= flip;
      w.y ^= flip;
      w.z ^= flip;
      w.w ^= flip;
      qf[rt][kk] = __builtin_bit_cast(bf16x8, w);
    }
  }
  // ... and the exact-dot layout: lane (pr = lane & 31, hf = lane >> 5) keeps half hf
  // (dims [hf h, hf h + h)) of row wr0 + pr, sign-flipped, packed two per word.
  const int pr = lane & 31, hf = lane >> 5;
  const int prow = wr0 + pr;
  const bool pin = prow < nr;
  uint32_t qh[HF / 2];
  float pn2 = 0.f;
  bool psafe = true;
#pragma unroll
  for (int w4 = 0; w4 < HF / 4; ++w4) {  // 8-byte loads: 4 dims each
    uint2 x = make_uint2(0u, 0u);
    if (pin && 4 * w4 < h) x = *reinterpret_cast<const uint2*>(iq + (r0 + prow) * Di + hf * h + 4 * w4);
    x.x ^= flip;
    x.y ^= flip;
    qh[2 * w4] = x.x;
    qh[2 * w4 + 1] = x.y;
    pn2 = fmaf(bf16_lo(x.x), bf16_lo(x.x), pn2);
    pn2 = fmaf(bf16_hi(x.x), bf16_hi(x.x), pn2);
    pn2 = fmaf(bf16_lo(x.y), bf16_lo(x.y), pn2);
    pn2 = fmaf(bf16_hi(x.y), bf16_hi(x.y), pn2);
    psafe = psafe && word_safe(x.x) && word_safe(x.y);
  }
  pn2 += __shfl_xor(pn2, 32, kWave);
  psafe = psafe && __shfl_xor(static_cast<int>(psafe), 32, kWave) != 0;  // both halves of the row
  const float pnorm = sqrtf(pn2) * 1.0001f;  // ||q|| of row prow, rounded up
  float mnorm[2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) mnorm[rt] = __shfl(pnorm, 16 * rt + c, kWave);
  bool msafe[2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) msafe[rt] = __shfl(static_cast<int>(psafe), 16 * rt + c, kWave) != 0;
  const int64_t ptok = pin ? (r0 + prow) / G : -1;

  // ---- key block staging
  uint4 kreg[FULLD ? 1 : KCH];  // register staging of partial-width blocks
  // Full width: wave wid's instruction i fills physical chunks p = (wid KCH + i) 64 + lane
  // of the buffer (1 KiB per instruction), holding row p / CPK, logical chunk
  // (p % CPK) ^ swz(row). Rows advance by 16 every KCH / 2 instructions and the swizzle
  // repeats every 16 rows, so the offsets of the first half serve the second.
  constexpr int SH = NK == 4 ? 0 : (NK == 2 ? 1 : 2);
  constexpr int NP = FULLD ? KCH / 2 : 1;
  // element offset of instruction i's chunk within a complete block (block-invariant)
  auto chunk_off = [&](int i) {
    const int p = (wid * KCH + i % NP) * 64 + lane;
    const int row = p / CPK, pc = p % CPK;
    return static_cast<uint32_t>(row * DP + 8 * (pc ^ ((row >> SH) & (CPK - 1))) + (i < NP ? 0 : 16 * DP));
  };
  auto fetch = [&](const BlockCursor& bc, const uint16_t* gsrc, uint16_t* into) {
    if (bc.s >= nseq) return;
    const int64_t kb = cu[bc.s] + static_cast<int64_t>(bc.b) * B;
    const int64_t end = cu[bc.s + 1];
    const int nk = static_cast<int>(end - kb < B ? end - kb : B);
    if constexpr (FULLD) {
      char* dst = reinterpret_cast<char*>(into) + wid * KCH * 1024;
      if (nk == 128) {  // a complete block: scalar base plus the precomputed offsets
        const uint16_t* src = gsrc + kb * DP;
#pragma unroll
        for (int i = 0; i < KCH; ++i)
          __builtin_amdgcn_global_load_lds(src + static_cast<int>(chunk_off(i)),
                                           (__attribute__((address_space(3))) void*)(dst + i * 1024), 16, 0, 0);
      } else {  // rows past the block's end repeat its last key (masked later)
#pragma unroll
        for (int i = 0; i < KCH; ++i) {
          const int p = (wid * KCH + i) * 64 + lane;
          const int row = p / CPK, pc = p % CPK;
          const int lc = pc ^ ((row >> SH) & (CPK - 1));
          const int rowc = row < nk ? row : nk - 1;
          __builtin_amdgcn_global_load_lds(gsrc + (kb + rowc) * Di + 8 * lc,
                                           (__attribute__((address_space(3))) void*)(dst + i * 1024), 16, 0, 0);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < KCH; ++i) {
        const int e = tid + kThreads * i;
        const int kl = e / CPK, d0 = 8 * (e % CPK);
        kreg[i] = (kl < nk && d0 < Di) ? *reinterpret_cast<const uint4*>(gsrc + (kb + kl) * Di + d0)
                                       : make_uint4(0u, 0u, 0u, 0u);
      }
    }
  };
  auto commit = [&](int into) {
    if constexpr (!FULLD) {
#pragma unroll
      for (int i = 0; i < KCH; ++i) {
        const int e = tid + kThreads * i;
        const int kl = e / CPK, d0 = 8 * (e % CPK);
        *reinterpret_cast<uint4*>(sm.k[into] + key_off<NK, FULLD>(kl, d0)) = kreg[i];
      }
    }
  };
  // the block's largest key norm, negated when a key of the block is not safe
  auto block_norm = [&](const BlockCursor& bc) {
    return bc.s < nseq ? bnorm[cu[bc.s] + static_cast<int64_t>(bc.b) * B] : 0.f;
  };

  // first (sequence, block) of the tile
  BlockCursor cur{nseq, 0, -1};
  {
    const int64_t t_first = r0 / G;
    const int s0 = find_seq(cu, nseq, t_first);
    cur = BlockCursor{s0, 0, last_block_of(cu, s0, r0, nr, G, B)};
  }
  const float cn = block_norm(cur);
  fetch(cur, ik, sm.k[0]);
  commit(0);
  __builtin_amdgcn_s_waitcnt(0);  // this thread's direct-to-LDS loads have landed
  __syncthreads();
  float kmax = fabsf(cn);
  bool bsafe = !__builtin_signbit(cn);  // -0 marks an unsafe block too
  int buf = 0;
  while (cur.s < nseq) {
    const BlockCursor nxt = next_block(cu, nseq, cur, r0, nr, G, B);
    const float nn = block_norm(nxt);
    // The next block's fetch and this block's LDS reads go through the restrict-qualified
    // pointers of one inlined call, so the compiler's wait insertion can tell the fetch's
    // LDS writes (buffer buf ^ 1) from the reads (buffer buf): without that it waits for
    // the whole fetch before the first read, and the fetch would not overlap the block.
    [&](const uint16_t* __restrict__ ksrc, const uint16_t* __restrict__ kt_base, uint16_t* __restrict__ knext) {
    fetch(nxt, ksrc, knext);  // in flight while this block is evaluated (that buffer's readers passed the last barrier)

    const int64_t start = cu[cur.s], end = cu[cur.s + 1];
    const int64_t kb = start + static_cast<int64_t>(cur.b) * B;
    const int nk = static_cast<int>(end - kb < B ? end - kb : B);
    // visible keys of the lane's MFMA rows (0: row not in this sequence or block in its future)
    int lim[2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const int64_t t = mtok[rt];
      const int64_t v = (t >= start && t < end) ? t - kb + 1 : 0;
      lim[rt] = v <= 0 ? 0 : (v < nk ? static_cast<int>(v) : nk);
    }
    const bool wave_on = __ballot(lim[0] > 0 || lim[1] > 0) != 0;  // wave-uniform
    // approximate logits, 16 keys at a time, key position packed into their low bits,
    // folded into a per-row running top 2: m1 the maximum, m2 the largest other value
    // (med3(m1, v, m2) is the new second largest)
    float m1[2] = {kMaskedLogit, kMaskedLogit}, m2[2] = {kMaskedLogit, kMaskedLogit};
    // med3(m1, v, +inf) is the maximum; unlike fmaxf it needs no canonicalised inputs. The
    // +inf sits in a register the optimiser cannot see through, or it would turn the med3
    // back into a maximum with canonicalisations.
    float pinf = __builtin_inff();
    asm volatile("" : "+v"(pinf));
    auto scan = [&](auto masked) {
#pragma unroll
      for (int kt = 0; kt < 8; ++kt) {
        bf16x8 kf[NK];
#pragma unroll
        for (int kk = 0; kk < NK; ++kk) kf[kk] = load_frag(kt_base + key_off<NK, FULLD>(16 * kt + c, 32 * kk + 8 * q4));
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
          f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kk = 0; kk < NK; ++kk) a = mfma(kf[kk], qf[rt][kk], a);
#pragma unroll
          for (int i = 0; i < 4; i += 2) {  // two logits x, y at a time (m1 >= m2 throughout):
            float x = a[i], y = a[i + 1];     // second largest of {m1, m2, x, y} = max(m2, med3(m1, x, y))
            if constexpr (decltype(masked)::value) {
              x = 16 * kt + 4 * q4 + i < lim[rt] ? x : kMaskedLogit;
              y = 16 * kt + 4 * q4 + i + 1 < lim[rt] ? y : kMaskedLogit;
            }
            x = pack_key(x, 4 * kt + i);
            y = pack_key(y, 4 * kt + i + 1);
            const float t = __builtin_amdgcn_fmed3f(m1[rt], x, y);
            m2[rt] = __builtin_amdgcn_fmed3f(m2[rt], t, pinf);
            m1[rt] = max3(m1[rt], x, y);
          }
        }
      }
    };
    if (wave_on) {
      if (__ballot(lim[0] < 128 || lim[1] < 128) == 0)  // no key masked in the wave
        scan(std::false_type{});
      else
        scan(std::true_type{});
    }
    if (wave_on) {
      // merge the four key quarters of each row; the winner is certified unique iff no
      // other key comes within the bound of the maximum
      int widx[2], wcnt[2];
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        float a1 = m1[rt], a2 = m2[rt];
#pragma unroll
        for (int o = 16; o <= 32; o <<= 1) {  // with the quarter of lane ^ o
          const LanePair p1 = o == 16 ? pair_xor16(__float_as_uint(a1)) : pair_xor32(__float_as_uint(a1));
          const LanePair p2 = o == 16 ? pair_xor16(__float_as_uint(a2)) : pair_xor32(__float_as_uint(a2));
          const float u = __uint_as_float(p1.a), v = __uint_as_float(p1.b);
          a2 = max3(__uint_as_float(p2.a), __uint_as_float(p2.b), min2(u, v));
          a1 = max3(u, v, v);
        }
        // the quarter holding the maximum (unique whenever the row is certified)
        int wq = m1[rt] == a1 ? q4 : 4;
        const LanePair w16 = pair_xor16(static_cast<uint32_t>(wq));
        wq = min(static_cast<int>(w16.a), static_cast<int>(w16.b));
        const LanePair w32 = pair_xor32(static_cast<uint32_t>(wq));
        wq = min(static_cast<int>(w32.a), static_cast<int>(w32.b));
        const int pos = static_cast<int>(__float_as_uint(a1) & 0x7fu);  // 4 kt + i
        widx[rt] = 16 * (pos >> 2) + 4 * wq + (pos & 3);
        const float bound = 2.f * cerr * mnorm[rt] * kmax + 0x1p-15f * fmaxf(fabsf(a1), fabsf(a2)) + 0x1p-126f;
        // 2: at least two candidates, or products not certainly exact in fp32
        wcnt[rt] = (a2 >= a1 - bound || !(bsafe && msafe[rt])) ? 2 : 1;
      }
      // lane pair (pr, hf): row wr0 + pr = 16 rt + c with rt = pr >> 4 -- this lane's c matches
      const int prt = pr >> 4;
      const int myidx = prt ? widx[1] : widx[0];
      const int mycnt = prt ? wcnt[1] : wcnt[0];
      const int mylim = prt ? lim[1] : lim[0];
      const bool row_ok = pin && mylim > 0;
      // unique winner: its exact dot, half per lane, in exact_dot's order (exact fp32
      // products of safe bf16 values added in FP64)
      double half = 0.0;
      if (row_ok && mycnt == 1) {
#pragma unroll
        for (int j8 = 0; j8 < HF / 8; ++j8) {  // 8 dims per 16-byte read
          if (FULLD || 8 * j8 < h) {
            const uint16_t* kp = kt_base + key_off<NK, FULLD>(myidx, hf * h + 8 * j8);
            uint32_t kx[4];
            if (FULLD) {
              const uint4 kw = *reinterpret_cast<const uint4*>(kp);
              kx[0] = kw.x, kx[1] = kw.y, kx[2] = kw.z, kx[3] = kw.w;
            } else if (8 * j8 + 8 <= h) {  // the second half may start 8 bytes into a 16-byte unit (h % 8 == 4)
              const uint2 ka = *reinterpret_cast<const uint2*>(kp), kb = *reinterpret_cast<const uint2*>(kp + 4);
              kx[0] = ka.x, kx[1] = ka.y, kx[2] = kb.x, kx[3] = kb.y;
            } else {  // h % 8 == 4: the last four dims of the half
              const uint2 kw = *reinterpret_cast<const uint2*>(kp);
              kx[0] = kw.x, kx[1] = kw.y, kx[2] = kx[3] = 0u;
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              if (FULLD || 8 * j8 + 2 * u < h) {
                half += static_cast<double>(prod_lo(qh[4 * j8 + u], kx[u]));
                half += static_cast<double>(prod_hi(qh[4 * j8 + u], kx[u]));
              }
            }
          }
        }
      }
      // the two halves of the row (lanes pr and pr + 32), summed
      const uint64_t hbits = static_cast<uint64_t>(__double_as_longlong(half));
      const LanePair hlo = pair_xor32(static_cast<uint32_t>(hbits));
      const LanePair hhi = pair_xor32(static_cast<uint32_t>(hbits >> 32));
      const double h0 = __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(hhi.a) << 32) | hlo.a));
      const double h1 = __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(hhi.b) << 32) | hlo.b));
      if (row_ok && mycnt == 1 && hf == 0) {
        const int64_t out = (r0 + prow) * NB + cur.b;
        scores[out] = public_score(h0 + h1, fscale);
        if (tie) tie[out] = myidx + 1;
      }
      // ambiguous rows: marked for score_fwd_resolve
      if (row_ok && mycnt != 1 && hf == 0) {
        const int64_t bit = static_cast<int64_t>(cur.b) * rows_pad + r0 + prow;
        atomicOr(amb + (bit >> 5), 1u << (bit & 31));
      }
    }
    }(ik, sm.k[buf], sm.k[buf ^ 1]);
    if (nxt.s < nseq) commit(buf ^ 1);  // that buffer's readers finished before the last barrier
    __builtin_amdgcn_s_waitcnt(0);       // the next block's direct-to-LDS loads have landed
    __syncthreads();  // this block's readers are done; the next block is visible
    kmax = fabsf(nn);
    bsafe = !__builtin_signbit(nn);
    buf ^= 1;
    cur = nxt;
  }

  // ---- blocks without a causal key: -inf, tie code 0 (each wave fills its rows)
  const int64_t pstart = pin ? cu[find_seq(cu, nseq, ptok)] : 0;
  const int pqb = pin ? static_cast<int>((ptok - pstart) / B) : NB;
  for (int j = 0; j < 32; ++j) {
    const int qbj = __shfl(pqb, j, kWave);
    if (wr0 + j >= nr) break;
    const int64_t base = (r0 + wr0 + j) * NB;
    for (int b = qbj + 1 + lane; b < NB; b += kWave) {
      scores[base + b] = -__builtin_inff();
      if (tie) tie[base + b] = 0;
    }
  }
}

// The ambiguous (row, block) pairs the main pass marked, settled exactly. Workgroup
// (b, c) takes block b for rows [c, c + kResolveRows): it lists the marked rows in
// order, and for each run of listed rows of one sequence stages that sequence's block
// b in LDS; the four waves then take windows of up to kResolvePairs rows of the run
// independently. In a window, lane l runs exact_dot's two FMA chains (over the halves
// of the index dim) for keys l and l + 64 and every row of the window at once (each
// key element and each query element converted to FP64 once per window), from the
// window's query rows staged in the wave's LDS slot (sign-directed bf16), and adds
// the halves half 0 first; the maximum is reduced over the wave, tie count and first
// winner come from ballots. The score and tie code are written as the exact kernel
// writes them.
constexpr int kResolvePairs = 4;
__global__ __launch_bounds__(256) void score_fwd_resolve(const uint16_t* __restrict__ iq,
                                                         const uint16_t* __restrict__ ik,
                                                         const int32_t* __restrict__ cu, int nseq, int64_t rows,
                                                         int64_t rows_pad, int G, int Di, int NB, int B,
                                                         double scale, const uint32_t* __restrict__ amb,
                                                         float* __restrict__ scores, int32_t* __restrict__ tie) {
  constexpr int KS = 136;  // key row stride in LDS (bf16): consecutive rows hit distinct 16-byte bank groups
  constexpr int P = kResolvePairs;
  __shared__ alignas(16) uint16_t keys[128 * KS];
  __shared__ alignas(16) uint16_t qs[4][P][128];
  __shared__ uint16_t list[kResolveRows];
  __shared__ int wsum[4];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int b = blockIdx.x;
  const int64_t c0 = static_cast<int64_t>(blockIdx.y) * kResolveRows;
  // ---- the marked rows of this chunk, ascending (one bitmap word per thread)
  constexpr int NW = kResolveRows / 32;  // bitmap words of the chunk (<= threads)
  static_assert(NW <= 256, "one bitmap word per thread");
  uint32_t mine = tid < NW ? amb[(static_cast<int64_t>(b) * rows_pad + c0) / 32 + tid] : 0u;
  const int cnt = __popc(mine);
  int incl = cnt;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o, kWave);
    if (lane >= o) incl += y;
  }
  if (lane == 63) wsum[wv] = incl;
  if (__syncthreads_or(mine != 0u) == 0) return;  // nothing marked (uniform)
  int o = incl - cnt;
  for (int w = 0; w < wv; ++w) o += wsum[w];
  for (; mine; mine &= mine - 1) list[o++] = static_cast<uint16_t>(32 * tid + __builtin_ctz(mine));
  const int n = wsum[0] + wsum[1] + wsum[2] + wsum[3];
  const uint16_t flip = scale < 0.0 ? 0x8000u : 0u;
  const int h = Di / 2;  // a multiple of 4
  __syncthreads();  // the list is complete
  for (int i = 0; i < n;) {  // runs of rows of one sequence (uniform)
    const int s = find_seq(cu, nseq, (c0 + list[i]) / G);
    const int64_t start = cu[s], end = cu[s + 1];
    const int64_t end_row = end * G - c0;  // chunk-relative end of the sequence's rows
    int j = i + 1;
    while (j < n && list[j] < end_row) ++j;
    const int64_t k0 = start + static_cast<int64_t>(b) * B;
    const int nk = static_cast<int>((k0 + B < end ? k0 + B : end) - k0);  // >= 1: a listed row sees block b
    const int cpr = Di / 8;
    for (int e = tid; e < nk * cpr; e += 256) {
      const int r = e / cpr, c = e % cpr;
      *reinterpret_cast<uint4*>(keys + r * KS + 8 * c) = *reinterpret_cast<const uint4*>(ik + (k0 + r) * Di + 8 * c);
    }
    __syncthreads();  // the block is staged
    for (int w0 = i + P * wv; w0 < j; w0 += 4 * P) {  // this wave's windows
      const int np = j - w0 < P ? j - w0 : P;
      for (int e = lane; e < np * Di; e += kWave) {
        const int p = e / Di, d = e % Di;
        qs[wv][p][d] = iq[(c0 + list[w0 + p]) * Di + d] ^ flip;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      double acc[2][2][P];  // [key lane / lane + 64][half][row]
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
          for (int p = 0; p < P; ++p) acc[kh][hh][p] = 0.0;
      for (int d = 0; d < h; d += 4) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          double qv[P][4];
#pragma unroll
          for (int p = 0; p < P; ++p) {
            const uint2 w = *reinterpret_cast<const uint2*>(&qs[wv][p][hh * h + d]);
            qv[p][0] = static_cast<double>(bf16_lo(w.x));
            qv[p][1] = static_cast<double>(bf16_hi(w.x));
            qv[p][2] = static_cast<double>(bf16_lo(w.y));
            qv[p][3] = static_cast<double>(bf16_hi(w.y));
          }
#pragma unroll
          for (int kh = 0; kh < 2; ++kh) {
            const uint2 w = *reinterpret_cast<const uint2*>(keys + (lane + 64 * kh) * KS + hh * h + d);
            const double k4[4] = {static_cast<double>(bf16_lo(w.x)), static_cast<double>(bf16_hi(w.x)),
                                  static_cast<double>(bf16_lo(w.y)), static_cast<double>(bf16_hi(w.y))};
#pragma unroll
            for (int p = 0; p < P; ++p) {
              double a = acc[kh][hh][p];
#pragma unroll
              for (int u = 0; u < 4; ++u) a = fma(qv[p][u], k4[u], a);
              acc[kh][hh][p] = a;
            }
          }
        }
      }
#pragma unroll
      for (int p = 0; p < P; ++p) {
        if (p < np) {
          const int64_t row = c0 + list[w0 + p];
          const int vis = static_cast<int>((row / G + 1 < k0 + nk ? row / G + 1 : k0 + nk) - k0);
          const double v0 = lane < vis ? acc[0][0][p] + acc[0][1][p] : -__builtin_inf();
          const double v1 = lane + 64 < vis ? acc[1][0][p] + acc[1][1][p] : -__builtin_inf();
          const double wbest = wave_max_f64(fmax(v0, v1));
          // visible keys only: with NaN dots (skipped by the maximum) wbest may be -inf, the value
          // of the masked lanes; a row without any non-NaN visible dot gets count 0 (code 0)
          const uint64_t m0 = __ballot(lane < vis && v0 == wbest), m1 = __ballot(lane + 64 < vis && v1 == wbest);
          if (lane == 0) {
            const int count = __popcll(m0) + __popcll(m1);
            const int first = m0 ? __builtin_ctzll(m0) : 64 + __builtin_ctzll(m1);
            const int64_t out = row * NB + b;
            scores[out] = public_score(wbest, static_cast<float>(fabs(scale)));
            if (tie) tie[out] = count == 1 ? first + 1 : -count;
          }
        }
      }
      __builtin_amdgcn_wave_barrier();  // qs is rewritten by the next window
    }
    __syncthreads();  // the block's readers are done before the next run restages it
    i = j;
  }
}

bool score_mfma_supported(int Di, int B, double scale) {
  return scale != 0.0 && Di >= 8 && Di <= 128 && Di % 8 == 0 && B >= 1 && B <= 128;
}

int64_t score_fwd_mfma_workspace_bytes(int64_t total_tokens, int64_t rows, int64_t NB) {
  return ws_bitmap_offset(total_tokens) + 4 * bitmap_words(rows, NB);
}

int score_fwd_mfma_launch(const void* iq, const void* ik, const int32_t* cu, int nseq, int64_t rows, int G, int Di,
                          int NB, int B, double scale, float* scores, int32_t* tie, void* ws, hipStream_t st) {
  if (!ws) return kErrInvalidArgument;
  const dim3 grid(grid_1d(rows, kTileRows)), block(kThreads);
  const auto* q = static_cast<const uint16_t*>(iq);
  const auto* k = static_cast<const uint16_t*>(ik);
  const int64_t T = rows / G;
  char* wsb = static_cast<char*>(ws);
  float* knorm2 = reinterpret_cast<float*>(wsb);
  float* bnorm = reinterpret_cast<float*>(wsb + ws_bnorm_offset(T));
  auto* amb = reinterpret_cast<uint32_t*>(wsb + ws_bitmap_offset(T));
  const int64_t words = bitmap_words(rows, NB);
  const int64_t rows_pad = rows_padded(rows);
  hipLaunchKernelGGL(score_key_norms, dim3(grid_1d(T > words ? T : words, 256)), dim3(256), 0, st, k, T, Di,
                     knorm2, amb, words);
  hipLaunchKernelGGL(score_block_norms, dim3(grid_1d(T, 256)), dim3(256), 0, st, knorm2, cu, nseq, T, B, bnorm);
#define MSA_SCORE_MFMA(NKV, FD) hipLaunchKernelGGL((score_fwd_mfma_kernel<NKV, FD>), grid, block, 0, st, q, k, cu, nseq, rows, G, Di, NB, B, scale, bnorm, amb, rows_pad, scores, tie)
  const int nk = Di <= 32 ? 1 : (Di <= 64 ? 2 : 4);
  const bool fd = Di == 32 * nk;
  if (nk == 1) { if (fd) MSA_SCORE_MFMA(1, true); else MSA_SCORE_MFMA(1, false); }
  else if (nk == 2) { if (fd) MSA_SCORE_MFMA(2, true); else MSA_SCORE_MFMA(2, false); }
  else { if (fd) MSA_SCORE_MFMA(4, true); else MSA_SCORE_MFMA(4, false); }
#undef MSA_SCORE_MFMA
  hipLaunchKernelGGL(score_fwd_resolve, dim3(NB, static_cast<unsigned>(rows_pad / kResolveRows)), dim3(256), 0, st,
                     q, k, cu, nseq, rows, rows_pad, G, Di, NB, B, scale, amb, scores, tie);
  return status_from(hipGetLastError());
}

}  // namespace msa
