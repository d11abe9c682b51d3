// Shared device helpers for the MiniMax-M3 sparse-attention kernels (gfx950).
//
// Conventions used by every kernel in this library:
//  * Public metadata (cu_seqlens, block indices, CSR arrays) is int32; every
//    address is formed in int64 before any multiply-add, mirroring the
//    reference's widening rule (triton/_addressing.py:11-18).
//  * Element types are selected by a compile-time dtype tag; arithmetic is
//    fp32 (MFMA accumulate / VALU) or fp64 where exactness is required.
//  * One wavefront is 64 lanes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace msa {

constexpr int kWave = 64;

enum DType : int { kF32 = 0, kF16 = 1, kBF16 = 2 };

enum Status : int {
  kOk = 0,
  kErrInvalidArgument = 1,
  kErrUnsupported = 2,
  kErrLaunch = 3,
};

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;

// ---- scalar conversions ----------------------------------------------------

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even fp32 -> bf16 bits (NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float bf16_round(float f) { return bf16_bits_to_f32(f32_to_bf16_bits(f)); }

// x rounded to fp32 toward zero with any inexact remainder folded into the last bit
// ("round to odd"). Rounding that value to nearest in a format of at most 22 significand
// bits (fp16) gives the correctly rounded x itself: no double-rounding error from going
// through fp32. NaN stays NaN, infinities and overflow round as x would.
__device__ __forceinline__ float f64_to_f32_odd(double x) {
  const float f = __double2float_rz(x);
  return static_cast<double>(f) == x ? f : __uint_as_float(__float_as_uint(f) | 1u);
}

template <int DT>
__device__ __forceinline__ float load_as_f32(const void* base, int64_t i) {
  if constexpr (DT == kF32) {
    return static_cast<const float*>(base)[i];
  } else if constexpr (DT == kF16) {
    return static_cast<float>(static_cast<const _Float16*>(base)[i]);
  } else {
    return bf16_bits_to_f32(static_cast<const uint16_t*>(base)[i]);
  }
}

template <int DT>
__device__ __forceinline__ void store_from_f32(void* base, int64_t i, float v) {
  if constexpr (DT == kF32) {
    static_cast<float*>(base)[i] = v;
  } else if constexpr (DT == kF16) {
    static_cast<_Float16*>(base)[i] = static_cast<_Float16>(v);
  } else {
    static_cast<uint16_t*>(base)[i] = f32_to_bf16_bits(v);
  }
}

// An FP64 result in the output dtype, rounded as the reference's casts round it: fp32
// once; fp16 once (torch's float64 -> float16 cast rounds once); bf16 through fp32 (the
// reference computes in fp32 and casts to bf16, and torch's float64 -> bfloat16 cast also
// goes through fp32, which keeps FP64 results a few ulps apart on the same side of a
// bf16 rounding midpoint).
template <int DT>
__device__ __forceinline__ void store_from_f64(void* base, int64_t i, double v) {
  if constexpr (DT == kF32) {
    static_cast<float*>(base)[i] = static_cast<float>(v);
  } else if constexpr (DT == kF16) {
    static_cast<_Float16*>(base)[i] = static_cast<_Float16>(f64_to_f32_odd(v));
  } else {
    static_cast<uint16_t*>(base)[i] = f32_to_bf16_bits(static_cast<float>(v));
  }
}

// ---- sequence metadata -----------------------------------------------------

// Sequence s such that cu[s] <= t < cu[s+1] (empty sequences are skipped).
// cu has nseq+1 nondecreasing entries with cu[0]=0 and cu[nseq]=T.
__device__ __forceinline__ int find_seq(const int32_t* __restrict__ cu, int nseq, int64_t t) {
  int lo = 0, hi = nseq;  // answer in [lo, hi)
  while (hi - lo > 1) {
    int mid = (lo + hi) >> 1;
    if (static_cast<int64_t>(cu[mid]) <= t) lo = mid; else hi = mid;
  }
  return lo;
}

// Largest index i in [0, n) with a[i] <= x, for nondecreasing a with a[0] <= x.
__device__ __forceinline__ int upper_index(const int32_t* __restrict__ a, int n, int64_t x) {
  int lo = 0, hi = n;
  while (hi - lo > 1) {
    int mid = (lo + hi) >> 1;
    if (static_cast<int64_t>(a[mid]) <= x) lo = mid; else hi = mid;
  }
  return lo;
}

// ---- wavefront reductions --------------------------------------------------

__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

__device__ __forceinline__ double wave_max_f64(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmax(v, __shfl_xor(v, o, kWave));
  return v;
}

__device__ __forceinline__ int wave_sum_i32(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    uint32_t lo = static_cast<uint32_t>(v), hi = static_cast<uint32_t>(v >> 32);
    uint32_t olo = __shfl_xor(lo, o, kWave), ohi = __shfl_xor(hi, o, kWave);
    uint64_t other = (static_cast<uint64_t>(ohi) << 32) | olo;
    v = other > v ? other : v;
  }
  return v;
}

inline int status_from(hipError_t e) { return e == hipSuccess ? kOk : kErrLaunch; }

inline unsigned grid_1d(int64_t work, int per_block) {
  int64_t g = (work + per_block - 1) / per_block;
  return static_cast<unsigned>(g < 1 ? 1 : g);
}

}  // namespace msa
