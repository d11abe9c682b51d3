// MFMA fragment helpers shared by the gfx950 kernels (v_mfma_f32_16x16x32_bf16).
//
// Lane l (c = l % 16, q4 = l / 16) holds A[c][8*q4 + j], B[8*q4 + j][c] (j = 0..7)
// and C[4*q4 + i][c] (i = 0..3). Fragments are assembled in 32-bit words: the
// 8-wide __bf16 vector type is only used as the MFMA operand container (element
// extraction from it is avoided: it yields element 0 for every index on this
// toolchain).
#pragma once
#include "common.hpp"

namespace msa {

__device__ __forceinline__ bf16x8 zero_frag() { return __builtin_bit_cast(bf16x8, make_uint4(0u, 0u, 0u, 0u)); }

__device__ __forceinline__ bf16x8 load_frag(const uint16_t* __restrict__ p) {
  const uint4 raw = *reinterpret_cast<const uint4*>(p);
  return __builtin_bit_cast(bf16x8, raw);
}

__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Exact split of an fp32 value into three bf16 terms by truncation: hi keeps the
// top 8 significant bits of x, mid the top 8 of x - hi, lo the remaining <= 8
// bits, so x == hi + mid + lo exactly (24 = 3 x 8) for normal x. The terms are
// returned as fp32 bit patterns whose low 16 bits are ignored by pack_hi16.
__device__ __forceinline__ void split3_bits(float x, uint32_t& hi, uint32_t& mid, uint32_t& lo) {
  hi = __float_as_uint(x);
  const float r1 = x - __uint_as_float(hi & 0xffff0000u);
  mid = __float_as_uint(r1);
  lo = __float_as_uint(r1 - __uint_as_float(mid & 0xffff0000u));
}

// One 32-bit word holding the bf16 truncations (upper halves) of a (low half) and b (high half).
__device__ __forceinline__ uint32_t pack_hi16(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

// gfx950 LDS transpose read (ds_read_b64_tr_b16). Within each 16-lane group the
// lanes' 8-byte reads form M[lane][e] (e = 0..3), and lane 4a + b receives
// M[4j + a][b] as element j. For a row-major tile T[k][n], a lane (c = lane % 16)
// pointing at &T[k0 + c/4][n0 + 4 (c%4)] therefore receives T[k0 + j][n0 + c]:
// the MFMA operand layout (n = c, 4 consecutive k) of the transposed tile.
typedef short v4i16 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint2 lds_read_tr16(const uint16_t* p) {
  const v4i16 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((v4i16 __attribute__((address_space(3)))*)(p));
  return __builtin_bit_cast(uint2, r);
}

// Operand fragment from a row-major LDS tile T[k][n] (row stride `stride`): element
// j of lane (c, q4) is T[ka + j][n0 + c] for j < 4 and T[kb + j - 4][n0 + c] for j >= 4.
__device__ __forceinline__ bf16x8 frag_tr(const uint16_t* tile, int stride, int ka, int kb, int n0, int c) {
  const uint16_t* base = tile + (c >> 2) * stride + n0 + 4 * (c & 3);
  const uint2 lo = lds_read_tr16(base + ka * stride);
  const uint2 hi = lds_read_tr16(base + kb * stride);
  return __builtin_bit_cast(bf16x8, make_uint4(lo.x, lo.y, hi.x, hi.y));
}

// frag_tr with the two 8-byte read addresses of this lane given directly (for
// swizzled tiles): elements 0..3 from the read at lo, 4..7 from the read at hi.
__device__ __forceinline__ bf16x8 frag_tr_at(const uint16_t* lo_p, const uint16_t* hi_p) {
  const uint2 lo = lds_read_tr16(lo_p);
  const uint2 hi = lds_read_tr16(hi_p);
  return __builtin_bit_cast(bf16x8, make_uint4(lo.x, lo.y, hi.x, hi.y));
}

__device__ __forceinline__ float quad_max(float v) {
  v = fmaxf(v, __shfl_xor(v, 16, kWave));
  return fmaxf(v, __shfl_xor(v, 32, kWave));
}


}  // namespace msa
