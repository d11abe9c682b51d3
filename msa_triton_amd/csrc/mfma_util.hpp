// MFMA fragment helpers shared by the gfx950 kernels (v_mfma_f32_16x16x32_bf16 and its
// fp16 form v_mfma_f32_16x16x32_f16).
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

typedef __bf16 bf16x2_pk __attribute__((ext_vector_type(2)));
typedef float f32x2_pk __attribute__((ext_vector_type(2)));

// Two fp32 values rounded to nearest bf16, packed (x0 in the low half): v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t cvt_pk_bf16(float x0, float x1) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_pk){x0, x1}, bf16x2_pk));
}

// x - (bf16 half of w) as one v_dot2_f32_bf16 against (-1, -0): the products are -h and
// +-0 (exact) and the difference is representable (below), so the result is exact. The
// other half is -0, not +0: the word (-1 in the low half, +0 high) would be emitted as the
// inline constant -1.0, which the hardware reads as the fp32 pattern (-1 in the high half).
__device__ __forceinline__ float sub_lo_half(uint32_t w, float x) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_pk, w), __builtin_bit_cast(bf16x2_pk, 0x8000bf80u), x,
                                         false);
}
__device__ __forceinline__ float sub_hi_half(uint32_t w, float x) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_pk, w), __builtin_bit_cast(bf16x2_pk, 0xbf808000u), x,
                                         false);
}

// Exact split of two fp32 values into three packed bf16 words by round-to-nearest:
// hi = rn(x), mid = rn(x - hi), lo = rn(x - hi - mid) with x0 in the low halves. For
// normal x: x - hi is a multiple of ulp(x) below half an ulp of hi (<= 16 significant
// bits, exact in fp32), x - hi - mid has <= 8 significant bits, so lo is exact and
// x == hi + mid + lo. Seven VALU operations per pair (packing included).
__device__ __forceinline__ void split3_pk(float x0, float x1, uint32_t& hi, uint32_t& mid, uint32_t& lo) {
  hi = cvt_pk_bf16(x0, x1);
  const float r0 = sub_lo_half(hi, x0), r1 = sub_hi_half(hi, x1);
  mid = cvt_pk_bf16(r0, r1);
  lo = cvt_pk_bf16(sub_lo_half(mid, r0), sub_hi_half(mid, r1));
}

// ---- fp16 operands (v_mfma_f32_16x16x32_f16: the fragment layout of the bf16 form; the
// bf16x8 container carries the 16-bit words unchanged)

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_pk __attribute__((ext_vector_type(2)));

// The MFMA of the input type DT (kBF16 or kF16): products exact in fp32 for both.
template <int DT>
__device__ __forceinline__ f32x4 mfma_t(bf16x8 a, bf16x8 b, f32x4 c) {
  if constexpr (DT == kF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  else
    return mfma(a, b, c);
}

// Two fp32 values rounded to nearest fp16, packed (x0 in the low half): v_cvt_pk_f16_f32.
__device__ __forceinline__ uint32_t cvt_pk_f16(float x0, float x1) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_pk){x0, x1}, f16x2_pk));
}

// x - (fp16 half of w) as one v_dot2_f32_f16 against (-1, -0): exact as in sub_lo_half.
__device__ __forceinline__ float sub_lo_half_f16(uint32_t w, float x) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_pk, w), __builtin_bit_cast(f16x2_pk, 0x8000bc00u), x, false);
}
__device__ __forceinline__ float sub_hi_half_f16(uint32_t w, float x) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_pk, w), __builtin_bit_cast(f16x2_pk, 0xbc008000u), x, false);
}

// Split of two fp32 values into three packed fp16 words by round-to-nearest: hi = rn(x),
// mid = rn(x - hi), lo = rn(x - hi - mid) (x0 in the low halves). x - hi and x - hi - mid
// are exact in fp32 (multiples of ulp(x) below half an ulp of the term before), and
// x == hi + mid + lo exactly when 2^-1 <= |x| <= 2^15: the last residual has <= 2
// significant bits on the grid of ulp(x) >= 2^-24, fp16's smallest subnormal. Below
// 2^-1 the error is at most 2^-25 (half that subnormal). Callers scale their values
// into that range by a power of two first (fp16's exponent range is 2^-24 .. 2^15).
__device__ __forceinline__ void split3_pk_f16(float x0, float x1, uint32_t& hi, uint32_t& mid, uint32_t& lo) {
  hi = cvt_pk_f16(x0, x1);
  const float r0 = sub_lo_half_f16(hi, x0), r1 = sub_hi_half_f16(hi, x1);
  mid = cvt_pk_f16(r0, r1);
  lo = cvt_pk_f16(sub_lo_half_f16(mid, r0), sub_hi_half_f16(mid, r1));
}

// The fp32 value of the low / high 16-bit element of w, read as the input type DT
// (scalar bit casts: no element extraction from 16-bit vector types).
template <int DT>
__device__ __forceinline__ float lo16_f32(uint32_t w) {
  if constexpr (DT == kF16)
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w)));
  else
    return __uint_as_float(w << 16);
}
template <int DT>
__device__ __forceinline__ float hi16_f32(uint32_t w) {
  if constexpr (DT == kF16)
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16)));
  else
    return __uint_as_float(w & 0xffff0000u);
}

// fp16 -> two bf16 terms, exactly: an fp16 value has 11 significant bits and its
// exponent range lies inside bf16's, so hi = rn_bf16(x) and lo = x - hi (<= 3 bits) are
// both exact. One 32-bit word of two fp16 values gives a word of his and one of los.
__device__ __forceinline__ void f16_pair_to_bf16_terms(uint32_t w, uint32_t& hi, uint32_t& lo) {
  const float x0 = lo16_f32<kF16>(w), x1 = hi16_f32<kF16>(w);
  hi = cvt_pk_bf16(x0, x1);
  lo = cvt_pk_bf16(sub_lo_half(hi, x0), sub_hi_half(hi, x1));
}

// Four FP64 results as four elements of DT (x0 lowest), each rounded as store_from_f64
// rounds it: bf16 through fp32, fp16 once (round-to-odd through fp32).
template <int DT>
__device__ __forceinline__ uint2 pack4_from_f64(double x0, double x1, double x2, double x3) {
  if constexpr (DT == kF16) {
    auto h = [](double x) {
      return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(f64_to_f32_odd(x))));
    };
    return make_uint2(h(x0) | (h(x1) << 16), h(x2) | (h(x3) << 16));
  } else {
    auto b = [](double x) { return static_cast<uint32_t>(f32_to_bf16_bits(static_cast<float>(x))); };
    return make_uint2(b(x0) | (b(x1) << 16), b(x2) | (b(x3) << 16));
  }
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
