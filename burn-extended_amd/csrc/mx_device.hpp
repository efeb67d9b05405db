// mx_device.hpp -- gfx950 device helpers: e2m1 / e8m0 decoding, bf16 splitting, wave reductions.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace burnext {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// 2^(s-127) for an e8m0 exponent byte, built from bits: s = 0 is the subnormal 2^-127,
// s = 255 is +inf -- the values (2.0f32).powi(s - 127) gives (reference src/loader/mxfp4.rs:46,68).
__device__ __forceinline__ float e8m0_to_f32(uint32_t s) {
  return __uint_as_float(s == 0u ? 0x00400000u : (s << 23));
}

// e2m1 code -> float (reference LUT src/loader/mxfp4.rs:11-13): magnitude bits e1 e0 m give
// 2^(e-1) * (1 + m/2) for e >= 1 and m/2 for e = 0; bit 3 is the sign (code 8 is -0.0).
__device__ __forceinline__ float fp4_to_f32(uint32_t nib) {
  const uint32_t mag = nib & 7u;
  const uint32_t bits =
      mag == 0u ? 0u : (mag == 1u ? 0x3F000000u : ((((mag >> 1) + 126u) << 23) | ((mag & 1u) << 22)));
  return __uint_as_float(bits | ((nib & 8u) << 28));
}

// float -> bf16 bits, round to nearest even (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) { return __uint_as_float(((uint32_t)b) << 16); }

// Split an f32 into NT bf16 terms t0 + t1 + ... (each the rounded residual of the previous).
// NT = 3 reproduces any normal float to within 2^-24 relative; NT = 1 is plain rounding.
template <int NT>
__device__ __forceinline__ void split_bf16(float v, uint16_t (&t)[NT]) {
  float r = v;
#pragma unroll
  for (int i = 0; i < NT; ++i) {
    t[i] = f32_to_bf16_bits(r);
    r = r - bf16_bits_to_f32(t[i]);
  }
}

// Butterfly sum over the 64 lanes of a wave: after step `off` lane l holds p[l] + p[l ^ off].
// IEEE addition is commutative, so all lanes finish with the same bits.
__device__ __forceinline__ float wave_sum_butterfly(float p) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) p = p + __shfl_xor(p, off, 64);
  return p;
}

// Packed top-k key with the same strict total order as `beats`: a beats b iff key(a) > key(b)
// (unsigned).  High word: order-preserving map of the float with NaN -> 0 (lowest) and -0 -> +0;
// low word: ~index, so equal values rank the lower index first.
__device__ __forceinline__ uint64_t topk_key(float v, uint32_t idx) {
  const uint32_t u = __float_as_uint(v);
  uint32_t k;
  if (v != v)
    k = 0u;
  else if (v == 0.0f)
    k = 0x80000000u;
  else
    k = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)k << 32) | (uint64_t)(0xFFFFFFFFu - idx);
}

// Strict total order for top-k: larger value first, NaN lowest, ties to the lower index.
__device__ __forceinline__ bool beats(float va, int ia, float vb, int ib) {
  const bool na = va != va, nb = vb != vb;
  if (na || nb) return (na && nb) ? (ia < ib) : nb;
  if (va > vb) return true;
  if (va < vb) return false;
  return ia < ib;
}

// Two e2m1 codes of byte `sel` of `w`, times `scale`, as a bf16 pair (exact for e8m0 scales).
#define BURNEXT_CVT_FP4x2_BF16(w, scale, sel) __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4((w), (scale), (sel))

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Two e2m1 codes of byte `sel` of `w` scaled, as the 32-bit word (low half = low nibble).
// Pairs are moved as 32-bit words: hipcc 7.2 miscompiles a store of element [1] of a __bf16
// ext_vector (it emits a store of the low half), so no code here extracts __bf16 elements.
template <int SEL>
__device__ __forceinline__ uint32_t fp4x2_to_bf16x2_bits(uint32_t w, float scale) {
  return __builtin_bit_cast(uint32_t, BURNEXT_CVT_FP4x2_BF16(w, scale, SEL));
}

// 8 consecutive e2m1 codes (one dword, low nibble first) scaled -> 8 bf16 in order.
__device__ __forceinline__ bf16x8_t fp4x8_to_bf16x8(uint32_t w, float scale) {
  const u32x4_t r = {fp4x2_to_bf16x2_bits<0>(w, scale), fp4x2_to_bf16x2_bits<1>(w, scale),
                     fp4x2_to_bf16x2_bits<2>(w, scale), fp4x2_to_bf16x2_bits<3>(w, scale)};
  return __builtin_bit_cast(bf16x8_t, r);
}

}  // namespace burnext
