// mx_device.hpp -- gfx950 device helpers: e2m1 / e8m0 decoding, bf16 splitting, wave reductions.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace burnext {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte load of weights read once per forward (nontemporal: the load does not keep the line in
// the caches for reuse; the expert GEMVs measured 2-2.5% shorter with it at 20B T = 8)
__device__ __forceinline__ uint4 load_stream16(const void *p) {
  const u32x4_t v = __builtin_nontemporal_load((const u32x4_t *)p);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

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

// The same rounding for two values in one instruction (gfx950's v_cvt_pk_bf16_f32, first value in
// the low half), checked on all 2^32 inputs against f32_to_bf16_bits.  Used by the activation
// splits of the GEMV stagings only.
typedef __bf16 bf16x2_hw_t __attribute__((ext_vector_type(2)));
typedef float f32x2_hw_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_bits(float lo, float hi) {
  const f32x2_hw_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_hw_t));
}

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) { return __uint_as_float(((uint32_t)b) << 16); }

// Split an f32 into NT bf16 terms t0 + t1 + ... (each the rounded residual of the previous).
// NT = 2 keeps ~2^-17 relative, NT = 3 any normal float to within 2^-24; NT = 1 is plain rounding.
template <int NT>
__device__ __forceinline__ void split_bf16(float v, uint16_t (&t)[NT]) {
  float r = v;
#pragma unroll
  for (int i = 0; i < NT; ++i) {
    t[i] = f32_to_bf16_bits(r);
    r = r - bf16_bits_to_f32(t[i]);
  }
}

// The same split for two values at once: term i of (lo, hi) packed as one bf16 pair, lo in the low
// half.
template <int NT>
__device__ __forceinline__ void split_bf16x2(float lo, float hi, uint32_t (&t)[NT]) {
  float r0 = lo, r1 = hi;
#pragma unroll
  for (int i = 0; i < NT; ++i) {
    t[i] = f32x2_to_bf16x2_bits(r0, r1);
    r0 = r0 - __uint_as_float(t[i] << 16);
    r1 = r1 - __uint_as_float(t[i] & 0xFFFF0000u);
  }
}


// Reductions of N values at once over the 64 lanes of a wave, valid in lane 0 only, without an LDS
// round trip: the xor-32 and xor-16 levels by permlane swaps, xor 8 by a row rotation (exact), and
// the xor-4/2/1 levels by a row rotation and quad permutations that pair lane l < 4 with l ^ 4,
// l ^ 2, l ^ 1 -- every operation lane 0's chain depends on combines the same two values, in the
// same operand order, as the butterfly's (so lane 0 ends with the butterfly's bits).  The N chains
// are interleaved level by level.
template <int CTRL> __device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int N, typename Op>
__device__ __forceinline__ void wave_reduce_to_lane0_n(float (&v)[N], Op op) {
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[i]), __float_as_uint(v[i]), false, false);
    v[i] = op(__uint_as_float(p[0]), __uint_as_float(p[1]));
  }
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[i]), __float_as_uint(v[i]), false, false);
    v[i] = op(__uint_as_float(p[0]), __uint_as_float(p[1]));
  }
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = op(v[i], dpp_mov<0x128>(v[i]));  // row_ror:8
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = op(v[i], dpp_mov<0x124>(v[i]));  // row_ror:4
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = op(v[i], dpp_mov<0x4E>(v[i]));   // quad_perm [2,3,0,1]
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = op(v[i], dpp_mov<0xB1>(v[i]));   // quad_perm [1,0,3,2]
}
template <int N>
__device__ __forceinline__ void wave_sum_to_lane0_n(float (&v)[N]) {
  wave_reduce_to_lane0_n(v, [](float a, float b) { return a + b; });
}
template <int N>
__device__ __forceinline__ void wave_max_to_lane0_n(float (&v)[N]) {
  wave_reduce_to_lane0_n(v, [](float a, float b) { return fmaxf(a, b); });
}
__device__ __forceinline__ float lane0_broadcast(float v) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
}

// Sum over the 64 lanes of a wave, in every lane, with the bits of the xor butterfly (after step
// `off` = 32 .. 1 lane l holds p[l] + p[l ^ off]; IEEE addition is commutative, so every lane
// finishes with lane 0's bits): lane 0's chain (wave_sum_to_lane0_n), broadcast from lane 0.
// Every lane of the wave must be active.
__device__ __forceinline__ float wave_sum_butterfly(float p) {
  float v[1] = {p};
  wave_sum_to_lane0_n<1>(v);
  return lane0_broadcast(v[0]);
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

// ---------------------------------------------------------------------------------------------
// MXFP8 (OCP e4m3fn with one e8m0 scale per 32 values), as the block-scaled MFMA reads it.
// A value v of a block with scale byte sb is stored as e4m3(v * 2^(127 - sb)).  The scale of a
// block is the smallest power of two that brings the block's largest magnitude to <= 448 (the
// largest finite e4m3fn value), so every code is finite; an all-zero block gets scale byte 0.
// The grouped GEMM carries activations as two terms: hi in this format and lo = the residual
// x - hi in MXFP4 at its own block scale (below), about 2^-6 relative per value at worst, where
// one e4m3 term alone (2^-4) is not accurate enough.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ uint32_t mx8_scale_byte(float amax) {
  const uint32_t u = __float_as_uint(amax);
  const uint32_t be = (u >> 23) & 0xFFu;  // biased exponent: amax = m * 2^(be - 127), m in [1, 2)
  if (amax <= 0.0f || be == 0u) return 0u;
  const uint32_t adj = (u & 0x7FFFFFu) > 0x600000u ? 1u : 0u;  // m > 1.75: m * 256 > 448
  const int sb = (int)be - 8 + (int)adj;
  return (uint32_t)min(max(sb, 1), 253);
}

// 2^(127 - sb) for sb in [1, 253] (exact), the multiplier that applies the inverse scale.
__device__ __forceinline__ float mx8_inv_scale(uint32_t sb) { return __uint_as_float((254u - sb) << 23); }

// Two floats -> two e4m3fn codes (round to nearest even) in the low 16 bits.
__device__ __forceinline__ uint32_t f32x2_to_fp8x2(float a, float b) {
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xFFFFu;
}

// e4m3fn code (byte SEL of w) -> float.
template <int SEL>
__device__ __forceinline__ float fp8_to_f32(uint32_t w) {
  return __builtin_amdgcn_cvt_f32_fp8((int)w, SEL);
}

// ---------------------------------------------------------------------------------------------
// MXFP4 (OCP e2m1, one e8m0 scale per 32 values) for the low term of the GEMM activations.  A
// block of residuals with largest magnitude amax gets the smallest power of two 2^(sb - 127) that
// brings amax to <= 6 (the largest e2m1 magnitude); an all-zero block gets scale byte 0.  Codes
// round to nearest even and saturate at 6; bit 3 is the sign.  Two codes per byte, the even K
// index in the low nibble (the MFMA's fp4 operand order).
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ uint32_t mx4_scale_byte(float amax) {
  const uint32_t u = __float_as_uint(amax);
  const uint32_t be = (u >> 23) & 0xFFu;  // amax = m * 2^(be - 127), m in [1, 2)
  if (amax <= 0.0f || be == 0u) return 0u;
  const uint32_t adj = (u & 0x7FFFFFu) > 0x400000u ? 1u : 0u;  // m > 1.5: amax / 2^(be-129) > 6
  const int sb = (int)be - 2 + (int)adj;
  return (uint32_t)min(max(sb, 1), 253);
}

// Two e2m1 codes, of a / s (low nibble) and b / s, into byte SEL of w (s = the block scale 2^k as
// f32, a normal number): gfx950's scaled convert, which rounds to nearest with ties to the even
// code (the midpoints 0.25, 0.75, ..., 5 between the magnitudes 0, 0.5, 1, 1.5, 2, 3, 4, 6 decide)
// and saturates magnitudes above 6 to 6 (measured against a comparison encoder on every f32 of
// [-8, 8) in steps of 2^-13 at five scales; only a NaN input differs: code 7).
template <int SEL>
__device__ __forceinline__ uint32_t e2m1x2(uint32_t w, float a, float b, float s) {
  return __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, a, b, s, SEL);
}
// The f32 divisor of an MXFP4 block whose scale byte is sb (1.0 for sb = 0: such a block's values
// are zero or below 2^-126 and encode to code 0 either way).
__device__ __forceinline__ float mx4_divisor(uint32_t sb) { return sb ? e8m0_to_f32(sb) : 1.0f; }

// Clamped SwiGLU of one (gate, linear) pair (reference src/activation/mod.rs:5-45,
// src/quant/gpu.rs:140-145): g = min(g, limit), l = clamp(l, +-limit), g * sigmoid(alpha g) * (l + 1).
__device__ __forceinline__ float swiglu_clamp_f(float g, float l, float alpha, float limit) {
  const float xg = fminf(g, limit);
  const float xl = fmaxf(-limit, fminf(l, limit));
  const float sig = 1.0f / (1.0f + expf(-alpha * xg));
  return (xg * sig) * (xl + 1.0f);
}

// One block of 32 values (largest magnitude amax) -> the GEMM's two activation terms: 32 MXFP8
// hi codes (e4m3), 16 bytes of MXFP4 lo codes (e2m1 of the residual, two per byte; 16-byte
// aligned destinations) and the two scale bytes.
__device__ __forceinline__ void mx84_quantize32(const float (&v)[32], float amax, uint8_t *hi, uint8_t *lo,
                                                uint8_t *shi, uint8_t *slo) {
  const uint32_t sbh = mx8_scale_byte(amax);
  const float ih = sbh ? mx8_inv_scale(sbh) : 0.0f, sh = e8m0_to_f32(sbh);
  uint32_t wh[8];
  float r[32], rmax = 0.0f;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const uint32_t c = f32x2_to_fp8x2(v[2 * k] * ih, v[2 * k + 1] * ih);
    r[2 * k] = v[2 * k] - fp8_to_f32<0>(c) * sh;
    r[2 * k + 1] = v[2 * k + 1] - fp8_to_f32<1>(c) * sh;
    rmax = fmaxf(rmax, fmaxf(fabsf(r[2 * k]), fabsf(r[2 * k + 1])));
    if (k & 1) wh[k >> 1] |= c << 16; else wh[k >> 1] = c;
  }
  const uint32_t sbl = mx4_scale_byte(rmax);
  const float sl = mx4_divisor(sbl);
  uint32_t w4[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t w = 0u;
    w = e2m1x2<0>(w, r[8 * j], r[8 * j + 1], sl);
    w = e2m1x2<1>(w, r[8 * j + 2], r[8 * j + 3], sl);
    w = e2m1x2<2>(w, r[8 * j + 4], r[8 * j + 5], sl);
    w4[j] = e2m1x2<3>(w, r[8 * j + 6], r[8 * j + 7], sl);
  }
  *(uint4 *)hi = make_uint4(wh[0], wh[1], wh[2], wh[3]);
  *(uint4 *)(hi + 16) = make_uint4(wh[4], wh[5], wh[6], wh[7]);
  *(uint4 *)lo = make_uint4(w4[0], w4[1], w4[2], w4[3]);
  *shi = (uint8_t)sbh;
  *slo = (uint8_t)sbl;
}

}  // namespace burnext
