// Device arithmetic of the fp8 cold store (include/barq_kv.h, barq_kv_cold): OCP FP8 E4M3 codes
// with power-of-two (E8M0) scales.  Shared by the compress / dequantising-gather kernels
// (barq_kv_quant.hip) and the decode-attention kernel reading quantised pages
// (barq_kv_attention.hip), so both produce the same dequantised bits.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "barq_kv.h"

namespace barq_fp8 {

// Element types of a pool, numbered as BARQ_KV_BF16 / BARQ_KV_FP16 / BARQ_KV_FP32.
template <int KIND>
struct Elem;
template <>
struct Elem<BARQ_KV_BF16> {
  using Bits = uint16_t;
  __device__ static float to_float(Bits b) { return __uint_as_float((uint32_t)b << 16); }
  __device__ static Bits from_float(float f) {  // round to nearest even, NaN kept quiet
    const uint32_t u = __float_as_uint(f);
    if (f != f) return (Bits)((u >> 16) | 0x40);
    return (Bits)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
  }
};
template <>
struct Elem<BARQ_KV_FP16> {
  using Bits = uint16_t;
  __device__ static float to_float(Bits b) { return (float)__builtin_bit_cast(_Float16, b); }
  __device__ static Bits from_float(float f) { return __builtin_bit_cast(Bits, (_Float16)f); }
};
template <>
struct Elem<BARQ_KV_FP32> {
  using Bits = uint32_t;
  __device__ static float to_float(Bits b) { return __uint_as_float(b); }
  __device__ static Bits from_float(float f) { return __float_as_uint(f); }
};

// E4M3 code of a float, rounded to nearest even; finite values beyond 448 saturate, NaN and
// infinities give the NaN code (with their sign).
__device__ __forceinline__ uint32_t e4m3_encode(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t sign = (u >> 24) & 0x80u;
  const float a = fabsf(x);
  if (!(a <= 3.402823466e38f)) return sign | 0x7Fu;
  if (a < 0.015625f) return sign | (uint32_t)rintf(a * 512.0f);  // subnormal codes 0..8
  const uint32_t au = u & 0x7FFFFFFFu;
  int e = (int)(au >> 23) - 127;
  uint32_t m = (au >> 20) & 7u;
  const uint32_t rem = au & 0xFFFFFu;
  if (rem > 0x80000u || (rem == 0x80000u && (m & 1u))) {
    if (++m == 8u) {
      m = 0;
      ++e;
    }
  }
  const int code = min(((e + 7) << 3) | (int)m, 0x7E);
  return sign | (uint32_t)code;
}

// Four E4M3 codes, x0 in the low byte, each exactly as e4m3_encode gives it, for values whose
// finite magnitudes are at most 464 (a quantised group's elements over its power-of-two scale
// are at most 448): gfx950's v_cvt_pk_fp8_f32 rounds to nearest even with the same subnormal
// and signed-zero codes -- checked against e4m3_encode on the GPU for every finite fp32 value up
// to 464 in magnitude (2,278,555,650 values, no difference) -- and a group holding an infinity or
// a NaN takes e4m3_encode element by element.
__device__ __forceinline__ uint32_t e4m3_encode4(float x0, float x1, float x2, float x3) {
  constexpr float kMax = 3.402823466e38f;
  if (fabsf(x0) <= kMax && fabsf(x1) <= kMax && fabsf(x2) <= kMax && fabsf(x3) <= kMax) {
    const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(x0, x1, 0, false);
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(x2, x3, lo, true);
  }
  return e4m3_encode(x0) | (e4m3_encode(x1) << 8) | (e4m3_encode(x2) << 16) | (e4m3_encode(x3) << 24);
}

// The exact value of an E4M3 code; NaN codes give the quiet NaN with the code's sign.
__device__ __forceinline__ float e4m3_decode(uint32_t c) {
  const uint32_t c7 = c & 0x7Fu;
  const uint32_t sign = (c & 0x80u) << 24;
  if (c7 == 0x7Fu) return __uint_as_float(sign | 0x7FC00000u);
  const float mag = c7 >= 8u ? __uint_as_float((((c7 >> 3) + 120u) << 23) | ((c7 & 7u) << 20))
                             : (float)c7 * 0.001953125f;
  return __uint_as_float(__float_as_uint(mag) | sign);
}

// Smallest e with a <= 448 * 2^e (0 for a == 0), clamped to [-127, 127]: with a = m * 2^x,
// m in [0.5, 1), e = x - 9, plus 1 when m > 0.875 (448 = 0.875 * 2^9).
__device__ __forceinline__ int group_exponent(float a) {
  if (a == 0.0f) return 0;
  int x;
  const float m = frexpf(a, &x);
  return max(-127, min(127, x - 9 + (m > 0.875f ? 1 : 0)));
}

__device__ __forceinline__ float finite_abs(float v) {
  const float a = fabsf(v);
  return a <= 3.402823466e38f ? a : 0.0f;
}

// Fast dequantisation into two-byte values: a normal E4M3 code (exponent field E in 1..15) times
// 2^(s - 127) has the output exponent field E + s - kBias and the code's 3 mantissa bits on top
// of the output mantissa, so the bits are ((c & 0x7F) << kShift) + ((s - kBias) << kExpShift)
// with the sign moved to bit 15 -- two values per 32-bit word.  It applies when no code is zero,
// subnormal or NaN and every scale keeps every result a normal number (s in [kBias, kMaxScale]);
// otherwise the per-element path runs.  Both give the exact product, which the output type holds.
template <int KIND>
struct FastDeq;
template <>
struct FastDeq<BARQ_KV_BF16> {
  static constexpr uint32_t kShift = 4, kExpShift = 7, kBias = 7, kMaxScale = 254 - 15 + 7;
};
template <>
struct FastDeq<BARQ_KV_FP16> {
  static constexpr uint32_t kShift = 7, kExpShift = 10, kBias = 119, kMaxScale = 30 - 15 + 119;
};

__device__ __forceinline__ bool codes_normal(uint32_t w) {  // 4 codes: none zero/subnormal or NaN
  const uint32_t e = w & 0x78787878u;
  const uint32_t nan = (w & 0x7F7F7F7Fu) ^ 0x7F7F7F7Fu;
  const uint32_t any_zero = ((e - 0x01010101u) & ~e) | ((nan - 0x01010101u) & ~nan);
  return (any_zero & 0x80808080u) == 0;
}

__device__ __forceinline__ uint32_t spread_lo(uint32_t w) { return (w & 0xFFu) | ((w << 8) & 0xFF0000u); }
__device__ __forceinline__ uint32_t spread_hi(uint32_t w) { return ((w >> 16) & 0xFFu) | ((w >> 8) & 0xFF0000u); }

template <int KIND>
__device__ __forceinline__ uint32_t fast_pair(uint32_t codes2, uint32_t scales2) {
  using F = FastDeq<KIND>;
  const uint32_t bias = F::kBias | (F::kBias << 16);
  return (((codes2 & 0x007F007Fu) << F::kShift) + ((scales2 - bias) << F::kExpShift)) |
         ((codes2 & 0x00800080u) << 8);
}

template <int KIND>
__device__ __forceinline__ bool scale_fast(uint32_t s) {
  return s >= FastDeq<KIND>::kBias && s <= FastDeq<KIND>::kMaxScale;
}

template <int KIND>
__device__ __forceinline__ bool scales_fast4(uint32_t w) {  // 4 scale bytes
  return scale_fast<KIND>(w & 0xFFu) && scale_fast<KIND>((w >> 8) & 0xFFu) &&
         scale_fast<KIND>((w >> 16) & 0xFFu) && scale_fast<KIND>(w >> 24);
}

// 8 codes (two words) with 8 scale bytes (two words, one per code): may dequant8_fast decode them?
template <int KIND>
__device__ __forceinline__ bool dequant8_fast_ok(uint32_t c0, uint32_t c1, uint32_t s0, uint32_t s1) {
  return codes_normal(c0) && codes_normal(c1) && scales_fast4<KIND>(s0) && scales_fast4<KIND>(s1);
}

// 8 two-byte values (4 words, element 2i in the low half of word i) by exponent arithmetic.
template <int KIND>
__device__ __forceinline__ void dequant8_fast(uint32_t c0, uint32_t c1, uint32_t s0, uint32_t s1, uint32_t (&out)[4]) {
  out[0] = fast_pair<KIND>(spread_lo(c0), spread_lo(s0));
  out[1] = fast_pair<KIND>(spread_hi(c0), spread_hi(s0));
  out[2] = fast_pair<KIND>(spread_lo(c1), spread_lo(s1));
  out[3] = fast_pair<KIND>(spread_hi(c1), spread_hi(s1));
}

// The same values element by element, for any codes and scales (one out-of-line copy: the rare
// path must not cost the callers' registers).
template <int KIND>
__device__ __noinline__ uint32_t dequant2_exact(uint32_t codes2, uint32_t scales2) {
  using E = Elem<KIND>;
  const uint32_t lo = E::from_float(ldexpf(e4m3_decode(codes2 & 0xFFu), (int)(scales2 & 0xFFu) - 127));
  const uint32_t hi = E::from_float(ldexpf(e4m3_decode((codes2 >> 8) & 0xFFu), (int)((scales2 >> 8) & 0xFFu) - 127));
  return lo | (hi << 16);
}

// Two codes (low 16 bits of each word: code 0 in bits 0-7, code 1 in bits 8-15) with their
// scale bytes -> two two-byte values, exactly, for any codes and scales (inline).
template <int KIND>
__device__ __forceinline__ uint32_t dequant2_inline(uint32_t codes2, uint32_t scales2) {
  using E = Elem<KIND>;
  const uint32_t lo = E::from_float(ldexpf(e4m3_decode(codes2 & 0xFFu), (int)(scales2 & 0xFFu) - 127));
  const uint32_t hi = E::from_float(ldexpf(e4m3_decode((codes2 >> 8) & 0xFFu), (int)((scales2 >> 8) & 0xFFu) - 127));
  return lo | (hi << 16);
}

struct Words4 {
  uint32_t w[4];
};

// 8 codes element by element (one out-of-line copy).
template <int KIND>
__device__ __noinline__ Words4 dequant8_exact(uint32_t c0, uint32_t c1, uint32_t s0, uint32_t s1) {
  Words4 r;
  r.w[0] = dequant2_exact<KIND>(c0, s0);
  r.w[1] = dequant2_exact<KIND>(c0 >> 16, s0 >> 16);
  r.w[2] = dequant2_exact<KIND>(c1, s1);
  r.w[3] = dequant2_exact<KIND>(c1 >> 16, s1 >> 16);
  return r;
}

// 8 codes with their 8 scale bytes -> 8 two-byte values: exponent arithmetic when it applies
// (all but ~1 in 10^3 vectors of normally distributed data), else the exact element path.
template <int KIND>
__device__ __forceinline__ void dequant8(uint32_t c0, uint32_t c1, uint32_t s0, uint32_t s1, uint32_t (&out)[4]) {
  if (dequant8_fast_ok<KIND>(c0, c1, s0, s1)) {
    dequant8_fast<KIND>(c0, c1, s0, s1, out);
  } else {
    const Words4 r = dequant8_exact<KIND>(c0, c1, s0, s1);
    out[0] = r.w[0];
    out[1] = r.w[1];
    out[2] = r.w[2];
    out[3] = r.w[3];
  }
}

}  // namespace barq_fp8
