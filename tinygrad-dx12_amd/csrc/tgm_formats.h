// Packed low-bit formats shared by every gfx950 kernel of this library.
//
// Storage contract (alexandreteles/tinygrad-dx12 src/tinygrad_dx12/codegen/decomp/dx12.py:69-77,
// ARCHITECTURE.md:614-618): payloads form one continuous little-endian bit stream over
// the flattened row-major logical array; element i occupies bits [i*bits, i*bits+bits).
// For 4-bit formats byte j holds elements 2j (low nibble) and 2j+1 (high nibble); for
// 6-bit formats three bytes hold four elements.
//
// Value contract (dx12.py:93-100): int4 = two's complement nibble, uint4 = nibble,
// floats: s | e | f with value (-1)^s * sig * 2^((e ? e : 1) - bias - p), sig = e ? f + 2^p : f.
// All encodings are finite and -0 is kept.
#pragma once

#include <stdint.h>

#include "../../include/tgm_packed.h"

#if defined(__HIPCC__)
#define TGM_HD __host__ __device__ __forceinline__
#else
#define TGM_HD static inline
#endif

namespace tgm {

struct FormatInfo {
  int bits, exp_bits, man_bits, bias;
};

TGM_HD FormatInfo format_info(int fmt) {
  switch (fmt) {
    case TGM_FMT_INT4: return {4, 0, 0, 0};
    case TGM_FMT_UINT4: return {4, 0, 0, 0};
    case TGM_FMT_FP4_E2M1: return {4, 2, 1, 1};
    case TGM_FMT_FP6_E2M3: return {6, 2, 3, 1};
    case TGM_FMT_FP6_E3M2: return {6, 3, 2, 3};
    default: return {0, 0, 0, 0};
  }
}

TGM_HD bool is_int_format(int fmt) { return fmt == TGM_FMT_INT4 || fmt == TGM_FMT_UINT4; }

// Payload of element ``idx``: two bytes always cover a payload of at most 6 bits that
// starts at bit offset <= 7 inside its first byte.  Bytes beyond ``nbytes`` read as zero,
// which is the zero padding of dx12.py:72.
TGM_HD uint32_t payload_at(const uint8_t* data, int64_t nbytes, int64_t idx, int bits) {
  const int64_t bit = idx * bits;
  const int64_t byte = bit >> 3;
  const int shift = (int)(bit & 7);
  uint32_t lo = byte < nbytes ? data[byte] : 0u;
  uint32_t hi = byte + 1 < nbytes ? data[byte + 1] : 0u;
  return ((lo | (hi << 8)) >> shift) & ((1u << bits) - 1u);
}

// Exact fp32 value of a float payload, built from bit fields (no exp2 call).
TGM_HD float decode_float(uint32_t p, FormatInfo f) {
  const uint32_t man_mask = (1u << f.man_bits) - 1u;
  const uint32_t frac = p & man_mask;
  const uint32_t e = (p >> f.man_bits) & ((1u << f.exp_bits) - 1u);
  // sig * 2^((e?e:1) - bias - p): every value is a small integer times a power of two.
  const float sig = (float)(e ? (frac | (1u << f.man_bits)) : frac);
  const int pw = (int)(e ? e : 1u) - f.bias - f.man_bits;  // in [-4, 2] for these formats
  float scale = 1.0f;
  if (pw >= 0) scale = (float)(1u << pw); else scale = 1.0f / (float)(1u << (-pw));
  const float mag = sig * scale;
  return (p >> (f.bits - 1)) & 1u ? -mag : mag;
}

TGM_HD int32_t decode_int(uint32_t p, int fmt) {
  return fmt == TGM_FMT_INT4 ? (int32_t)((p ^ 8u)) - 8 : (int32_t)p;
}

// Unscaled FP4/FP6 payload re-encoded as an FP8 byte (dx12.py:78-92).
// target_man/target_bias are (3,7) for E4M3FN and (2,15) for E5M2.
TGM_HD uint8_t fp8_direct(uint32_t p, FormatInfo f, int target_man, int target_bias) {
  const uint32_t fraction = p & ((1u << f.man_bits) - 1u);
  const uint32_t exponent = (p >> f.man_bits) & ((1u << f.exp_bits) - 1u);
  uint32_t mag;
  if (exponent == 0) {
    mag = 0;
    for (int high = 0; high < f.man_bits; ++high) {
      if (fraction >= (1u << high)) {
        mag = ((uint32_t)(target_bias + 1 - f.bias - f.man_bits + high) << target_man) |
              ((fraction << (target_man - high)) & ((1u << target_man) - 1u));
      }
    }
  } else {
    mag = ((exponent + target_bias - f.bias) << target_man) | (fraction << (target_man - f.man_bits));
  }
  return (uint8_t)((((p >> (f.bits - 1)) & 1u) << 7) | mag);
}

// E8M0 (OCP MX) scale: 2^(e-127); 0xFF is NaN.  e == 0 is the fp32 subnormal 2^-127.
TGM_HD float e8m0_to_float(uint32_t e) {
  union { uint32_t u; float f; } v;
  v.u = e == 0 ? 0x00400000u : (e == 255 ? 0x7FC00000u : (e << 23));
  return v.f;
}

// ---------------------------------------------------------------------- conversions
TGM_HD uint32_t f32_bits(float x) { union { float f; uint32_t u; } v; v.f = x; return v.u; }
TGM_HD float bits_f32(uint32_t x) { union { uint32_t u; float f; } v; v.u = x; return v.f; }
TGM_HD uint64_t f64_bits(double x) { union { double f; uint64_t u; } v; v.f = x; return v.u; }

// fp32 -> bf16 round-to-nearest-even in integer arithmetic; NaN stays a quiet NaN (payload's
// upper bits kept, bit 6 set).
TGM_HD uint16_t f32_to_bf16_int(float x) {
  const uint32_t u = f32_bits(x);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
#if defined(__HIPCC__)
// On the device the same rounding is one v_cvt_pk_bf16_f32 (gfx950), which rounds a pair at once;
// tgm_probe_bf16_rounding compares it with f32_to_bf16_int over every fp32 bit pattern.
typedef __bf16 tgm_bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t bf16x2_bits(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, tgm_bf16x2{(__bf16)lo, (__bf16)hi});
}
__device__ __forceinline__ uint16_t f32_to_bf16(float x) { return (uint16_t)(bf16x2_bits(x, 0.0f) & 0xFFFFu); }
__host__ inline uint16_t f32_to_bf16(float x) { return f32_to_bf16_int(x); }
#else
static inline uint16_t f32_to_bf16(float x) { return f32_to_bf16_int(x); }
#endif
TGM_HD float bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

// Generic IEEE-style narrowing of a double to a small float format with RNE.
// exp_bits/man_bits/bias describe the target; has_inf selects IEEE (E5M2/F16) vs
// OCP E4M3FN (no infinities, saturating here to +-max finite, NaN = 0x7F).
// Used for fp16 and fp8 results so that the rounding is single and identical to the oracle.
TGM_HD uint32_t narrow_rne(double x, int exp_bits, int man_bits, int bias, bool fn) {
  const uint64_t u = f64_bits(x);
  const uint32_t sign = (uint32_t)(u >> 63);
  const uint32_t total = 1 + exp_bits + man_bits;
  const uint32_t sign_bit = sign << (total - 1);
  const uint32_t exp_all = (1u << exp_bits) - 1u;
  const bool isnan = ((u >> 52) & 0x7FF) == 0x7FF && (u & 0xFFFFFFFFFFFFFull);
  if (isnan) return fn ? (sign_bit | (exp_all << man_bits) | ((1u << man_bits) - 1u))
                       : (sign_bit | (exp_all << man_bits) | (1u << (man_bits - 1)));
  // max finite magnitude encoding
  const uint32_t max_enc = fn ? ((exp_all << man_bits) | ((1u << man_bits) - 2u))
                              : (((exp_all - 1u) << man_bits) | ((1u << man_bits) - 1u));
  const uint32_t inf_enc = fn ? max_enc : (exp_all << man_bits);
  const double a = x < 0 ? -x : x;
  if (a == 0.0) return sign_bit;
  if (((u >> 52) & 0x7FF) == 0x7FF) return sign_bit | inf_enc;  // infinity
  // exponent of a (unbiased) and scaled significand
  int e = (int)((u >> 52) & 0x7FF) - 1023;
  const int emin = 1 - bias;  // smallest normal exponent
  int q_exp = e < emin ? emin : e;  // quantum exponent = q_exp - man_bits
  // q = a / 2^(q_exp - man_bits), exact in double because the shift is a power of two
  double q = a;
  int sh = q_exp - man_bits;
  // multiply by 2^-sh using repeated scaling to stay exact
  while (sh > 60) { q *= 0x1p-60; sh -= 60; }
  while (sh < -60) { q *= 0x1p60; sh += 60; }
  q *= (sh >= 0) ? 1.0 / (double)(1ull << sh) : (double)(1ull << (-sh));
  // round q to integer, ties to even
  double fl = (double)(uint64_t)q;
  double rem = q - fl;
  uint64_t n = (uint64_t)fl;
  if (rem > 0.5 || (rem == 0.5 && (n & 1))) n += 1;
  // renormalise: n in [0, 2^(man+1)]
  uint32_t enc;
  if (n == 0) return sign_bit;
  if (e < emin && n < (1ull << man_bits)) {
    enc = (uint32_t)n;  // subnormal
  } else {
    int be = q_exp + bias;
    if (n >= (2ull << man_bits)) { n >>= 1; be += 1; }
    if (n < (1ull << man_bits)) { be = 0; }
    enc = ((uint32_t)be << man_bits) | ((uint32_t)n & ((1u << man_bits) - 1u));
    if (fn) {
      if (enc > max_enc) enc = max_enc;
    } else if ((uint32_t)be >= exp_all) {
      enc = inf_enc;
    }
  }
  return sign_bit | enc;
}

TGM_HD uint16_t to_f16_bits(double x) { return (uint16_t)narrow_rne(x, 5, 10, 15, false); }
TGM_HD uint8_t to_fp8e4m3(double x) { return (uint8_t)narrow_rne(x, 4, 3, 7, true); }
// E5M2 results saturate to +-max finite like E4M3FN (tinygrad's fp8 casts clamp).
TGM_HD uint8_t to_fp8e5m2(double x) {
  const double m = 57344.0;
  if (x > m) x = m;
  if (x < -m) x = -m;
  return (uint8_t)narrow_rne(x, 5, 2, 15, false);
}

TGM_HD float f16_bits_to_f32(uint16_t h) {
  const uint32_t s = (uint32_t)(h >> 15) << 31;
  const uint32_t e = (h >> 10) & 0x1F, m = h & 0x3FF;
  if (e == 0) {
    float v = (float)m * 0x1p-24f;
    return s ? -v : v;
  }
  if (e == 31) return bits_f32(s | 0x7F800000u | (m << 13));
  return bits_f32(s | ((e + 112u) << 23) | (m << 13));
}

TGM_HD double fp8_bits_to_double(uint8_t b, int man_bits, int bias, bool fn) {
  const int e_bits = 7 - man_bits;
  const uint32_t frac = b & ((1u << man_bits) - 1u);
  const uint32_t e = (b >> man_bits) & ((1u << e_bits) - 1u);
  double v;
  if (fn && (b & 0x7F) == 0x7F) v = __builtin_nan("");
  else if (!fn && e == (1u << e_bits) - 1u) v = frac ? __builtin_nan("") : __builtin_inf();
  else if (e == 0) v = (double)frac * __builtin_ldexp(1.0, 1 - bias - man_bits);
  else v = (double)(frac | (1u << man_bits)) * __builtin_ldexp(1.0, (int)e - bias - man_bits);
  return (b & 0x80) ? -v : v;
}

}  // namespace tgm
