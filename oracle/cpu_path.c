/*
 * C restatement of the reference's CPU matmul path for packed weights
 * (test infrastructure: the CPU baseline of bench.py and a second check of the
 * NumPy oracle; never linked into the product).
 *
 * Reference: alexandreteles/tinygrad-dx12 src/tinygrad_dx12/codegen/linalg.py:169-174 --
 * on a non-DX12 device every packed operand is decoded to the fp32 intermediate and
 * materialised (``x.unpack(intermediate).contiguous()``), then ordinary
 * ``lhs.matmul(rhs, dtype=fp32)`` runs.  Decoding follows codegen/decomp/dx12.py:69-106.
 * The same three steps are restated here: (1) materialise deq(W) in fp32, (2) fp32
 * accumulating GEMV/GEMM, (3) round the output once (RNE) to bf16 or fp16.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* (bits, exponent bits, mantissa bits, bias) per format id: int4, uint4, fp4_e2m1, fp6_e2m3, fp6_e3m2 */
static const int FMT[5][4] = {{4, 0, 0, 0}, {4, 0, 0, 0}, {4, 2, 1, 1}, {6, 2, 3, 1}, {6, 3, 2, 3}};

static float decode_one(uint32_t p, int fmt) {
  const int bits = FMT[fmt][0], eb = FMT[fmt][1], mb = FMT[fmt][2], bias = FMT[fmt][3];
  if (fmt == 0) return (float)((int32_t)(p ^ 8u) - 8);
  if (fmt == 1) return (float)p;
  const uint32_t frac = p & ((1u << mb) - 1u);
  const uint32_t e = (p >> mb) & ((1u << eb) - 1u);
  const float sig = (float)(e ? (frac + (1u << mb)) : frac);
  const float v = ldexpf(sig, (int)(e ? e : 1u) - bias - mb);
  return (p >> (bits - 1)) & 1u ? -v : v;
}

/* deq[i] for the flattened [rows, k] array: code * scale in fp32 (dx12.py:101-106).  Codes decode
 * through a table of every code's value (decode_one), as a vectorising CPU compiler would; byte-
 * aligned rows of 4-bit codes take two codes per byte, low nibble first. */
void oracle_dequant_f32(const uint8_t* data, int64_t nbytes, int fmt, int64_t rows, int64_t k,
                        const float* scales, int64_t block, float* out) {
  const int bits = FMT[fmt][0];
  const int64_t nblk = (k + block - 1) / block;
  float lut[64];
  for (uint32_t p = 0; p < (1u << bits); ++p) lut[p] = decode_one(p, fmt);
  if (bits == 4 && k % 2 == 0 && block % 2 == 0 && nbytes >= rows * k / 2) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
      const uint8_t* src = data + r * k / 2;
      float* dst = out + r * k;
      for (int64_t b = 0; b < nblk; ++b) {
        const float sc = scales ? scales[r * nblk + b] : 1.0f;
        const int64_t c1 = (b + 1) * block < k ? (b + 1) * block : k;
        for (int64_t c = b * block; c < c1; c += 2) {
          const uint8_t v = src[c / 2];
          dst[c] = lut[v & 15u] * sc;
          dst[c + 1] = lut[v >> 4] * sc;
        }
      }
    }
    return;
  }
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t c = 0; c < k; ++c) {
      const int64_t i = r * k + c, bit = i * bits, byte = bit >> 3;
      const uint32_t lo = byte < nbytes ? data[byte] : 0u, hi = byte + 1 < nbytes ? data[byte + 1] : 0u;
      const uint32_t p = ((lo | (hi << 8)) >> (bit & 7)) & ((1u << bits) - 1u);
      float v = lut[p];
      if (scales) v = v * scales[r * nblk + c / block];
      out[i] = v;
    }
  }
}

/* y[m, n] = sum_k x[m, k] * w[n, k] in fp32: 16 interleaved partial sums per output (lane l
 * takes k = l mod 16), added pairwise at the end -- the split-accumulator order a vectorising
 * CPU compiler gives a long dot product. */
#define ACC_LANES 16
void oracle_linear_f32(const float* w, const float* x, int64_t m, int64_t n, int64_t k, float* y) {
#pragma omp parallel for schedule(static) collapse(2)
  for (int64_t i = 0; i < m; ++i) {
    for (int64_t j = 0; j < n; ++j) {
      const float* wr = w + j * k;
      const float* xr = x + i * k;
      float acc[ACC_LANES] = {0.f};
      int64_t t = 0;
      for (; t + ACC_LANES <= k; t += ACC_LANES)
        for (int l = 0; l < ACC_LANES; ++l) acc[l] += xr[t + l] * wr[t + l];
      for (int l = 0; t < k; ++t, ++l) acc[l] += xr[t] * wr[t];
      for (int h = ACC_LANES / 2; h > 0; h /= 2)
        for (int l = 0; l < h; ++l) acc[l] += acc[l + h];
      y[i * n + j] = acc[0];
    }
  }
}

static uint16_t f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

/* IEEE binary32 -> binary16, round to nearest even, overflow to infinity. */
static uint16_t f32_to_f16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint32_t sign = (u >> 16) & 0x8000u;
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);
  if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 rounds to inf */
  if (a < 0x38800000u) {                                  /* below 2^-14: subnormal or zero */
    const float q = ldexpf(fabsf(f), 24);                 /* exact: units of 2^-24 */
    const float r = nearbyintf(q);                        /* default mode is RNE */
    return (uint16_t)(sign | (uint32_t)r);
  }
  const uint32_t mant = a & 0x7FFFFFu, e = (a >> 23) - 112u;
  uint32_t h = (e << 10) | (mant >> 13);
  const uint32_t rem = mant & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
  return (uint16_t)(sign | h);
}

void oracle_round_bf16(const float* x, int64_t n, uint16_t* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = f32_to_bf16(x[i]);
}

void oracle_round_f16(const float* x, int64_t n, uint16_t* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = f32_to_f16(x[i]);
}

/* The whole CPU path: deq(W) materialised, fp32 GEMV/GEMM, RNE to ``out_bits`` (16 = bf16, 17 = fp16). */
void oracle_cpu_path(const uint8_t* data, int64_t nbytes, int fmt, int64_t n, int64_t k, const float* scales,
                     int64_t block, const float* x, int64_t m, float* wdeq, float* yf, uint16_t* y, int out_kind) {
  oracle_dequant_f32(data, nbytes, fmt, n, k, scales, block, wdeq);
  oracle_linear_f32(wdeq, x, m, n, k, yf);
  if (out_kind == 16) oracle_round_bf16(yf, m * n, y);
  else oracle_round_f16(yf, m * n, y);
}
