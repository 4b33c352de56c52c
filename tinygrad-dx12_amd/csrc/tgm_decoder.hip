// Decoder-step kernels for a Llama-style model on the packed matmul path (tgm_decoder.h).
//
// The reference has no model code; a decoder on it would be tinygrad ops around
// PackedTensor.matmul (alexandreteles/tinygrad-dx12 src/tinygrad_dx12/codegen/decomp/
// dx12.py:108-112).  These kernels are the layer's non-matmul work on gfx950: embedding
// gather, residual add fused with RMSNorm, RoPE fused with the KV-cache store, split-K
// grouped-query attention, SwiGLU, a bf16 GEMV for the output head and a greedy argmax
// that advances the sequence positions on the device.  Everything a step launches reads its
// position from device memory, so a decode step is the same launch sequence every time and
// can be replayed as a HIP graph.  Nothing here allocates or issues a memset.
#include <math.h>

#include "../../include/tgm_decoder.h"
#include "tgm_common.h"
#include "tgm_lanes.h"

namespace tgm {

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 dec_bf16x2;
typedef unsigned dec_u32x4 __attribute__((ext_vector_type(4)));
typedef float dec_f32x4 __attribute__((ext_vector_type(4)));

// Whole-wave reductions without LDS: DPP exchanges inside the 16-lane rows, then the gfx950
// row swaps (every lane ends with the result).  A __shfl_xor butterfly is six dependent
// ds_bpermute round trips through LDS.  All 64 lanes must be active.
__device__ __forceinline__ float wave_sum(float v) {
  v += xor1(v);
  v += xor2(v);
  v += xor4(v);
  v += xor8(v);
  float a = v, b = v;
  swap16(a, b);  // lane l: a + b = v[l] + v[l ^ 16]
  v = a + b;
  a = v, b = v;
  swap32(a, b);  // lane l: a + b = v[l] + v[l ^ 32]
  return a + b;
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, xor1(v));
  v = fmaxf(v, xor2(v));
  v = fmaxf(v, xor4(v));
  v = fmaxf(v, xor8(v));
  float a = v, b = v;
  swap16(a, b);
  v = fmaxf(a, b);
  a = v, b = v;
  swap32(a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float lo_bf16(unsigned w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) { return __builtin_bit_cast(float, (unsigned)h << 16); }
__device__ __forceinline__ float hi_bf16(unsigned w) { return __builtin_bit_cast(float, w & 0xFFFF0000u); }

// ------------------------------------------------------------------ embedding
// 16 bytes (8 bf16) of the table row per thread and pass, written as two float4.
__global__ void __launch_bounds__(512) dec_embed(const uint16_t* __restrict__ table, int64_t vocab, int d,
                                                 const int32_t* __restrict__ tokens, float* __restrict__ h) {
  const int64_t r = blockIdx.x;
  int64_t tok = tokens[r];
  if (tok < 0 || tok >= vocab) tok = 0;
  const uint16_t* src = table + tok * d;
  float* dst = h + r * d;
  for (int c = threadIdx.x; c < d / 8; c += 512) {
    const dec_u32x4 v = *(const dec_u32x4*)(src + 8 * c);
    *(dec_f32x4*)(dst + 8 * c) = dec_f32x4{lo_bf16(v[0]), hi_bf16(v[0]), lo_bf16(v[1]), hi_bf16(v[1])};
    *(dec_f32x4*)(dst + 8 * c + 4) = dec_f32x4{lo_bf16(v[2]), hi_bf16(v[2]), lo_bf16(v[3]), hi_bf16(v[3])};
  }
}

// ------------------------------------------------------------------ residual add + RMSNorm
// One workgroup of 1024 threads per row.  A row of up to 16384 floats stays in registers (four
// float4 per thread) between the sum of squares and the scaled store, so every element is
// loaded once; the loads of a thread are independent and issued together.
constexpr int kNormThreads = 1024, kNormMaxD = 4 * 4 * kNormThreads;

__device__ __forceinline__ void store4(void* out, int odt, int64_t i, dec_f32x4 y) {
  if (odt == TGM_F32) {
    *(dec_f32x4*)((float*)out + i) = y;
  } else if (odt == TGM_BF16) {
    *(uint2*)((uint16_t*)out + i) = uint2{f32_to_bf16(y[0]) | ((unsigned)f32_to_bf16(y[1]) << 16),
                                          f32_to_bf16(y[2]) | ((unsigned)f32_to_bf16(y[3]) << 16)};
  } else {
    *(uint2*)((uint16_t*)out + i) =
        uint2{__builtin_bit_cast(unsigned short, (_Float16)y[0]) | ((unsigned)__builtin_bit_cast(unsigned short, (_Float16)y[1]) << 16),
              __builtin_bit_cast(unsigned short, (_Float16)y[2]) | ((unsigned)__builtin_bit_cast(unsigned short, (_Float16)y[3]) << 16)};
  }
}

// h += the nparts deltas (part p at delta + p part_stride), then RMSNorm(h) * w -> out.
__global__ void __launch_bounds__(kNormThreads) dec_add_rmsnorm(float* __restrict__ h, const float* __restrict__ delta,
                                                                int nparts, int64_t part_stride, int d,
                                                                const uint16_t* __restrict__ w, float eps,
                                                                void* __restrict__ out, int odt) {
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int d4 = d >> 2;
  dec_f32x4* hr = (dec_f32x4*)(h + r * d);
  const dec_f32x4* dr = delta ? (const dec_f32x4*)(delta + r * d) : nullptr;
  dec_f32x4 v[4];
  // the norm weights are loaded with the row, not after the reduction: one memory round trip
  const uint2* w4 = (const uint2*)w;
  uint2 wv[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int i = tid + q * kNormThreads;
    if (i < d4) wv[q] = w4[i];
  }
  float ss = 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int i = tid + q * kNormThreads;
    if (i < d4) {
      dec_f32x4 x = hr[i];
      if (nparts > 0) {
        dec_f32x4 y = dr[i];
        for (int p = 1; p < nparts; ++p) {  // parts summed in order, then added to h
          const dec_f32x4 z = dr[(int64_t)p * (part_stride / 4) + i];
          y = dec_f32x4{y[0] + z[0], y[1] + z[1], y[2] + z[2], y[3] + z[3]};
        }
        x = dec_f32x4{x[0] + y[0], x[1] + y[1], x[2] + y[2], x[3] + y[3]};
        hr[i] = x;
      }
      v[q] = x;
      ss += x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3];
    }
  }
  __shared__ float part[kNormThreads / 64];
  ss = wave_sum(ss);
  if (lane == 0) part[wave] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; ++i) tot += part[i];
  const float inv = 1.0f / sqrtf(tot / (float)d + eps);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int i = tid + q * kNormThreads;
    if (i < d4) {
      const uint2 ww = wv[q];
      const dec_f32x4 x = v[q];
      store4(out, odt, r * d + 4 * i,
             dec_f32x4{x[0] * inv * lo_bf16(ww.x), x[1] * inv * hi_bf16(ww.x), x[2] * inv * lo_bf16(ww.y),
                       x[3] * inv * hi_bf16(ww.y)});
    }
  }
}

// ------------------------------------------------------------------ RoPE + KV store
// Rotate the pair (x1, x2) = (x[i], x[i + hd / 2]) of one head at position p: rotate-half RoPE
// with angle p * base^(-2 i / hd).  The frequency exp2(-(2 i / hd) log2(base)) and the angle
// are formed in double and reduced to [-pi, pi] by a two-term Cody-Waite subtraction of 2 pi,
// so that the float sine and cosine need no large-argument reduction.
__device__ __forceinline__ void rope_pair(float x1, float x2, int p, int i, int hd, double log2_base, float& y1,
                                          float& y2) {
  constexpr double kTwoPiHi = 6.28318530717958623200e+00;  // 2 pi rounded to double
  constexpr double kTwoPiLo = 2.44929359829470641e-16;     // 2 pi - kTwoPiHi
  const double a = (double)p * exp2(-(2.0 * i / hd) * log2_base);
  const double n = rint(a * (1.0 / kTwoPiHi));
  const float r = (float)fma(-n, kTwoPiLo, fma(-n, kTwoPiHi, a));
  float sn, cs;
  sincosf(r, &sn, &cs);
  y1 = x1 * cs - x2 * sn;
  y2 = x2 * cs + x1 * sn;
}

// Grid (rows, heads + kv_heads), head_dim / 2 threads: thread i rotates the pair
// (i, i + head_dim / 2) of one q or k head; k heads also store k (rotated) and v as bf16.
__global__ void dec_rope_kv(float* __restrict__ qkv, int T, int H, int HK, int hd, const int32_t* __restrict__ pos,
                            double log2_base, uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int max_seq,
                            uint16_t* __restrict__ qs, uint16_t* __restrict__ ks, int parts) {
  const int64_t r = blockIdx.x;
  const int hh = blockIdx.y, i = threadIdx.x, half = hd / 2;
  const int b = (int)(r / T), t = (int)(r % T);
  const int p = pos[b] + t;
  const int64_t ld = (int64_t)(H + 2 * HK) * hd;
  float* x = qkv + r * ld + (int64_t)hh * hd;
  float y1, y2;
  rope_pair(x[i], x[i + half], p, i, hd, log2_base, y1, y2);
  x[i] = y1;
  x[i + half] = y2;
  if (hh < H && qs) {  // rotated q split into `parts` bf16 terms, [b, head, t, parts * hd]
    const int64_t o = (((int64_t)b * H + hh) * T + t) * parts * hd;
    float r1 = y1, r2 = y2;
    for (int s = 0; s < parts; ++s) {
      const uint16_t a1 = f32_to_bf16(r1), a2 = f32_to_bf16(r2);
      qs[o + s * hd + i] = a1;
      qs[o + s * hd + i + half] = a2;
      r1 -= bf16_bits_to_f32(a1);  // exact in fp32: the residual has at most 16 significant bits
      r2 -= bf16_bits_to_f32(a2);
    }
  }
  if (hh >= H && p >= 0 && p < max_seq) {
    const int j = hh - H;
    const int64_t o = (((int64_t)b * HK + j) * max_seq + p) * hd;
    const uint16_t k1 = f32_to_bf16(y1), kk2 = f32_to_bf16(y2);
    kc[o + i] = k1;
    kc[o + i + half] = kk2;
    const float* v = qkv + r * ld + (int64_t)(H + HK + j) * hd;
    const uint16_t v1 = f32_to_bf16(v[i]), v2 = f32_to_bf16(v[i + half]);
    vc[o + i] = v1;
    vc[o + i + half] = v2;
    if (ks) {  // the cached k `parts` times, [b, kv head, t, parts * hd], against q's terms
      const int64_t o2 = (((int64_t)b * HK + j) * T + t) * parts * hd;
      for (int s = 0; s < parts; ++s) {
        ks[o2 + s * hd + i] = k1;
        ks[o2 + s * hd + i + half] = kk2;
      }
    }
  }
}

// Grid (ceil(T / 64), batch * kv_heads), 256 threads: the cached v of 64 tokens of one kv head
// (bf16 [64, hd] at positions pos[b] + t, as tgm_dec_rope_kv stored them; tokens past the cache
// are skipped) transposed through LDS, 128 columns at a time, into `parts` copies of vt [hd,
// ldvt] at columns s * ldvt / parts + t; each thread stores 8 tokens (16 bytes) of one row.
// Needs hd % 8 == 0 and ldvt / parts % 8 == 0.
__global__ void __launch_bounds__(256) dec_vt_terms(const uint16_t* __restrict__ vc, const int32_t* __restrict__ pos,
                                                    int T, int HK, int hd, int max_seq, uint16_t* __restrict__ vt,
                                                    int64_t ldvt, int parts) {
  __shared__ uint16_t tile[64][130];
  const int t0 = blockIdx.x * 64, tid = threadIdx.x;
  const int p0 = pos[blockIdx.y / HK];
  const int rows = min(min(64, T - t0), max_seq - p0 - t0);
  if (p0 < 0 || rows <= 0) return;  // uniform over the workgroup, before any barrier
  const uint16_t* src = vc + ((int64_t)blockIdx.y * max_seq + p0 + t0) * hd;
  uint16_t* dst = vt + (int64_t)blockIdx.y * hd * ldvt + t0;
  const int64_t w = ldvt / parts;
  for (int c0 = 0; c0 < hd; c0 += 128) {
    const int cw = min(128, hd - c0);
    for (int idx = tid; idx < 64 * 16; idx += 256) {
      const int r = idx >> 4, c = (idx & 15) * 8;
      if (r < rows && c < cw) {
        const dec_u32x4 v = *(const dec_u32x4*)(src + (int64_t)r * hd + c0 + c);
        unsigned* tp = (unsigned*)&tile[r][c];  // 4-byte aligned: c is even, rows are 260 bytes
        tp[0] = v[0]; tp[1] = v[1]; tp[2] = v[2]; tp[3] = v[3];
      }
    }
    __syncthreads();
    for (int idx = tid; idx < 128 * 8; idx += 256) {
      const int c = idx >> 3, r = (idx & 7) * 8;
      if (c < cw && r < rows) {
        uint16_t* o = dst + (int64_t)(c0 + c) * ldvt + r;
        if (r + 8 <= rows) {
          dec_u32x4 pk;
#pragma unroll
          for (int q = 0; q < 4; ++q) pk[q] = (unsigned)tile[r + 2 * q][c] | ((unsigned)tile[r + 2 * q + 1][c] << 16);
          for (int s = 0; s < parts; ++s) *(dec_u32x4*)(o + s * w) = pk;
        } else {
          for (int s = 0; s < parts; ++s)
            for (int e = 0; e < rows - r; ++e) o[s * w + e] = tile[r + e][c];
        }
      }
    }
    __syncthreads();
  }
}

// ------------------------------------------------------------------ prefill softmax
// p[j] = softmax over j <= t of scale * S[row, j] for row = z * T + t (causal, the prompt
// starting at position 0), split into `parts` bf16 terms: term s of p[j] at P[row, s * w + j]
// (w = ldp / parts; term 0 = bf16(p), term s = bf16 of what the earlier terms leave), all 0 for
// t < j < w.  One wave per row; scores are read as float4 (ld_scores % 4 == 0) and each term is
// written with 16-byte stores (w % 8 == 0).
__global__ void __launch_bounds__(256) dec_causal_softmax(const float* __restrict__ S, int64_t rows, int T,
                                                          int64_t lds_, float scale, uint16_t* __restrict__ P,
                                                          int64_t ldp, int parts) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;  // whole waves leave together
  const int len = (int)(row % T) + 1;
  const float* s = S + row * lds_;
  uint16_t* pr = P + row * ldp;
  // pass 1: running (max, sum of exp) per lane over 4-float groups, then across the wave
  float m = -INFINITY, l = 0.f;
  for (int j0 = lane * 4; j0 < len; j0 += 256) {
    dec_f32x4 v;
    if (j0 + 4 <= len) {
      v = *(const dec_f32x4*)(s + j0);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = j0 + e < len ? s[j0 + e] : -INFINITY;
    }
    const float mn = fmaxf(m, fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])));
    l = (m == -INFINITY ? 0.f : l * expf((m - mn) * scale)) + expf((v[0] - mn) * scale) +
        expf((v[1] - mn) * scale) + expf((v[2] - mn) * scale) + expf((v[3] - mn) * scale);
    m = mn;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float m2 = __shfl_xor(m, off, 64), l2 = __shfl_xor(l, off, 64);
    const float mn = fmaxf(m, m2);
    l = (m == -INFINITY ? 0.f : l * expf((m - mn) * scale)) + (m2 == -INFINITY ? 0.f : l2 * expf((m2 - mn) * scale));
    m = mn;
  }
  const float inv = 1.0f / l;
  // pass 2: 8 consecutive probabilities per lane, split into terms, 16-byte stores per term
  const int64_t w = ldp / parts;
  for (int j0 = lane * 8; j0 < w; j0 += 512) {
    float r[8];
    if (j0 + 8 <= len) {
      const dec_f32x4 a = *(const dec_f32x4*)(s + j0), b = *(const dec_f32x4*)(s + j0 + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        r[e] = expf((a[e] - m) * scale) * inv;
        r[e + 4] = expf((b[e] - m) * scale) * inv;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) r[e] = j0 + e < len ? expf((s[j0 + e] - m) * scale) * inv : 0.f;
    }
    for (int q = 0; q < parts; ++q) {
      dec_u32x4 pk;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint16_t lo = f32_to_bf16(r[2 * e]), hi = f32_to_bf16(r[2 * e + 1]);
        pk[e] = (unsigned)lo | ((unsigned)hi << 16);
        r[2 * e] -= bf16_bits_to_f32(lo);
        r[2 * e + 1] -= bf16_bits_to_f32(hi);
      }
      *(dec_u32x4*)(pr + q * w + j0) = pk;
    }
  }
}

// ------------------------------------------------------------------ attention
constexpr int kMaxSplits = 32;

// Grid (rows, kv_heads, splits), 256 threads.  A workgroup takes the G = heads / kv_heads q
// heads that share kv head j, and the chunks of 64 cache positions [z * cps * 64, +cps * 64)
// of its split, clipped to the token's causal length.  Per chunk:
//   1. scores: 4 lanes per position, each a quarter of head_dim, dot with the G scaled q's
//      (q kept in LDS), combined by two lane swaps;
//   2. wave g (g, g + 4) folds the chunk into the running max / sum of head g (online
//      softmax) and turns the chunk's scores into probabilities;
//   3. lane l accumulates dims (2 l, 2 l + 1) of p . v over the positions of its wave
//      (positions w, w + 4, ...), rescaled by exp(m_old - m_new).
// A chunk's k and v are loaded together into registers; the first chunk's before q is staged.
// One split writes the normalised output; several write (o, m, l) partials per (row, head,
// split) that dec_attention_merge combines.  Loads use positions clamped into the valid range
// (their probabilities are zero), so every load in a chunk is unconditional.
//
// With ``base`` > 0 (one token per sequence) the kernel also does tgm_dec_rope_kv's work for
// its token in the same arithmetic: q is rotated as it is staged, and the workgroup whose split
// holds the token's own position rotates k, stores k and v into the cache and uses those bf16
// values for that position from LDS.
template <int G, int HD>
__global__ void __launch_bounds__(256) dec_attention(const float* __restrict__ qkv, int T, int H, int HK,
                                                     const int32_t* __restrict__ pos, uint16_t* __restrict__ kc,
                                                     uint16_t* __restrict__ vc, int max_seq, int cps, float scale,
                                                     int own, double log2_base, float* __restrict__ part,
                                                     void* __restrict__ out,
                                                     int odt, int hs) {
  constexpr int CH = 64, NP = HD / 2, QD = HD / 4;
  // blockIdx.y = kv head * hs + sub-group: the workgroup takes q heads [blockIdx.y * G, + G)
  // of the G * hs heads that share kv head j
  const int r = blockIdx.x, j = blockIdx.y / hs, z = blockIdx.z, S = gridDim.z;
  const int hq0 = blockIdx.y * G;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b = r / T, t = r % T;
  const int p = pos[b] + t;
  const int len = p + 1 < max_seq ? p + 1 : max_seq;
  const int c_begin = z * cps * CH;
  const int c_end = len < c_begin + cps * CH ? len : c_begin + cps * CH;
  const int64_t ld = (int64_t)(H + 2 * HK) * HD;
  __shared__ float qs[G][HD];
  __shared__ float sc[G][CH];
  __shared__ float m_sh[G], l_sh[G], a_sh[G];
  __shared__ float red[4][G][HD];
  const int64_t kvbase = ((int64_t)b * HK + j) * max_seq;
  // own: rotate q, k and store this token's k, v
  const bool mine = own && p >= c_begin && p < c_end;   // this split holds the token's position
  __shared__ __attribute__((aligned(16))) uint16_t kp[HD], vp[HD];  // bf16 bits
  const float* qrow = qkv + (int64_t)r * ld + (int64_t)hq0 * HD;
  // k (4 lanes per position, a quarter of head_dim each) and v (lane l: dims 2 l, 2 l + 1 of
  // the wave's positions w, w + 4, ...) of a chunk; the first chunk's loads are issued before
  // q is staged, later chunks' at the top of their iteration
  const int pi = tid >> 2, qd = tid & 3;
  dec_u32x4 kreg[QD / 8];
  unsigned vreg[CH / 4];
  // lane l's dims 2 l, 2 l + 1 of the wave's first cache row; the wave's positions are uniform,
  // so a whole chunk inside the split is one base and constant offsets
  const uint16_t* vlane = vc + (kvbase + wave) * HD + 2 * lane;
  auto load_chunk = [&](int c0) __attribute__((always_inline)) {
    const int last = c_end - 1;
    const int tk = c0 + pi;
    const uint16_t* kr = kc + (kvbase + (tk < last ? tk : last)) * HD + qd * QD;
#pragma unroll
    for (int e = 0; e < QD / 8; ++e) kreg[e] = *(const dec_u32x4*)(kr + 8 * e);
    if (lane < NP) {
      if (c0 + CH <= c_end) {
        const uint16_t* vb = vlane + (int64_t)c0 * HD;
#pragma unroll
        for (int i = 0; i < CH / 4; ++i) vreg[i] = *(const unsigned*)(vb + 4 * i * HD);
      } else {  // the split's last chunk: positions clamped to its last one
#pragma unroll
        for (int i = 0; i < CH / 4; ++i) {
          const int tt = c0 + wave + 4 * i;
          vreg[i] = *(const unsigned*)(vlane + (int64_t)((tt < last ? tt : last) - wave) * HD);
        }
      }
    }
  };
  // (the split holding the token's own position may read that position's k, v before this
  // workgroup stores them: those two values are taken from LDS instead)
  if (c_begin < c_end) load_chunk(c_begin);
  if (own) {
    for (int i = tid; i < G * NP; i += 256) {
      const int g = i / NP, e = i % NP;
      float y1, y2;
      rope_pair(qrow[g * HD + e], qrow[g * HD + e + NP], p, e, HD, log2_base, y1, y2);
      qs[g][e] = y1 * scale;
      qs[g][e + NP] = y2 * scale;
    }
    if (mine && tid < NP) {
      const float* kx = qkv + (int64_t)r * ld + (int64_t)(H + j) * HD;
      const float* vx = qkv + (int64_t)r * ld + (int64_t)(H + HK + j) * HD;
      float y1, y2;
      rope_pair(kx[tid], kx[tid + NP], p, tid, HD, log2_base, y1, y2);
      const uint16_t k1 = f32_to_bf16(y1), k2 = f32_to_bf16(y2);
      const uint16_t v1 = f32_to_bf16(vx[tid]), v2 = f32_to_bf16(vx[tid + NP]);
      const int64_t o = (kvbase + p) * HD;
      if (blockIdx.y % hs == 0) {  // one sub-group stores; every sub-group uses the values from LDS
        kc[o + tid] = k1;
        kc[o + tid + NP] = k2;
        vc[o + tid] = v1;
        vc[o + tid + NP] = v2;
      }
      kp[tid] = k1;
      kp[tid + NP] = k2;
      vp[tid] = v1;
      vp[tid + NP] = v2;
    }
  } else {
    for (int i = tid; i < G * HD; i += 256) qs[i / HD][i % HD] = qrow[i] * scale;
  }
  if (tid < G) {
    m_sh[tid] = -INFINITY;
    l_sh[tid] = 0.f;
  }
  float oa[G][2];
#pragma unroll
  for (int g = 0; g < G; ++g) oa[g][0] = oa[g][1] = 0.f;
  __syncthreads();
  for (int c0 = c_begin; c0 < c_end; c0 += CH) {
    if (c0 != c_begin) load_chunk(c0);
    if (mine) {  // uniform: the loaded k, v of the token's own position predate its store
      if (c0 + pi == p)
#pragma unroll
        for (int e = 0; e < QD / 8; ++e) kreg[e] = *(const dec_u32x4*)(kp + qd * QD + 8 * e);
      if (lane < NP) {
        const unsigned own_v = *(const unsigned*)(vp + 2 * lane);
#pragma unroll
        for (int i = 0; i < CH / 4; ++i) vreg[i] = c0 + wave + 4 * i == p ? own_v : vreg[i];
      }
    }
    {
      const int tt = c0 + pi;
      float s[G];
#pragma unroll
      for (int g = 0; g < G; ++g) s[g] = 0.f;
#pragma unroll
      for (int e = 0; e < QD; e += 8) {
        const dec_u32x4 kv = kreg[e / 8];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float k0 = lo_bf16(kv[q]), k1 = hi_bf16(kv[q]);
#pragma unroll
          for (int g = 0; g < G; ++g) s[g] += qs[g][qd * QD + e + 2 * q] * k0 + qs[g][qd * QD + e + 2 * q + 1] * k1;
        }
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        s[g] += xor1(s[g]);
        s[g] += xor2(s[g]);
      }
      if (qd == 0)
#pragma unroll
        for (int g = 0; g < G; ++g) sc[g][pi] = tt < c_end ? s[g] : -INFINITY;
    }
    __syncthreads();
    for (int g = wave; g < G; g += 4) {
      const float v = sc[g][lane];
      const float m_old = m_sh[g];
      const float m_new = fmaxf(m_old, wave_max(v));  // the chunk has a valid position
      const float pv = v == -INFINITY ? 0.f : expf(v - m_new);
      const float sum = wave_sum(pv);
      sc[g][lane] = pv;
      if (lane == 0) {
        const float alpha = m_old == -INFINITY ? 0.f : expf(m_old - m_new);
        a_sh[g] = alpha;
        l_sh[g] = l_sh[g] * alpha + sum;
        m_sh[g] = m_new;
      }
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float al = a_sh[g];
      oa[g][0] *= al;
      oa[g][1] *= al;
    }
    if (lane < NP) {
#pragma unroll
      for (int i = 0; i < CH / 4; ++i) {
        const int pv_i = wave + 4 * i;
        const unsigned vv = vreg[i];
        const float v0 = lo_bf16(vv), v1 = hi_bf16(vv);
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float pg = sc[g][pv_i];
          oa[g][0] += pg * v0;
          oa[g][1] += pg * v1;
        }
      }
    }
    __syncthreads();  // the next chunk rewrites sc and a_sh
  }
  if (lane < NP)
#pragma unroll
    for (int g = 0; g < G; ++g) {
      red[wave][g][2 * lane] = oa[g][0];
      red[wave][g][2 * lane + 1] = oa[g][1];
    }
  __syncthreads();
  for (int i = tid; i < G * HD; i += 256) {
    const int g = i / HD, d = i % HD, h = hq0 + g;
    const float o = red[0][g][d] + red[1][g][d] + red[2][g][d] + red[3][g][d];
    if (part == nullptr) {
      const float l = l_sh[g];
      store_from_f32(out, odt, (int64_t)r * H * HD + (int64_t)h * HD + d, l > 0.f ? o / l : 0.f);
    } else {
      float* pp = part + (((int64_t)r * H + h) * S + z) * (HD + 2);
      pp[d] = o;
      if (d == 0) {
        pp[HD] = m_sh[g];
        pp[HD + 1] = l_sh[g];
      }
    }
  }
}

// One pass, no partials: grid (rows, kv_heads * hs), 1024 threads (16 waves).  Workgroup (r, y)
// takes kv head j = y % HK and the GW q heads j * G + (y / HK) * GW + [0, GW) of it (G = H / HK,
// GW = G / hs).  Workgroup ids r + rows (s HK + j) put every sub-group of kv head j on the same
// XCD (ids are dealt to the 8 XCDs round robin), and a row's kv heads on one XCD when rows is a
// multiple of 8, so the sub-groups' re-reads of a kv head hit that XCD's L2.  Wave w takes the
// chunks of 16 positions w, w + 16, ... of [0, len):
//   lanes 4 i .. 4 i + 3 hold a quarter of head_dim of position c0 + i's k each; their dot
//   products with the GW scaled q's (read from LDS per chunk) are combined by two lane swaps;
//   the wave folds the chunk into its own running max / sum per q head (online softmax);
//   lane l accumulates dims (2 l, 2 l + 1) of p . v, each probability read from the lane that
//   holds it.
// The first chunk's loads are issued before q is staged; later chunks' k loads as soon as the
// previous chunk's scores are done and their v loads as soon as its p . v is, so a wave's next
// chunk is in flight while it computes.  At the end the 16 waves' (o, m, l) meet in LDS and are
// merged with weights exp(m_w - M).  Loads use positions clamped into the valid range (their
// probabilities are zero).  With ``own`` the kernel does tgm_dec_rope_kv's work for the token as
// dec_attention does: sub-group 0 stores the rotated k and v, and every workgroup takes the
// token's own position from LDS.
constexpr int kOneWaves = 16, kOneChunk = 16;

template <int GW, int HD>
__global__ void __launch_bounds__(kOneWaves * 64) dec_attention_one(const float* __restrict__ qkv, int T, int H, int HK,
                                                                    const int32_t* __restrict__ pos,
                                                                    uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
                                                                    int max_seq, float scale, int own, double log2_base,
                                                                    void* __restrict__ out, int odt) {
  constexpr int NP = HD / 2;  // rotation pairs; lanes [0, NP) hold two dims of v each
  constexpr int QD = HD / 4;  // dims of k per lane (four lanes per position)
  constexpr int KL = QD / 8;  // 16-byte k loads per lane and chunk
  const int r = blockIdx.x, y = blockIdx.y, j = y % HK, sub = y / HK;
  const int hq0 = j * (H / HK) + sub * GW;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b = r / T, t = r % T;
  const int p = pos[b] + t;
  const int len = p + 1 < max_seq ? p + 1 : max_seq;
  const int64_t ld = (int64_t)(H + 2 * HK) * HD;
  const int64_t kvbase = ((int64_t)b * HK + j) * max_seq;
  __shared__ __attribute__((aligned(16))) float qs[GW][HD];
  __shared__ __attribute__((aligned(16))) uint16_t kp[HD], vp[HD];  // the token's own k, v (bf16 bits)
  __shared__ float mw[kOneWaves][GW], lw[kOneWaves][GW];
  __shared__ float ow[kOneWaves][GW][HD];
  const float* qrow = qkv + (int64_t)r * ld + (int64_t)hq0 * HD;
  const int pi = lane >> 2, qd = lane & 3;
  dec_u32x4 kreg[KL];
  unsigned vreg[kOneChunk];
  auto load_k = [&](int c0) __attribute__((always_inline)) {
    const int tk = c0 + pi < len ? c0 + pi : len - 1;
    const uint16_t* kr = kc + (kvbase + tk) * HD + qd * QD;
#pragma unroll
    for (int e = 0; e < KL; ++e) kreg[e] = *(const dec_u32x4*)(kr + 8 * e);
  };
  // lane l's dims 2 l, 2 l + 1 of cache row 0 (lanes past NP read, and ignore, dims 0, 1); a
  // chunk's positions are wave-uniform, so a whole chunk is one base and immediate offsets
  const uint16_t* vlane = vc + kvbase * HD + 2 * (lane < NP ? lane : 0);
  auto load_v = [&](int c0) __attribute__((always_inline)) {
    if (c0 + kOneChunk <= len) {
      const uint16_t* vb = vlane + (int64_t)c0 * HD;
#pragma unroll
      for (int i = 0; i < kOneChunk; ++i) vreg[i] = *(const unsigned*)(vb + i * HD);
    } else {  // the last chunk: positions clamped to the last one
#pragma unroll
      for (int i = 0; i < kOneChunk; ++i) {
        const int tt = c0 + i < len ? c0 + i : len - 1;
        vreg[i] = *(const unsigned*)(vlane + (int64_t)tt * HD);
      }
    }
  };
  const int c_first = wave * kOneChunk;
  constexpr int c_step = kOneWaves * kOneChunk;
  if (c_first < len) {
    load_k(c_first);
    load_v(c_first);
  }
  if (own) {
    for (int i = tid; i < GW * NP; i += kOneWaves * 64) {
      const int g = i / NP, e = i % NP;
      float y1, y2;
      rope_pair(qrow[g * HD + e], qrow[g * HD + e + NP], p, e, HD, log2_base, y1, y2);
      qs[g][e] = y1 * scale;
      qs[g][e + NP] = y2 * scale;
    }
    if (tid < NP) {
      const float* kx = qkv + (int64_t)r * ld + (int64_t)(H + j) * HD;
      const float* vx = qkv + (int64_t)r * ld + (int64_t)(H + HK + j) * HD;
      float y1, y2;
      rope_pair(kx[tid], kx[tid + NP], p, tid, HD, log2_base, y1, y2);
      const uint16_t k1 = f32_to_bf16(y1), k2 = f32_to_bf16(y2);
      const uint16_t v1 = f32_to_bf16(vx[tid]), v2 = f32_to_bf16(vx[tid + NP]);
      if (sub == 0 && p < max_seq) {  // one sub-group stores; every workgroup uses the values from LDS
        const int64_t o = (kvbase + p) * HD;
        kc[o + tid] = k1;
        kc[o + tid + NP] = k2;
        vc[o + tid] = v1;
        vc[o + tid + NP] = v2;
      }
      kp[tid] = k1;
      kp[tid + NP] = k2;
      vp[tid] = v1;
      vp[tid + NP] = v2;
    }
  } else {
    for (int i = tid; i < GW * HD; i += kOneWaves * 64) qs[i / HD][i % HD] = qrow[i] * scale;
  }
  __syncthreads();
  float m[GW], l[GW], oa[GW][2];
#pragma unroll
  for (int g = 0; g < GW; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
    oa[g][0] = oa[g][1] = 0.f;
  }
  for (int c0 = c_first; c0 < len; c0 += c_step) {
    const int cn = c0 + c_step;  // this wave's next chunk
    if (own && c0 + pi == p)  // the token's own position (the loads may predate its store): from LDS
#pragma unroll
      for (int e = 0; e < KL; ++e) kreg[e] = *(const dec_u32x4*)(kp + qd * QD + 8 * e);
    // q is re-read from LDS for every chunk: an opaque zero offset keeps the compiler from holding
    // the lane's GW * QD q values in registers across the loop
    int zero;
    asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
    const float* qb = &qs[0][0] + qd * QD + zero;
    float s[GW];
#pragma unroll
    for (int g = 0; g < GW; ++g) s[g] = 0.f;
#pragma unroll
    for (int e = 0; e < KL; ++e) {
      const dec_u32x4 kv = kreg[e];
#pragma unroll
      for (int g = 0; g < GW; ++g) {
        const dec_f32x4 qa = *(const dec_f32x4*)(qb + g * HD + 8 * e), qb4 = *(const dec_f32x4*)(qb + g * HD + 8 * e + 4);
        s[g] += qa[0] * lo_bf16(kv[0]) + qa[1] * hi_bf16(kv[0]) + qa[2] * lo_bf16(kv[1]) + qa[3] * hi_bf16(kv[1]) +
                qb4[0] * lo_bf16(kv[2]) + qb4[1] * hi_bf16(kv[2]) + qb4[2] * lo_bf16(kv[3]) + qb4[3] * hi_bf16(kv[3]);
      }
    }
    if (cn < len) load_k(cn);
    const bool valid = c0 + pi < len;
    float pe[GW];
#pragma unroll
    for (int g = 0; g < GW; ++g) {
      float sv = s[g] + xor1(s[g]);
      sv = valid ? sv + xor2(sv) : -INFINITY;
      const float m_new = fmaxf(m[g], wave_max(sv));  // position c0 is valid
      pe[g] = valid ? expf(sv - m_new) : 0.f;
      const float alpha = m[g] == -INFINITY ? 0.f : expf(m[g] - m_new);
      l[g] = l[g] * alpha + wave_sum(qd == 0 ? pe[g] : 0.f);
      m[g] = m_new;
      oa[g][0] *= alpha;
      oa[g][1] *= alpha;
    }
    if (own && p >= c0 && p < c0 + kOneChunk && lane < NP) {  // the chunk holding the token's position
      const unsigned own_v = *(const unsigned*)(vp + 2 * lane);
#pragma unroll
      for (int i = 0; i < kOneChunk; ++i) vreg[i] = c0 + i == p ? own_v : vreg[i];
    }
#pragma unroll
    for (int i = 0; i < kOneChunk; ++i) {
      const float v0 = lo_bf16(vreg[i]), v1 = hi_bf16(vreg[i]);
#pragma unroll
      for (int g = 0; g < GW; ++g) {
        const float pg = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pe[g]), 4 * i));
        oa[g][0] += pg * v0;
        oa[g][1] += pg * v1;
      }
    }
    if (cn < len) load_v(cn);
  }
  if (lane == 0)
#pragma unroll
    for (int g = 0; g < GW; ++g) {
      mw[wave][g] = m[g];
      lw[wave][g] = l[g];
    }
  if (lane < NP)
#pragma unroll
    for (int g = 0; g < GW; ++g) {
      ow[wave][g][2 * lane] = oa[g][0];
      ow[wave][g][2 * lane + 1] = oa[g][1];
    }
  __syncthreads();
  for (int i = tid; i < GW * HD; i += kOneWaves * 64) {
    const int g = i / HD, d = i % HD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kOneWaves; ++w) M = fmaxf(M, mw[w][g]);
    float L = 0.f, o = 0.f;
#pragma unroll
    for (int w = 0; w < kOneWaves; ++w) {
      const float wgt = mw[w][g] == -INFINITY ? 0.f : expf(mw[w][g] - M);
      L += lw[w][g] * wgt;
      o += ow[w][g][d] * wgt;
    }
    store_from_f32(out, odt, (int64_t)r * H * HD + (int64_t)(hq0 + g) * HD + d, L > 0.f ? o / L : 0.f);
  }
}

// Grid (rows, heads), head_dim threads: combine the splits' (o, m, l) partials.  The (m, l) of
// every split go to LDS and become merge weights exp(m_s - M); each thread issues the loads of
// its S partial sums at once.  (The kernel boundary publishes the partials; merging in the last
// attention workgroup instead needs agent-scope fences, which on gfx950 write back and
// invalidate the per-XCD L2 and cost more than this launch.)
template <int HD>
__global__ void __launch_bounds__(HD) dec_attention_merge(const float* __restrict__ part, int S, int H,
                                                          void* __restrict__ out, int odt) {
  const int r = blockIdx.x, h = blockIdx.y, d = threadIdx.x;
  const float* pp = part + ((int64_t)r * H + h) * S * (HD + 2);
  __shared__ float mw[kMaxSplits], lw[kMaxSplits], inv_l;
  if (d < kMaxSplits) {
    mw[d] = d < S ? pp[d * (HD + 2) + HD] : -INFINITY;
    lw[d] = d < S ? pp[d * (HD + 2) + HD + 1] : 0.f;
  }
  float ov[kMaxSplits];
#pragma unroll
  for (int s2 = 0; s2 < kMaxSplits; ++s2) ov[s2] = s2 < S ? pp[s2 * (HD + 2) + d] : 0.f;
  __syncthreads();
  if (d == 0) {
    float M = -INFINITY;
    for (int s2 = 0; s2 < kMaxSplits; ++s2) M = fmaxf(M, mw[s2]);
    float L = 0.f;
    for (int s2 = 0; s2 < kMaxSplits; ++s2) {
      const float wgt = mw[s2] == -INFINITY ? 0.f : expf(mw[s2] - M);
      mw[s2] = wgt;
      L += lw[s2] * wgt;
    }
    inv_l = L > 0.f ? 1.0f / L : 0.f;
  }
  __syncthreads();
  float o = 0.f;
#pragma unroll
  for (int s2 = 0; s2 < kMaxSplits; ++s2) o += mw[s2] * ov[s2];
  store_from_f32(out, odt, (int64_t)r * H * HD + (int64_t)h * HD + d, o * inv_l);
}

// ------------------------------------------------------------------ SwiGLU
__global__ void __launch_bounds__(256) dec_silu_mul(const float* __restrict__ gu, int64_t rows, int64_t F,
                                                    void* __restrict__ out, int odt) {
  const int64_t n = rows * F;
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const float g = gu[2 * i], u = gu[2 * i + 1];  // gate and up rows interleaved
    store_from_f32(out, odt, i, g / (1.0f + expf(-g)) * u);
  }
}

// ------------------------------------------------------------------ bf16 GEMV (output head)
// x (M rows) is staged in LDS once per workgroup; each wave then streams whole weight rows
// (lane l reads 16-byte chunks l, l + 64, ...) and reduces its dot products over the wave.
// R weight rows per wave at a time: each x chunk read from LDS serves R rows (for M > 1 the
// LDS reads of x, M per weight chunk, would otherwise bound the kernel).
template <int M, int R>
__global__ void __launch_bounds__(256) dec_gemv_bf16(const uint16_t* __restrict__ w, int N, int K,
                                                     const uint16_t* __restrict__ x, int64_t ldx, float* __restrict__ y,
                                                     int64_t ldy) {
  __shared__ dec_u32x4 xs[32768 / 8];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kc = K / 8;  // 16-byte chunks per row
  for (int i = tid; i < M * kc; i += 256) xs[i] = *(const dec_u32x4*)(x + (int64_t)(i / kc) * ldx + (int64_t)(i % kc) * 8);
  __syncthreads();
  const int nw = gridDim.x * 4;
  // bf16 pairs are loaded as pairs: bit-casting the dwords of a loaded 4-dword vector to
  // bf16 pairs has been compiled into one repeated pair
  const dec_bf16x2* xp = (const dec_bf16x2*)xs;
  for (int n = (blockIdx.x * 4 + wave) * R; n < N; n += nw * R) {
    float acc[R][M];
    const dec_bf16x2* wr[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      wr[r] = (const dec_bf16x2*)(w + (int64_t)(n + r < N ? n + r : N - 1) * K);  // rows past N are not stored
#pragma unroll
      for (int m = 0; m < M; ++m) acc[r][m] = 0.f;
    }
#pragma unroll (R == 1 ? 8 : 2)
    for (int c = lane; c < kc; c += 64) {  // 16-byte chunk c: pairs 4 c .. 4 c + 3
      dec_bf16x2 xv[M][4];
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int e = 0; e < 4; ++e) xv[m][e] = xp[4 * (m * kc + c) + e];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        dec_bf16x2 wv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) wv[e] = wr[r][4 * c + e];
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[r][m] = __builtin_amdgcn_fdot2_f32_bf16(wv[e], xv[m][e], acc[r][m], false);
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) acc[r][m] = wave_sum(acc[r][m]);
    if (lane == 0)
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (n + r < N)
#pragma unroll
          for (int m = 0; m < M; ++m) y[m * ldy + n + r] = acc[r][m];
  }
}

// The same product for 2 <= M <= 8 rows on bf16 MFMA (K a multiple of 128, M x K <= 32768):
// each weight pair meets every x row in its own dot2 above, which makes that form VALU-bound at
// 8 rows.  x is staged in LDS once per workgroup (16-byte chunk c of row m at c ^ m, so that
// the 8 rows' reads of one chunk fall in different banks); each wave streams 16-row tiles of W.
// In a 128-element step lane (r, q) loads 16 bytes of weight row r at K 32 s + 8 q for s = 0..3
// (each load instruction reads 64 contiguous bytes of 16 rows; a ring of kHeadRing steps in
// flight), and MFMA s (v_mfma_f32_16x16x32_bf16, A = those weights, B = x) takes load s against
// x at the same K, so lane l ends with Y[m = l & 15][n0 + 4 (l / 16) + i] (rows m >= M read x
// row 0 and are not stored).
// Products of bf16 values are exact in the fp32 accumulator, as in the dot2 form.  Two steps in
// flight per wave (8 KB; about 16 MB over the chip at 8 waves per CU) beat 3, 4, 6 and 8.
constexpr int kHeadRing = 2;
__global__ void __launch_bounds__(256) dec_gemv_bf16_mfma(const uint16_t* __restrict__ w, int N, int K,
                                                          const uint16_t* __restrict__ x, int64_t ldx, int M,
                                                          float* __restrict__ y, int64_t ldy) {
  typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
  __shared__ dec_u32x4 xs[32768 / 8];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kc = K / 8;  // 16-byte chunks per row (a multiple of 16)
  for (int i = tid; i < M * kc; i += 256) {
    const int m = i / kc, c = i % kc;
    xs[m * kc + (c ^ m)] = *(const dec_u32x4*)(x + (int64_t)m * ldx + (int64_t)c * 8);
  }
  __syncthreads();
  const int r = lane & 15, q = lane >> 4;
  const int xr = r < M ? r : 0;
  const dec_u32x4* xrow = xs + xr * kc;
  const int S = K / 128;
  const int ntiles = (N + 15) / 16;
  for (int tile = blockIdx.x * 4 + wave; tile < ntiles; tile += gridDim.x * 4) {  // uniform per wave
    const int n0 = tile * 16;
    const uint16_t* wrow = w + (int64_t)(n0 + r < N ? n0 + r : N - 1) * K + 8 * q;  // rows past N: not stored
    dec_u32x4 ring[kHeadRing][4];
    auto load = [&](int t, int slot) __attribute__((always_inline)) {
      const uint16_t* p = wrow + 128 * (t < S ? t : S - 1);  // past the end: the last step
#pragma unroll
      for (int e = 0; e < 4; ++e) ring[slot][e] = __builtin_nontemporal_load((const dec_u32x4*)(p + 32 * e));
    };
#pragma unroll
    for (int j = 0; j < kHeadRing; ++j) load(j, j);
    dec_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int t0 = 0; t0 < S; t0 += kHeadRing) {
#pragma unroll
      for (int jj = 0; jj < kHeadRing; ++jj) {
        const int t = t0 + jj;
        if (t < S) {
#pragma unroll
          for (int s2 = 0; s2 < 4; ++s2) {
            const int chunk = 16 * t + 4 * s2 + q;
            const dec_u32x4 xv = xrow[chunk ^ xr];
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, ring[jj][s2]),
                                                          __builtin_bit_cast(bf16x8_t, xv), acc, 0, 0, 0);
          }
        }
        load(t + kHeadRing, jj);
        __builtin_amdgcn_sched_barrier(0);  // each refill right after its slot's MFMAs
      }
    }
    if (r < M)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (n0 + 4 * q + i < N) y[(int64_t)r * ldy + n0 + 4 * q + i] = acc[i];
  }
}

// ------------------------------------------------------------------ greedy argmax
__global__ void __launch_bounds__(1024) dec_argmax(const float* __restrict__ logits, int n, int64_t ld,
                                                   int32_t* __restrict__ tokens, int32_t* __restrict__ pos,
                                                   int32_t* __restrict__ hist, int64_t hstride, int64_t hbase) {
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float* row = logits + r * ld;
  float best = -INFINITY;
  int bi = n;  // none yet (NaN and -inf never win)
  // float4 loads where the row is 16-byte aligned; a thread visits its indices in increasing
  // order, so the strict comparison keeps its first maximum
  const int n4 = ((uintptr_t)row & 15) == 0 ? n / 4 : 0;
  const dec_f32x4* row4 = (const dec_f32x4*)row;
#pragma unroll 4
  for (int i = tid; i < n4; i += 1024) {
    const dec_f32x4 v = row4[i];
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (v[c] > best) {
        best = v[c];
        bi = 4 * i + c;
      }
  }
  for (int i = 4 * n4 + tid; i < n; i += 1024) {
    const float v = row[i];
    if (v > best) {
      best = v;
      bi = i;
    }
  }
  auto better = [](float v, int i, float bv, int bidx) { return v > bv || (v == bv && i < bidx); };
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(best, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (better(ov, oi, best, bi)) {
      best = ov;
      bi = oi;
    }
  }
  __shared__ float bv[16];
  __shared__ int bx[16];
  if (lane == 0) {
    bv[wave] = best;
    bx[wave] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 16; ++w)
      if (better(bv[w], bx[w], best, bi)) {
        best = bv[w];
        bi = bx[w];
      }
    if (bi >= n) bi = 0;
    tokens[r] = bi;
    if (pos) {
      const int p = pos[r];
      const int64_t k = (int64_t)p + 1 - hbase;
      if (hist && k >= 0 && k < hstride) hist[r * hstride + k] = bi;
      pos[r] = p + 1;
    }
  }
}

}  // namespace tgm

using namespace tgm;

static bool out_dtype_ok(int dt) { return dt == TGM_F16 || dt == TGM_BF16 || dt == TGM_F32; }

extern "C" int tgm_dec_embed(const void* table, int64_t vocab, int64_t d, const int32_t* tokens, int64_t rows,
                             float* h, void* stream) {
  clear_error();
  TGM_CHECK_ARG(table && tokens && h, "null operand");
  TGM_CHECK_ARG(vocab > 0 && d > 0 && rows >= 0 && d < (1ll << 31) && rows < (1ll << 31), "invalid embedding sizes");
  if (d % 8 || (uintptr_t)table % 16 || (uintptr_t)h % 16)
    TGM_UNSUPPORTED("tgm_dec_embed: d must be a multiple of 8 and the table and h 16-byte aligned");
  if (rows == 0) return TGM_OK;
  hipLaunchKernelGGL(dec_embed, dim3((unsigned)rows), dim3(512), 0, (hipStream_t)stream, (const uint16_t*)table, vocab,
                     (int)d, tokens, h);
  return launch_status("tgm_dec_embed");
}

extern "C" int tgm_dec_add_rmsnorm(float* h, const float* delta, int64_t rows, int64_t d, const void* weight, float eps,
                                   void* out, int out_dtype, void* stream) {
  clear_error();
  TGM_CHECK_ARG(h && weight && out, "null operand");
  TGM_CHECK_ARG(rows >= 0 && d > 0 && d < (1ll << 31) && rows < (1ll << 31), "invalid norm sizes");
  TGM_CHECK_ARG(out_dtype_ok(out_dtype), "output must be f16, bf16 or f32");
  TGM_CHECK_ARG(eps >= 0.f, "eps must be non-negative");
  if (d % 4 || d > kNormMaxD || (uintptr_t)h % 16 || (uintptr_t)out % 16 || (delta && (uintptr_t)delta % 16) ||
      (uintptr_t)weight % 8)
    TGM_UNSUPPORTED("tgm_dec_add_rmsnorm: d must be a multiple of 4 and at most %d, rows 16-byte aligned", kNormMaxD);
  if (rows == 0) return TGM_OK;
  hipLaunchKernelGGL(dec_add_rmsnorm, dim3((unsigned)rows), dim3(kNormThreads), 0, (hipStream_t)stream, h, delta,
                     delta ? 1 : 0, (int64_t)0, (int)d, (const uint16_t*)weight, eps, out, out_dtype);
  return launch_status("tgm_dec_add_rmsnorm");
}

extern "C" int tgm_dec_add_rmsnorm_parts(float* h, const float* parts, int64_t nparts, int64_t part_stride, int64_t rows,
                                         int64_t d, const void* weight, float eps, void* out, int out_dtype,
                                         void* stream) {
  clear_error();
  TGM_CHECK_ARG(h && parts && weight && out, "null operand");
  TGM_CHECK_ARG(rows >= 0 && d > 0 && d < (1ll << 31) && rows < (1ll << 31), "invalid norm sizes");
  TGM_CHECK_ARG(nparts >= 1 && nparts <= 64 && part_stride >= rows * d, "1 .. 64 parts of at least rows x d floats each");
  TGM_CHECK_ARG(out_dtype_ok(out_dtype), "output must be f16, bf16 or f32");
  TGM_CHECK_ARG(eps >= 0.f, "eps must be non-negative");
  if (d % 4 || d > kNormMaxD || part_stride % 4 || (uintptr_t)h % 16 || (uintptr_t)out % 16 || (uintptr_t)parts % 16 ||
      (uintptr_t)weight % 8)
    TGM_UNSUPPORTED("tgm_dec_add_rmsnorm_parts: d and the part stride must be multiples of 4, d at most %d, rows "
                    "16-byte aligned", kNormMaxD);
  if (rows == 0) return TGM_OK;
  hipLaunchKernelGGL(dec_add_rmsnorm, dim3((unsigned)rows), dim3(kNormThreads), 0, (hipStream_t)stream, h, parts,
                     (int)nparts, part_stride, (int)d, (const uint16_t*)weight, eps, out, out_dtype);
  return launch_status("tgm_dec_add_rmsnorm_parts");
}

extern "C" int tgm_dec_rope_kv(float* qkv, int64_t rows, int64_t seq_rows, int64_t heads, int64_t kv_heads,
                               int64_t head_dim, const int32_t* pos, double rope_base, void* k_cache, void* v_cache,
                               int64_t max_seq, void* q_out, void* k_out, void* vt_out, int64_t ld_vt,
                               int64_t parts, void* stream) {
  clear_error();
  TGM_CHECK_ARG(qkv && pos && k_cache && v_cache, "null operand");
  TGM_CHECK_ARG(rows >= 0 && seq_rows > 0 && rows % seq_rows == 0, "rows must be a multiple of seq_rows");
  TGM_CHECK_ARG(heads > 0 && kv_heads > 0 && heads % kv_heads == 0, "heads must be a multiple of kv_heads");
  TGM_CHECK_ARG(head_dim > 0 && head_dim % 2 == 0 && head_dim <= 1024, "head_dim must be even and at most 1024");
  TGM_CHECK_ARG(max_seq > 0 && max_seq < (1ll << 31) && rows < (1ll << 31), "invalid cache sizes");
  TGM_CHECK_ARG(rope_base > 0.0, "rope base must be positive");
  TGM_CHECK_ARG(!(q_out || k_out || vt_out) || (parts >= 1 && parts <= 3), "parts must be 1, 2 or 3");
  TGM_CHECK_ARG(!vt_out || (ld_vt % parts == 0 && ld_vt / parts >= seq_rows && (ld_vt / parts) % 8 == 0 &&
                             head_dim % 8 == 0 && (uintptr_t)vt_out % 16 == 0 && (uintptr_t)v_cache % 16 == 0),
                "vt_out needs ld_vt / parts >= seq_rows and a multiple of 8, head_dim %% 8 == 0, 16-byte alignment");
  TGM_CHECK_ARG(!vt_out || rows / seq_rows * kv_heads <= 65535, "too many sequences for vt_out");
  if (rows == 0) return TGM_OK;
  hipLaunchKernelGGL(dec_rope_kv, dim3((unsigned)rows, (unsigned)(heads + kv_heads)), dim3((unsigned)(head_dim / 2)), 0,
                     (hipStream_t)stream, qkv, (int)seq_rows, (int)heads, (int)kv_heads, (int)head_dim, pos, log2(rope_base),
                     (uint16_t*)k_cache, (uint16_t*)v_cache, (int)max_seq, (uint16_t*)q_out, (uint16_t*)k_out, (int)parts);
  if (vt_out) {  // after the cache store on the same stream
    hipLaunchKernelGGL(dec_vt_terms, dim3((unsigned)((seq_rows + 63) / 64), (unsigned)(rows / seq_rows * kv_heads)),
                       dim3(256), 0, (hipStream_t)stream, (const uint16_t*)v_cache, pos, (int)seq_rows,
                       (int)kv_heads, (int)head_dim, (int)max_seq, (uint16_t*)vt_out, ld_vt, (int)parts);
  }
  return launch_status("tgm_dec_rope_kv");
}

extern "C" int64_t tgm_dec_attention_workspace(int64_t rows, int64_t heads, int64_t head_dim, int64_t splits) {
  return splits > 1 ? rows * heads * splits * (head_dim + 2) * (int64_t)sizeof(float) : 0;
}

template <int G, int HD>
static void launch_attention(dim3 grid, hipStream_t st, const float* qkv, int T, int H, int HK, const int32_t* pos,
                             void* kc, void* vc, int max_seq, int cps, float scale, int own, double log2_base,
                             float* part, void* out, int odt, int hs) {
  hipLaunchKernelGGL((dec_attention<G, HD>), grid, dim3(256), 0, st, qkv, T, H, HK, pos, (uint16_t*)kc, (uint16_t*)vc,
                     max_seq, cps, scale, own, log2_base, part, out, odt, hs);
}

extern "C" int tgm_dec_attention(const float* qkv, int64_t rows, int64_t seq_rows, int64_t heads, int64_t kv_heads,
                                 int64_t head_dim, const int32_t* pos, void* k_cache, void* v_cache, int64_t max_seq,
                                 double rope_base, int64_t splits, float* workspace, int64_t workspace_bytes,
                                 void* out, int out_dtype, void* stream) {
  clear_error();
  TGM_CHECK_ARG(qkv && pos && k_cache && v_cache && out, "null operand");
  TGM_CHECK_ARG(rows >= 0 && seq_rows > 0 && rows % seq_rows == 0, "rows must be a multiple of seq_rows");
  TGM_CHECK_ARG(heads > 0 && kv_heads > 0 && heads % kv_heads == 0, "heads must be a multiple of kv_heads");
  TGM_CHECK_ARG(out_dtype_ok(out_dtype), "output must be f16, bf16 or f32");
  TGM_CHECK_ARG(max_seq > 0 && max_seq < (1 << 30) && rows < (1ll << 31) && kv_heads <= 65535, "invalid sizes");
  const int64_t chunks = (max_seq + 63) / 64;
  TGM_CHECK_ARG(splits >= 1 && splits <= chunks && splits <= kMaxSplits, "splits must be in [1, min(ceil(max_seq / 64), %d)]",
                kMaxSplits);
  TGM_CHECK_ARG(rope_base <= 0.0 || seq_rows == 1, "the fused RoPE + cache store takes one token per sequence");
  TGM_CHECK_ARG(splits == 1 || (workspace && workspace_bytes >= tgm_dec_attention_workspace(rows, heads, head_dim, splits)),
                "split attention needs a workspace of tgm_dec_attention_workspace() bytes");
  const int64_t G = heads / kv_heads;
  if (head_dim != 64 && head_dim != 128) TGM_UNSUPPORTED("tgm_dec_attention: head_dim must be 64 or 128");
  if (G != 1 && G != 2 && G != 4 && G != 8) TGM_UNSUPPORTED("tgm_dec_attention: heads / kv_heads must be 1, 2, 4 or 8");
  if ((uintptr_t)k_cache % 16 || (uintptr_t)v_cache % 4) TGM_UNSUPPORTED("tgm_dec_attention: caches must be 16-byte aligned");
  if (rows == 0) return TGM_OK;
  const hipStream_t st = (hipStream_t)stream;
  const int own = rope_base > 0.0;
  const float scale = (float)(1.0 / sqrt((double)head_dim));
  if (splits == 1 && rows * heads <= stream_cu_count(st)) {
    // few (token, q head) pairs: one workgroup of 16 waves per pair, one pass over the cache (the
    // grid stays within one round of CUs, and each workgroup's q head fits the wave's registers)
    const dim3 g1((unsigned)rows, (unsigned)heads);
    if (head_dim == 64)
      hipLaunchKernelGGL((dec_attention_one<1, 64>), g1, dim3(kOneWaves * 64), 0, st, qkv, (int)seq_rows, (int)heads,
                         (int)kv_heads, pos, (uint16_t*)k_cache, (uint16_t*)v_cache, (int)max_seq, scale, own,
                         own ? log2(rope_base) : 0.0, out, out_dtype);
    else
      hipLaunchKernelGGL((dec_attention_one<1, 128>), g1, dim3(kOneWaves * 64), 0, st, qkv, (int)seq_rows, (int)heads,
                         (int)kv_heads, pos, (uint16_t*)k_cache, (uint16_t*)v_cache, (int)max_seq, scale, own,
                         own ? log2(rope_base) : 0.0, out, out_dtype);
    return launch_status("tgm_dec_attention");
  }
  const int cps = (int)((chunks + splits - 1) / splits);
  // few (token, kv head, split) workgroups leave most CUs idle: then the q heads of a kv head
  // are spread over hs workgroups (each re-reads the kv head's chunk, mostly from cache)
  int hs = 1;
  while (hs < G && rows * kv_heads * splits * hs * 2 <= 512) hs *= 2;
  const int64_t Gw = G / hs;
  const dim3 grid((unsigned)rows, (unsigned)(kv_heads * hs), (unsigned)splits);
  float* part = splits > 1 ? workspace : nullptr;
#define TGM_ATT(GG, HDD)                                                                                            \
  if (Gw == GG && head_dim == HDD)                                                                                  \
    launch_attention<GG, HDD>(grid, st, qkv, (int)seq_rows, (int)heads, (int)kv_heads, pos, k_cache, v_cache,        \
                              (int)max_seq, cps, scale, own, own ? log2(rope_base) : 0.0, part, out, out_dtype, hs);
  TGM_ATT(1, 64) TGM_ATT(2, 64) TGM_ATT(4, 64) TGM_ATT(8, 64)
  TGM_ATT(1, 128) TGM_ATT(2, 128) TGM_ATT(4, 128) TGM_ATT(8, 128)
#undef TGM_ATT
  int status = launch_status("tgm_dec_attention");
  if (status != TGM_OK || splits == 1) return status;
  const dim3 mgrid((unsigned)rows, (unsigned)heads);
  if (head_dim == 64)
    hipLaunchKernelGGL(dec_attention_merge<64>, mgrid, dim3(64), 0, st, part, (int)splits, (int)heads, out, out_dtype);
  else
    hipLaunchKernelGGL(dec_attention_merge<128>, mgrid, dim3(128), 0, st, part, (int)splits, (int)heads, out, out_dtype);
  return launch_status("tgm_dec_attention");
}

extern "C" int tgm_dec_causal_softmax(const float* scores, int64_t rows, int64_t seq_rows, int64_t ld_scores,
                                      float scale, void* probs, int64_t ld_probs, int64_t parts, void* stream) {
  clear_error();
  TGM_CHECK_ARG(scores && probs, "null operand");
  TGM_CHECK_ARG(rows >= 0 && seq_rows > 0 && rows % seq_rows == 0, "rows must be a multiple of seq_rows");
  TGM_CHECK_ARG(parts >= 1 && parts <= 3, "parts must be 1, 2 or 3");
  TGM_CHECK_ARG(ld_scores >= seq_rows && ld_probs % parts == 0 && ld_probs / parts >= seq_rows,
                "ld_scores must be at least seq_rows, ld_probs a multiple of parts and at least parts * seq_rows");
  TGM_CHECK_ARG(ld_scores % 4 == 0 && (ld_probs / parts) % 8 == 0 && (uintptr_t)scores % 16 == 0 &&
                    (uintptr_t)probs % 16 == 0,
                "ld_scores must be a multiple of 4, ld_probs / parts of 8, both operands 16-byte aligned");
  if (rows == 0) return TGM_OK;
  hipLaunchKernelGGL(dec_causal_softmax, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, (hipStream_t)stream, scores,
                     rows, (int)seq_rows, ld_scores, scale, (uint16_t*)probs, ld_probs, (int)parts);
  return launch_status("tgm_dec_causal_softmax");
}

extern "C" int tgm_dec_silu_mul(const float* gate_up, int64_t rows, int64_t ffn, void* out, int out_dtype,
                                void* stream) {
  clear_error();
  TGM_CHECK_ARG(gate_up && out, "null operand");
  TGM_CHECK_ARG(rows >= 0 && ffn > 0, "invalid sizes");
  TGM_CHECK_ARG(out_dtype_ok(out_dtype), "output must be f16, bf16 or f32");
  if (rows == 0) return TGM_OK;
  const int64_t n = rows * ffn;
  const int64_t blocks = (n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096;
  hipLaunchKernelGGL(dec_silu_mul, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, gate_up, rows, ffn, out,
                     out_dtype);
  return launch_status("tgm_dec_silu_mul");
}

extern "C" int tgm_dec_gemv_bf16(const void* w, int64_t n, int64_t k, const void* x, int64_t m, int64_t ldx, float* y,
                                 int64_t ldy, void* stream) {
  clear_error();
  TGM_CHECK_ARG(w && x && y, "null operand");
  TGM_CHECK_ARG(n >= 0 && k > 0 && m >= 0 && m <= 8, "m must be at most 8");
  TGM_CHECK_ARG(m <= 1 || (ldx >= k && ldy >= n), "row strides smaller than the rows");
  if (n == 0 || m == 0) return TGM_OK;
  if (k % 8 != 0 || m * k > 32768 || n >= (1ll << 31))
    TGM_UNSUPPORTED("tgm_dec_gemv_bf16: k must be a multiple of 8 with m * k <= 32768");
  if ((uintptr_t)w % 16 || (uintptr_t)x % 16 || (m > 1 && (ldx * 2) % 16))
    TGM_UNSUPPORTED("tgm_dec_gemv_bf16: operands and x rows must be 16-byte aligned");
  if (m >= 2 && k % 128 == 0) {  // bf16 MFMA (x staged as for the dot2 form: m * k <= 32768)
    const int64_t tiles = (n + 15) / 16;
    const unsigned g = (unsigned)((tiles + 3) / 4 < 1024 ? (tiles + 3) / 4 : 1024);
    hipLaunchKernelGGL(dec_gemv_bf16_mfma, dim3(g), dim3(256), 0, (hipStream_t)stream, (const uint16_t*)w, (int)n,
                       (int)k, (const uint16_t*)x, ldx, (int)m, y, ldy);
    return launch_status("tgm_dec_gemv_bf16");
  }
  const int rows_per_wave = m == 1 ? 1 : 4;
  const int64_t waves = (n + rows_per_wave - 1) / rows_per_wave;
  const unsigned blocks = (unsigned)((waves + 3) / 4 < 512 ? (waves + 3) / 4 : 512);
  const hipStream_t st = (hipStream_t)stream;
  const uint16_t* wp = (const uint16_t*)w;
  const uint16_t* xp = (const uint16_t*)x;
  switch (m) {
#define TGM_GV(MM)                                                                                                \
  case MM:                                                                                                        \
    hipLaunchKernelGGL((dec_gemv_bf16<MM, MM == 1 ? 1 : 4>), dim3(blocks), dim3(256), 0, st, wp, (int)n, (int)k, xp, \
                       ldx, y, ldy);                                                                              \
    break;
    TGM_GV(1) TGM_GV(2) TGM_GV(3) TGM_GV(4) TGM_GV(5) TGM_GV(6) TGM_GV(7) TGM_GV(8)
#undef TGM_GV
  }
  return launch_status("tgm_dec_gemv_bf16");
}

extern "C" int tgm_dec_argmax(const float* logits, int64_t rows, int64_t n, int64_t ld, int32_t* tokens, int32_t* pos,
                              int32_t* history, int64_t hist_stride, int64_t hist_base, void* stream) {
  clear_error();
  TGM_CHECK_ARG(logits && tokens, "null operand");
  TGM_CHECK_ARG(rows >= 0 && n > 0 && n < (1ll << 31) && (rows <= 1 || ld >= n), "invalid logits shape");
  TGM_CHECK_ARG(!history || (pos && hist_stride > 0), "history needs positions and a positive stride");
  if (rows == 0) return TGM_OK;
  hipLaunchKernelGGL(dec_argmax, dim3((unsigned)rows), dim3(1024), 0, (hipStream_t)stream, logits, (int)n, ld, tokens, pos,
                     history, hist_stride, hist_base);
  return launch_status("tgm_dec_argmax");
}
