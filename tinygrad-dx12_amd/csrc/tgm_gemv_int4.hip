// Kernel family 1, integer path: INT4 / UINT4 weights with fp16 / bf16 / f32 group scales
// (groups of 32, 64 or 128) x fp16 activations -- e.g. the 4096 x 4096 decode GEMV (fp16 x, int4
// codes, fp16 scales per 32).
//
// Replaces the reference's thread-scope matvec / N=1 LinAlg matmul over weights that a
// separate kernel first decoded to fp32 (alexandreteles/tinygrad-dx12
// src/tinygrad_dx12/renderer/linalg.py:127-166, codegen/linalg.py:244-245,
// codegen/decomp/dx12.py:93-106).
//
//   Y[m, n] = sum_b s[n, b / G] * sum_{k in block b} X[m, k] * code[n, k]     (32-element blocks)
//
// Exactness: an fp16 activation times an int4 code is exact in the fp32 accumulator of
// v_mfma_f32_16x16x32_f16, and every MFMA here covers exactly one 32-element block, so the
// per-group scale can be applied to the block's exact partial sum with one fp32 FMA per
// output -- the reference forms code * scale in fp32 (exact for fp16 scales) and then sums,
// so only rounding order differs.  (A scale folded into an fp16/bf16 MFMA operand would
// round code * scale.)
//
// Layout: the weight is the MFMA B operand, so lane l holds weight row n0 + l % 16 both as
// an operand (8 codes: K [32 u + 8 q, + 8) of block u, q = l / 16) and in the result (D
// column l % 16, rows m = 4 q + v): the row's scale is a per-lane value.  Codes become fp16
// operands exactly: nibble u (p ^ 8 for int4) placed under the fp16 pattern 0x6400 is
// 1024 + u, minus 1024 (+ 8 for int4) in a packed f16 add.
#include "tgm_common.h"
#include "tgm_lanes.h"

namespace tgm {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float f32x4v __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

constexpr size_t kInt4MaxLds = 160 * 1024;

// 8 codes (one dword, low nibble first) -> 8 exact fp16 values in K order.  ``flip`` is
// 0x88888888 for int4 (p ^ 8 turns two's complement into an offset of 8) and 0 for uint4;
// ``bias`` is 1032 or 1024 in both halves.
__device__ __forceinline__ half8 int4_to_half8(unsigned d, unsigned flip, half2v bias) {
  d ^= flip;
  const unsigned lo = d & 0x0F0F0F0Fu;         // codes 0, 2, 4, 6
  const unsigned hi = (d >> 4) & 0x0F0F0F0Fu;  // codes 1, 3, 5, 7
  half8 out;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    // bytes: [lo.j, 0, hi.j, 0] (v_perm selector: 0-3 pick from lo, 4-7 from hi, 0x0c is zero)
    const unsigned sel = (unsigned)j | (0x0Cu << 8) | ((unsigned)(4 + j) << 16) | (0x0Cu << 24);
    const unsigned pair = __builtin_amdgcn_perm(hi, lo, sel) | 0x64006400u;
    const half2v h = __builtin_bit_cast(half2v, pair) - bias;
    out[2 * j] = h[0];
    out[2 * j + 1] = h[1];
  }
  return out;
}

// 8 codes (one dword, low nibble first) -> 8 exact fp16 values in the order [0, 4, 1, 5, 2, 6,
// 3, 7], 9 VALU instructions: one AND + XOR places two nibbles under the fp16 pattern 0x6400
// (1024 + v for the low nibble of a byte, 1024 + 16 v for the high one, v = u ^ 8 for int4: the
// sign flip is the XOR's 0x0008 / 0x0080 bits), and one packed f16 add (or multiply by 1/16 and
// add) removes the offset.  klo / khi are 0x64006400 with the flip bits, bias 1032 or 1024,
// bias16 72 or 64.  The activation operand is permuted to the same order (permute_x8).
__device__ __forceinline__ half8 int4_to_half8_pairs(unsigned d, unsigned klo, unsigned khi, half2v bias,
                                                     half2v bias16) {
  const unsigned d8 = d >> 8;
  const half2v a = __builtin_bit_cast(half2v, (d & 0x000F000Fu) ^ klo);   // codes 0, 4
  const half2v b = __builtin_bit_cast(half2v, (d & 0x00F000F0u) ^ khi);   // codes 1, 5 (x 16)
  const half2v c = __builtin_bit_cast(half2v, (d8 & 0x000F000Fu) ^ klo);  // codes 2, 6
  const half2v e = __builtin_bit_cast(half2v, (d8 & 0x00F000F0u) ^ khi);  // codes 3, 7 (x 16)
  const half2v inv16 = {(_Float16)0.0625f, (_Float16)0.0625f};
  const half2v h0 = a - bias, h1 = b * inv16 - bias16, h2 = c - bias, h3 = e * inv16 - bias16;
  return half8{h0[0], h0[1], h1[0], h1[1], h2[0], h2[1], h3[0], h3[1]};
}

// x0 .. x7 -> x0, x4, x1, x5, x2, x6, x3, x7 (the order int4_to_half8_pairs produces codes in)
__device__ __forceinline__ half8 permute_x8(half8 x) {
  const u32x4 w = __builtin_bit_cast(u32x4, x);
  const u32x4 o = {__builtin_amdgcn_perm(w[2], w[0], 0x05040100u), __builtin_amdgcn_perm(w[2], w[0], 0x07060302u),
                   __builtin_amdgcn_perm(w[3], w[1], 0x05040100u), __builtin_amdgcn_perm(w[3], w[1], 0x07060302u)};
  return __builtin_bit_cast(half8, o);
}

// Transpose 4 x 4 dwords across the four 16-lane rows of a wave: on return register r of
// lane row g holds what register g of lane row r held.  A lane that loaded 16 bytes (block
// g = its row, dwords 0..3) then holds dword g of blocks 0..3, one per MFMA.
__device__ __forceinline__ void transpose4(unsigned& r0, unsigned& r1, unsigned& r2, unsigned& r3) {
  swap32(r0, r2);  // rows 2,3 of r0 <-> rows 0,1 of r2
  swap32(r1, r3);
  swap16(r0, r1);  // odd rows of r0 <-> even rows of r1
  swap16(r2, r3);
}

// A workgroup owns rpw consecutive weight rows (rpw <= 16 NT) and holds NT x NK waves: wave
// (ti, ki) owns the 16-row tile starting at row blockIdx.x * rpw + 16 ti (rows past the
// workgroup's range are clamped to its last row and not stored) and the ki-th of NK
// contiguous slices of its 128-element super-steps (at most SMAX).  Each super-step lane
// (c, q) loads 16 bytes of row c -- block q of the four -- and the row's scales of the
// super-step's blocks (4 / G groups, one vector load); a lane-row
// transpose hands each MFMA u the dword q of block u.  D super-steps are in flight;
// refills past the slice re-read its last super-step, so every load is unconditional.  The
// activations are copied to LDS once ([M][K + 8] fp16) and each step's operands are read
// one step ahead.  G = blocks per scale group (1, 2 or 4).
template <int NT, int NK, int SMAX, int G, int SDT, int XP>
__global__ void __launch_bounds__(NT * NK * 64) gemv_int4(const uint8_t* __restrict__ w, int64_t N, int64_t K,
                                                        const uint8_t* __restrict__ scales, int64_t ngroups,
                                                        unsigned flip, float bias, const _Float16* __restrict__ x,
                                                        int M, int64_t ldx, void* __restrict__ y, int ydt, int64_t ldy,
                                                        int rpw) {
  constexpr int D = SMAX < 8 ? SMAX : 8;
  constexpr bool SCALED = SDT >= 0;
  constexpr int SSIZE = SDT == TGM_F32 ? 4 : 2;
  constexpr int SBYTES = 4 / G * SSIZE;  // scale bytes per row and super-step: 2 .. 16
  constexpr int SWORDS = SBYTES < 4 ? 1 : SBYTES / 4;
  constexpr int NW = NT * NK;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  float* partial = (float*)smem;                                       // [NW][64][4] when NK > 1
  _Float16* xs = (_Float16*)(smem + (NK > 1 ? NW * 64 * 4 * 4 : 0));  // [M][K + 8]
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ti = wave % NT, ki = wave / NT;
  const int c = lane & 15, q = lane >> 4;
  const int64_t wg0 = (int64_t)blockIdx.x * rpw;
  const int64_t wg_end = wg0 + rpw < N ? wg0 + rpw : N;  // rows of this workgroup: [wg0, wg_end)
  const int64_t n0 = wg0 + 16 * ti;
  const int64_t row = n0 + c < wg_end ? n0 + c : wg_end - 1;  // clamped rows are computed, not stored
  const int S = (int)(K / 128);
  const int per = (S + NK - 1) / NK;
  const int t_begin = ki * per < S ? ki * per : S;
  const int t_end = t_begin + per < S ? t_begin + per : S;
  const int nsteps = t_end - t_begin;
  const int t_last = nsteps > 0 ? t_end - 1 : 0;
  const uint8_t* wrow = w + row * (K / 2) + 16 * q;
  const uint8_t* srow = scales + (SCALED ? row * ngroups * SSIZE : 0);
  const half2v hbias = {(_Float16)bias, (_Float16)bias};

  // Activations to LDS (16-byte chunks; K % 128 == 0 and ldx % 8 == 0 on the host).  The
  // first XP passes (all of them when M x K fits) are loaded before the weight ring and
  // stored after it is issued: the vector memory counter retires in order, so a staging load
  // issued after the ring would wait for all of it.  Chunks past the end re-read the last one
  // and store nothing.
  const int64_t xstride = K + 8;
  const int chunks_per_row = (int)(K / 8);
  const int xtotal = M * chunks_per_row;
  u32x4 xv[XP];
#pragma unroll
  for (int it = 0; it < XP; ++it) {
    int i = (int)threadIdx.x + it * NW * 64;
    i = i < xtotal ? i : xtotal - 1;
    const int m = i / chunks_per_row, kc = i - m * chunks_per_row;
    xv[it] = *(const u32x4*)(x + m * ldx + 8 * kc);
  }
  u32x4 codes[D];
  unsigned sraw[D][SWORDS];
  auto load = [&](int j, int slot) __attribute__((always_inline)) {
    const int t = t_begin + j < t_last ? t_begin + j : t_last;
    codes[slot] = *(const u32x4*)(wrow + 64 * t);
    if constexpr (SCALED) {
      const uint8_t* p = srow + (int64_t)t * SBYTES;
      if constexpr (SBYTES == 2) {
        sraw[slot][0] = *(const uint16_t*)p;
      } else if constexpr (SBYTES == 4) {
        sraw[slot][0] = *(const unsigned*)p;
      } else if constexpr (SBYTES == 8) {
        const u32x2 v = *(const u32x2*)p;
        sraw[slot][0] = v[0]; sraw[slot][1] = v[1];
      } else {
        const u32x4 v = *(const u32x4*)p;
        sraw[slot][0] = v[0]; sraw[slot][1] = v[1]; sraw[slot][2] = v[2]; sraw[slot][3] = v[3];
      }
    }
  };
#pragma unroll
  for (int j = 0; j < D; ++j) load(j, j);

#pragma unroll
  for (int it = 0; it < XP; ++it) {
    const int i = (int)threadIdx.x + it * NW * 64;
    if (i < xtotal) {
      const int m = i / chunks_per_row, kc = i - m * chunks_per_row;
      *(u32x4*)(xs + m * xstride + 8 * kc) = xv[it];
    }
  }
  for (int i = (int)threadIdx.x + XP * NW * 64; i < xtotal; i += NW * 64) {
    const int m = i / chunks_per_row, kc = i - m * chunks_per_row;
    *(u32x4*)(xs + m * xstride + 8 * kc) = *(const u32x4*)(x + m * ldx + 8 * kc);
  }
  __syncthreads();
  const int xm = c < M ? c : 0;  // activation row feeding A row c (rows >= M are never stored)
  const _Float16* xl = xs + xm * xstride + 8 * q;

  // scale of group i (0 .. 4 / G - 1) of a super-step from its raw words
  auto scale_of = [&](const unsigned* raw, int i) __attribute__((always_inline)) {
    if constexpr (SSIZE == 4) {
      return __builtin_bit_cast(float, raw[i]);
    } else {
      const unsigned h = (raw[i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
      if constexpr (SDT == TGM_F16) return (float)__builtin_bit_cast(_Float16, (unsigned short)h);
      else return __builtin_bit_cast(float, h << 16);
    }
  };
  f32x4v acc = {0.f, 0.f, 0.f, 0.f};
  half8 xa[2][4];
  auto read_x = [&](int j, half8 out[4]) __attribute__((always_inline)) {
    const int t = t_begin + j < t_last ? t_begin + j : t_last;
#pragma unroll
    for (int u = 0; u < 4; ++u) out[u] = *(const half8*)(xl + 128 * t + 32 * u);
  };
  read_x(0, xa[0]);
  auto step = [&](int j) __attribute__((always_inline)) {
    unsigned d[4] = {codes[j % D][0], codes[j % D][1], codes[j % D][2], codes[j % D][3]};
    transpose4(d[0], d[1], d[2], d[3]);
    f32x4v part = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const half8 wb = int4_to_half8(d[u], flip, hbias);
      part = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[j & 1][u], wb, part, 0, 0, 0);
      if ((u + 1) % G == 0) {  // end of a scale group
        const float s = SCALED ? scale_of(sraw[j % D], u / G) : 1.0f;
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[v] = __builtin_fmaf(s, part[v], acc[v]);
        part = f32x4v{0.f, 0.f, 0.f, 0.f};
      }
    }
  };
#pragma unroll
  for (int j = 0; j < SMAX; ++j) {
    if (j + 1 < SMAX) read_x(j + 1, xa[(j + 1) & 1]);
    if (j < nsteps) step(j);
    if (j + D < SMAX) load(j + D, j % D);
    __builtin_amdgcn_sched_barrier(0);  // keep each refill right after its slot's MFMAs
  }
  if constexpr (NK > 1) {
#pragma unroll
    for (int v = 0; v < 4; ++v) partial[(wave * 64 + lane) * 4 + v] = acc[v];
    __syncthreads();
    if (ki != 0) return;
#pragma unroll
    for (int kk = 1; kk < NK; ++kk)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[v] += partial[((kk * NT + ti) * 64 + lane) * 4 + v];
  }
  // Lane (c, q) holds Y[4 q + v][n0 + c].
  if (n0 + c < wg_end) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = 4 * q + v;
      if (m < M) store_from_f32(y, ydt, (int64_t)m * ldy + n0 + c, acc[v]);
    }
  }
}

// Activations in registers, for K = 1024 KS (KS = 1, 2, 4) and 2 <= M <= 16 (the decoder's
// projections at batch 2-16).  A workgroup owns rpw <= 16 T consecutive weight rows as T
// 16-row tiles (rows past its range clamped to its last row, computed and not stored) and
// holds 8 waves; wave ki owns K super-steps [ki KS, ki KS + KS) of every tile.  Its MFMA A
// operands -- X rows c < M at the 16 blocks of its slice (zero for c >= M, whose D rows are
// never stored) -- are loaded once into 16 KS registers straight from global memory, so no
// workgroup stages X through LDS and no barrier precedes the first MFMA.  Then, for every
// tile, the slice's codes (one 16-byte load per lane and super-step, transposed across lane
// rows as in gemv_int4) and the row's scale groups of the slice (one vector load) are all
// issued before the first MFMA.  The 8 waves' partial tiles meet in LDS; wave t < T sums
// tile t and stores it.  Exactness and nibble order as in gemv_int4.
template <int T, int KS, int G, int SDT>
__global__ void __launch_bounds__(512) gemv_int4_xr(const uint8_t* __restrict__ w, int64_t N, int64_t K,
                                                   const uint8_t* __restrict__ scales, int64_t ngroups,
                                                   unsigned flip, float bias, const _Float16* __restrict__ x,
                                                   int M, int64_t ldx, void* __restrict__ y, int ydt, int64_t ldy,
                                                   int rpw) {
  constexpr bool SCALED = SDT >= 0;
  constexpr int SSIZE = SDT == TGM_F32 ? 4 : 2;
  constexpr int GPS = 4 / G;              // scale groups per super-step
  constexpr int SB = KS * GPS * SSIZE;    // scale bytes per row and slice: 2 .. 64
  constexpr int SW = SB < 4 ? 1 : SB / 4;
  __shared__ __attribute__((aligned(16))) float partial[8][T][64][4];
  const int lane = threadIdx.x & 63;
  const int ki = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15, q = lane >> 4;
  const int64_t wg0 = (int64_t)blockIdx.x * rpw;
  const int64_t wg_end = wg0 + rpw < N ? wg0 + rpw : N;  // rows of this workgroup: [wg0, wg_end)
  const int t0 = ki * KS;                                 // first super-step of the slice
  const half2v hbias = {(_Float16)bias, (_Float16)bias};
  const half2v hbias16 = {(_Float16)(bias - 960.f), (_Float16)(bias - 960.f)};
  const unsigned klo = 0x64006400u ^ (flip & 0x00080008u), khi = 0x64006400u ^ (flip & 0x00800080u);

  // MFMA u of a super-step takes the lane's K elements 32 u + 8 q .. + 8 (the codes transposed
  // across lane rows), or with one scale group per super-step (G = 4) 32 q + 8 u .. + 8 (the
  // lane's own codes, no transpose).  Lanes of rows c >= M load nothing (their D rows are never
  // stored): M x 1 KB per super-step of requests instead of 16 x 1 KB.
  constexpr bool TRANSPOSE = G < 4;
  half8 xa[KS][4];
  {
    const _Float16* xp = x + (int64_t)(c < M ? c : 0) * ldx + t0 * 128;
#pragma unroll
    for (int j = 0; j < KS; ++j)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int k = TRANSPOSE ? 32 * u + 8 * q : 32 * q + 8 * u;
        xa[j][u] = c < M ? permute_x8(*(const half8*)(xp + j * 128 + k)) : half8{};
      }
  }
  u32x4 codes[T][KS];
  unsigned sraw[T][SW];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int64_t n0 = wg0 + 16 * t;
    const int64_t row = n0 + c < wg_end ? n0 + c : wg_end - 1;
    const uint8_t* wrow = w + row * (K / 2) + t0 * 64 + 16 * q;
#pragma unroll
    for (int j = 0; j < KS; ++j) codes[t][j] = __builtin_nontemporal_load((const u32x4*)(wrow + 64 * j));
    if constexpr (SCALED) {
      const uint8_t* p = scales + row * ngroups * SSIZE + t0 * GPS * SSIZE;  // SB-aligned (host)
      if constexpr (SB == 2) {
        sraw[t][0] = *(const uint16_t*)p;
      } else if constexpr (SB == 4) {
        sraw[t][0] = *(const unsigned*)p;
      } else if constexpr (SB == 8) {
        const u32x2 v = *(const u32x2*)p;
        sraw[t][0] = v[0]; sraw[t][1] = v[1];
      } else {
#pragma unroll
        for (int i = 0; i < SB / 16; ++i) {
          const u32x4 v = *(const u32x4*)(p + 16 * i);
          sraw[t][4 * i] = v[0]; sraw[t][4 * i + 1] = v[1]; sraw[t][4 * i + 2] = v[2]; sraw[t][4 * i + 3] = v[3];
        }
      }
    }
  }
  // Every load is issued before any of them is used: without this barrier the scheduler pulls
  // the first transpose's register copies up behind the first code load, and its wait for
  // that load holds back every load after it.
  __builtin_amdgcn_sched_barrier(0);
  // scale of group g (0 .. KS GPS - 1) of the slice from tile t's raw words
  auto scale_of = [&](int t, int g) __attribute__((always_inline)) {
    if constexpr (SSIZE == 4) {
      return __builtin_bit_cast(float, sraw[t][g]);
    } else {
      const unsigned h = (sraw[t][g >> 1] >> (16 * (g & 1))) & 0xFFFFu;
      if constexpr (SDT == TGM_F16) return (float)__builtin_bit_cast(_Float16, (unsigned short)h);
      else return __builtin_bit_cast(float, h << 16);
    }
  };
  f32x4v acc[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    acc[t] = f32x4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KS; ++j) {
      unsigned d[4] = {codes[t][j][0], codes[t][j][1], codes[t][j][2], codes[t][j][3]};
      if constexpr (TRANSPOSE) transpose4(d[0], d[1], d[2], d[3]);
      f32x4v part = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const half8 wb = int4_to_half8_pairs(d[u], klo, khi, hbias, hbias16);
        part = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[j][u], wb, part, 0, 0, 0);
        if ((u + 1) % G == 0) {  // end of a scale group
          const float s = SCALED ? scale_of(t, j * GPS + u / G) : 1.0f;
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[t][v] = __builtin_fmaf(s, part[v], acc[t][v]);
          part = f32x4v{0.f, 0.f, 0.f, 0.f};
        }
      }
    }
  }
#pragma unroll
  for (int t = 0; t < T; ++t) *(f32x4v*)partial[ki][t][lane] = acc[t];
  __syncthreads();
  if (ki >= T) return;
  const int t = ki;  // this wave sums and stores tile t
  f32x4v sum = *(const f32x4v*)partial[0][t][lane];
#pragma unroll
  for (int kk = 1; kk < 8; ++kk) {
    const f32x4v p = *(const f32x4v*)partial[kk][t][lane];
#pragma unroll
    for (int v = 0; v < 4; ++v) sum[v] += p[v];
  }
  // Lane (c, q) holds Y[4 q + v][n0 + c].
  const int64_t n0 = wg0 + 16 * t;
  if (n0 + c < wg_end) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = 4 * q + v;
      if (m < M) store_from_f32(y, ydt, (int64_t)m * ldy + n0 + c, sum[v]);
    }
  }
}

template <int T, int KS, int G, int SDT>
int launch_int4_xr_t(unsigned grid, hipStream_t s, const void* w, int64_t n, int64_t k, const void* scales,
                     int64_t ngroups, bool sgn, const void* x, int64_t m, int64_t ldx, void* y, int ydt, int64_t ldy,
                     int rpw) {
  hipLaunchKernelGGL((gemv_int4_xr<T, KS, G, SDT>), dim3(grid), dim3(512), 0, s, (const uint8_t*)w, n, k,
                     (const uint8_t*)scales, ngroups, sgn ? 0x88888888u : 0u, sgn ? 1032.0f : 1024.0f,
                     (const _Float16*)x, (int)m, ldx, y, ydt, ldy, rpw);
  return TGM_OK;
}

// gemv_int4_xr for K = 1024 KS (KS = 1, 2, 4: a slice's scale bytes are then a power of two,
// and so is their alignment): T tiles per workgroup so that one round of CUs covers the rows
// when it can (at most 4 tiles), spread evenly over whole rounds.
template <int G, int SDT>
int launch_int4_xr(bool sgn, hipStream_t s, const void* w, int64_t n, int64_t k, const void* scales, int64_t ngroups,
                   const void* x, int64_t m, int64_t ldx, void* y, int ydt, int64_t ldy) {
  const int ks = (int)(k / 1024);
  const int64_t tiles = (n + 15) / 16;
  const int cus = stream_cu_count(s);
  const int64_t per_cu = cus > 0 ? (tiles + cus - 1) / cus : 4;
  const int tt = per_cu <= 1 ? 1 : per_cu <= 2 ? 2 : 4;
  int rpw = 16 * tt;
  int64_t wgs = (n + rpw - 1) / rpw;
  if (cus > 0 && wgs % cus != 0) {
    const int64_t rounds = (wgs + cus - 1) / cus;
    const int64_t even = ((n + rounds * cus - 1) / (rounds * cus) + 3) / 4 * 4;
    if (even > 16 * (tt - 1) && even < rpw) {
      rpw = (int)even;
      wgs = (n + rpw - 1) / rpw;
    }
  }
  const unsigned grid = (unsigned)wgs;
#define TGM_XR(TT, KK)                                                                                              \
  if (tt == TT && ks == KK)                                                                                         \
    return launch_int4_xr_t<TT, KK, G, SDT>(grid, s, w, n, k, scales, ngroups, sgn, x, m, ldx, y, ydt, ldy, rpw);
  TGM_XR(1, 1) TGM_XR(1, 2) TGM_XR(1, 4)
  TGM_XR(2, 1) TGM_XR(2, 2) TGM_XR(2, 4)
  TGM_XR(4, 1) TGM_XR(4, 2) TGM_XR(4, 4)
#undef TGM_XR
  return TGM_E_UNSUPPORTED;
}

template <int NT, int NK, int G, int SDT>
int launch_int4_shape(unsigned grid, hipStream_t s, const void* w, int64_t n, int64_t k, const void* scales,
                      int64_t ngroups, bool sgn, const void* x, int64_t m, int64_t ldx, void* y, int ydt, int64_t ldy,
                      int per, int rpw) {
  const size_t lds = (NK > 1 ? NT * NK * 64 * 16 : 0) + (size_t)m * (size_t)(k + 8) * 2;
  if (lds > kInt4MaxLds) return TGM_E_UNSUPPORTED;
  const int64_t passes = (m * (k / 8) + NT * NK * 64 - 1) / (NT * NK * 64);  // staging passes
  const int xp = passes <= 2 ? 2 : passes <= 8 ? 8 : 16;
#define TGM_INT4(SMAX)                                                                                              \
  if (per <= SMAX) {                                                                                                \
    auto kernel = xp == 2 ? gemv_int4<NT, NK, SMAX, G, SDT, 2>                                                    \
                          : xp == 8 ? gemv_int4<NT, NK, SMAX, G, SDT, 8> : gemv_int4<NT, NK, SMAX, G, SDT, 16>;  \
    if (lds > 64 * 1024) {                                                                                          \
      static bool raised[3] = {};                                                                                   \
      if (!raised[xp / 8]) {                                                                                              \
        const hipError_t err = hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, \
                                                   (int)kInt4MaxLds);                                               \
        if (err != hipSuccess) {                                                                                    \
          set_error("tgm_gemv: cannot raise the LDS limit: %s", hipGetErrorString(err));                           \
          return (int)err;                                                                                          \
        }                                                                                                           \
        raised[xp / 8] = true;                                                                                            \
      }                                                                                                             \
    }                                                                                                               \
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(NT * NK * 64), lds, s,                                              \
                       (const uint8_t*)w, n, k, (const uint8_t*)scales, ngroups, sgn ? 0x88888888u : 0u,            \
                       sgn ? 1032.0f : 1024.0f, (const _Float16*)x, (int)m, ldx, y, ydt, ldy, rpw);                 \
    return TGM_OK;                                                                                                  \
  }
  TGM_INT4(4) TGM_INT4(8) TGM_INT4(16)
#undef TGM_INT4
  return TGM_E_UNSUPPORTED;
}

template <int G, int SDT>
int launch_int4_g(bool sgn, hipStream_t s, const void* w, int64_t n, int64_t k, const void* scales, int64_t ngroups,
                  const void* x, int64_t m, int64_t ldx, void* y, int ydt, int64_t ldy) {
  const int64_t tiles = (n + 15) / 16, S = k / 128;
  // 8 waves per workgroup as NT tiles x NK slices of K.  Every workgroup stages all of X, so
  // the more tiles there are, the more of them a workgroup takes (NT) before K is split
  // (NK): 6144 x 4096 at M = 8 took 9.4 us with one tile and 8 slices per workgroup.
  static const int order_big[3][2] = {{4, 2}, {2, 4}, {1, 8}};
  static const int order_mid[3][2] = {{2, 4}, {1, 8}, {4, 2}};
  static const int order_small[3][2] = {{1, 8}, {2, 4}, {4, 2}};
  const int(*order)[2] = tiles >= 768 ? order_big : tiles >= 384 ? order_mid : order_small;
  int nt = 0, nk = 0, per = 0;
  for (int i = 0; i < 3 && nt == 0; ++i) {
    const int p = (int)((S + order[i][1] - 1) / order[i][1]);
    if (p <= 16) nt = order[i][0], nk = order[i][1], per = p;
  }
  if (nt == 0) return TGM_E_UNSUPPORTED;
  // Rows per workgroup: 16 NT, unless the workgroups would leave part of the last round of
  // CUs idle; then the rows are spread evenly over whole rounds (a multiple of 4 rows each,
  // every tile of the shape keeping rows).
  int rpw = 16 * nt;
  int64_t wgs = (n + rpw - 1) / rpw;
  const int cus = stream_cu_count(s);
  if (cus > 0 && wgs % cus != 0) {
    const int64_t rounds = (wgs + cus - 1) / cus;
    const int64_t even = ((n + rounds * cus - 1) / (rounds * cus) + 3) / 4 * 4;
    if (even > 16 * (nt - 1) && even < rpw) {
      rpw = (int)even;
      wgs = (n + rpw - 1) / rpw;
    }
  }
  const unsigned grid = (unsigned)wgs;
  switch (nk) {
    case 2: return launch_int4_shape<4, 2, G, SDT>(grid, s, w, n, k, scales, ngroups, sgn, x, m, ldx, y, ydt, ldy, per, rpw);
    case 4: return launch_int4_shape<2, 4, G, SDT>(grid, s, w, n, k, scales, ngroups, sgn, x, m, ldx, y, ydt, ldy, per, rpw);
    default: return launch_int4_shape<1, 8, G, SDT>(grid, s, w, n, k, scales, ngroups, sgn, x, m, ldx, y, ydt, ldy, per, rpw);
  }
}

// INT4/UINT4 GEMV with fp16 activations; TGM_E_UNSUPPORTED when the operands do not fit it.
int launch_gemv_int4(hipStream_t s, const void* w, int fmt, int64_t n, int64_t k, const void* scales, int sdt,
                     int64_t bs, const void* x, int xdt, int64_t m, int64_t ldx, void* y, int ydt, int64_t ldy) {
  if (fmt != TGM_FMT_INT4 && fmt != TGM_FMT_UINT4) return TGM_E_UNSUPPORTED;
  if (xdt != TGM_F16 || k % 128 != 0 || ldx % 8 != 0 || (uintptr_t)x % 16 || (uintptr_t)w % 16) return TGM_E_UNSUPPORTED;
  if (m > 1 && ldx * m >= (1ll << 40)) return TGM_E_UNSUPPORTED;
  const int g = scales ? (int)(bs / 32) : 4;
  if (scales && (bs % 32 != 0 || (g != 1 && g != 2 && g != 4))) return TGM_E_UNSUPPORTED;
  if (scales && sdt != TGM_F16 && sdt != TGM_BF16 && sdt != TGM_F32) return TGM_E_UNSUPPORTED;
  if (scales && (uintptr_t)scales % (4 / g * dtype_size(sdt))) return TGM_E_UNSUPPORTED;  // one vector load per step
  const int64_t ngroups = scales ? k / bs : 0;
  const bool sg = fmt == TGM_FMT_INT4;
  // K = 1024, 2048 or 4096: activations in registers (gemv_int4_xr), whose scale loads take a
  // row's groups of a K slice at once (aligned to their size, at most 16 bytes)
  const int64_t slice_bytes = scales ? k / 1024 * (4 / g) * dtype_size(sdt) : 0;
  const bool xr = m >= 2 && (k == 1024 || k == 2048 || k == 4096) &&
                  (!scales || (uintptr_t)scales % (slice_bytes < 16 ? slice_bytes : 16) == 0);
#define TGM_SDT(SDT)                                                                                                 \
  if (xr)                                                                                                            \
    return g == 1   ? launch_int4_xr<1, SDT>(sg, s, w, n, k, scales, ngroups, x, m, ldx, y, ydt, ldy)               \
           : g == 2 ? launch_int4_xr<2, SDT>(sg, s, w, n, k, scales, ngroups, x, m, ldx, y, ydt, ldy)               \
                    : launch_int4_xr<4, SDT>(sg, s, w, n, k, scales, ngroups, x, m, ldx, y, ydt, ldy);              \
  return g == 1   ? launch_int4_g<1, SDT>(sg, s, w, n, k, scales, ngroups, x, m, ldx, y, ydt, ldy)                 \
         : g == 2 ? launch_int4_g<2, SDT>(sg, s, w, n, k, scales, ngroups, x, m, ldx, y, ydt, ldy)                 \
                  : launch_int4_g<4, SDT>(sg, s, w, n, k, scales, ngroups, x, m, ldx, y, ydt, ldy)
  if (!scales) { TGM_SDT(-1); }
  switch (sdt) {
    case TGM_F16: TGM_SDT(TGM_F16);
    case TGM_BF16: TGM_SDT(TGM_BF16);
    default: TGM_SDT(TGM_F32);
  }
#undef TGM_SDT
}

}  // namespace tgm
