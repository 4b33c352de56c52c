// Kernel family 1, single-row decode path (M = 1): FP4 E2M1 weights with E8M0 (or no)
// block-32 scales x bf16 activations, streamed row-contiguously and reduced on the VALU.
//
//   y[n] = sum_k x[k] * deq(W)[n, k]
//
// With one activation row an MFMA tile wastes 15 of its 16 columns, and an MFMA operand
// layout forces every load instruction to touch 16 weight rows.  Here a wave owns R
// consecutive rows -- R * K/2 contiguous bytes -- and reads them 1 KB per instruction in
// address order: lane l of instruction i gets bytes [16 l, 16 l + 16) of half-row (i % IPR)
// of row i / IPR (IPR = K / 2048 instructions per row), i.e. the 32 codes
// K [2048 h + 32 l, + 32) -- exactly one MX block, so one E8M0 byte per lane and row.
// Every lane therefore needs the same activations for every row: 32 bf16 per half-row,
// loaded once into registers.  Codes become bf16 pairs with v_cvt_scalef32_pk_bf16_fp4 (the
// E8M0 scale folded in exactly) and meet the activations in v_dot2_f32_bf16, whose bf16 x
// bf16 products are exact in fp32.  Per-lane row partials are reduced across the wave by a
// register-halving butterfly (each exchange moves useful data), one lane per row stores.
//
// Replaces the reference's thread-scope matvec / N=1 LinAlg matmul over a weight a
// separate kernel first decoded to fp32 (alexandreteles/tinygrad-dx12
// src/tinygrad_dx12/renderer/linalg.py:127-166, codegen/linalg.py:244-245,
// codegen/decomp/dx12.py:49-106).
#include "../../include/tgm_decoder.h"
#include "tgm_common.h"
#include "tgm_lanes.h"

namespace tgm {

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2r;
typedef unsigned u32x4r __attribute__((ext_vector_type(4)));

// Sum 8 per-lane partials (one per row) over the 64 lanes of a wave.  Two permlane swaps
// fold lane halves and 16-lane rows pairwise (each swap exchanges exactly the half of two
// registers the other side needs, so one add per register completes the stage), a DPP
// stage halves once more, and three DPP exchanges finish the sum within groups of 8 lanes.
// Lane l ends with row reduce_row8(l).
__device__ __forceinline__ float reduce_rows8(float (&a)[8], int lane) {
  float b[4], c[2];
#pragma unroll
  for (int r = 0; r < 4; ++r) {  // lanes 0-31 keep rows 0-3, lanes 32-63 rows 4-7
    float lo = a[r], hi = a[r + 4];
    swap32(lo, hi);
    b[r] = lo + hi;
  }
#pragma unroll
  for (int r = 0; r < 2; ++r) {  // even 16-lane rows keep b[r], odd rows b[r + 2]
    float lo = b[r], hi = b[r + 2];
    swap16(lo, hi);
    c[r] = lo + hi;
  }
  const bool up8 = lane & 8;  // lanes with bit 3 keep c[1]
  float v = (up8 ? c[1] : c[0]) + xor8(up8 ? c[0] : c[1]);
  v += xor4(v);
  v += xor2(v);
  v += xor1(v);
  return v;
}
__device__ __forceinline__ int reduce_row8(int lane) {
  return ((lane >> 5) & 1) << 2 | ((lane >> 4) & 1) << 1 | ((lane >> 3) & 1);
}

// The same for 4 rows: lane l ends with row reduce_row4(l) after folds over lane bits 5, 4.
__device__ __forceinline__ float reduce_rows4(float (&a)[4], int lane) {
  float b[2];
#pragma unroll
  for (int r = 0; r < 2; ++r) {  // lanes 0-31 keep rows 0-1, lanes 32-63 rows 2-3
    float lo = a[r], hi = a[r + 2];
    swap32(lo, hi);
    b[r] = lo + hi;
  }
  float lo = b[0], hi = b[1];  // even 16-lane rows keep b[0], odd rows b[1]
  swap16(lo, hi);
  float v = lo + hi;
  v += xor8(v);
  v += xor4(v);
  v += xor2(v);
  v += xor1(v);
  return v;
}
__device__ __forceinline__ int reduce_row4(int lane) { return ((lane >> 5) & 1) << 1 | ((lane >> 4) & 1); }

template <int R>
__device__ __forceinline__ float reduce_rows(float (&a)[R], int lane) {
  if constexpr (R == 8) return reduce_rows8(a, lane);
  else return reduce_rows4(a, lane);
}
template <int R>
__device__ __forceinline__ int reduce_row(int lane) {
  return R == 8 ? reduce_row8(lane) : reduce_row4(lane);
}

// Residual add + RMSNorm in front of a one-row GEMV (a decoder layer's norm and projection
// in one launch): x = (h + delta) / rms(h + delta) * w_norm, with h + delta stored to h_out by
// workgroup 0.  Each workgroup normalises the row once: thread t holds the float4 chunks
// [1024 j + 4 t, + 4) for j < 2 IPR (K = 2048 IPR values), the sum of squares is reduced over
// the wave and then over the four waves through LDS, and x goes to LDS, rounded to the GEMV's
// activation type, in its natural order, where the waves read it as they would read x from
// memory.  The loads of h, delta and w_norm are issued before the weight stream's first loads,
// so waiting for them does not wait for the weights (the vector memory counter retires in
// order), and the norm is computed while the weights are in flight.  Same arithmetic as
// dec_add_rmsnorm: x * (1 / sqrt(sum(x^2) / K + eps)) * w in fp32.
struct RowsNorm {
  const float* h = nullptr;
  const float* delta = nullptr;  // may be null
  const uint16_t* w = nullptr;   // bf16 norm weight
  float eps = 0.f;
  float* h_out = nullptr;        // may be null
};

typedef float f32x4n __attribute__((ext_vector_type(4)));
typedef unsigned u32x2n __attribute__((ext_vector_type(2)));

template <int IPR>
struct NormRegs {
  f32x4n a[2 * IPR], b[2 * IPR];
  u32x2n w[2 * IPR];
};

template <int IPR>
__device__ __forceinline__ void norm_issue(const RowsNorm& nm, NormRegs<IPR>& r) {
  const int t = threadIdx.x;
  const float* d = nm.delta ? nm.delta : nm.h;  // unconditional loads; the sum selects
#pragma unroll
  for (int j = 0; j < 2 * IPR; ++j) {
    const int o = 1024 * j + 4 * t;
    r.a[j] = *(const f32x4n*)(nm.h + o);
    r.b[j] = *(const f32x4n*)(d + o);
    r.w[j] = *(const u32x2n*)(nm.w + o);
  }
}

// LDS-only workgroup barrier: outstanding global loads (the weight stream) stay in flight.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <int IPR, typename T>
__device__ __forceinline__ void norm_finish(const RowsNorm& nm, const NormRegs<IPR>& r, T* xs, float* red) {
  constexpr int K = 2048 * IPR;
  const int t = threadIdx.x;
  const bool add = nm.delta != nullptr;
  f32x4n v[2 * IPR];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < 2 * IPR; ++j) {
    v[j] = add ? f32x4n{r.a[j][0] + r.b[j][0], r.a[j][1] + r.b[j][1], r.a[j][2] + r.b[j][2], r.a[j][3] + r.b[j][3]}
               : r.a[j];
#pragma unroll
    for (int e = 0; e < 4; ++e) ss += v[j][e] * v[j][e];
  }
  if (blockIdx.x == 0 && nm.h_out) {
#pragma unroll
    for (int j = 0; j < 2 * IPR; ++j) *(f32x4n*)(nm.h_out + 1024 * j + 4 * t) = v[j];
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
  if ((t & 63) == 0) red[t >> 6] = ss;
  lds_barrier();
  ss = (red[0] + red[1]) + (red[2] + red[3]);
  const float inv = 1.0f / sqrtf(ss / (float)K + nm.eps);
#pragma unroll
  for (int j = 0; j < 2 * IPR; ++j) {
    T o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const unsigned bits = (r.w[j][e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
      o[e] = (T)(v[j][e] * inv * __builtin_bit_cast(float, bits << 16));
    }
    *(u32x2n*)(xs + 1024 * j + 4 * t) = __builtin_bit_cast(u32x2n, o);
  }
  lds_barrier();
}

// Activations for the one-row kernels, staged once per 256-thread workgroup: K = 2048 IPR
// 16-bit values = IPR 16-byte chunks per thread, issued before the weight stream (so that
// waiting for them does not wait for the weights: the vector memory counter retires in order)
// and written to LDS once they land, where every wave reads the values its lanes need.
template <int IPR>
__device__ __forceinline__ void stage_issue(const unsigned char* x, u32x4r (&xg)[IPR]) {
#pragma unroll
  for (int j = 0; j < IPR; ++j) xg[j] = *(const u32x4r*)(x + 4096 * j + 16 * threadIdx.x);
}
template <int IPR>
__device__ __forceinline__ void stage_finish(const u32x4r (&xg)[IPR], unsigned char* xs) {
#pragma unroll
  for (int j = 0; j < IPR; ++j) *(u32x4r*)(xs + 4096 * j + 16 * threadIdx.x) = xg[j];
  lds_barrier();
}

// One wave per R (8 or 4) rows, four waves per workgroup; IPR instructions per row
// (K = 2048 IPR); D loads in flight per wave.
// SWIGLU: rows 2 i and 2 i + 1 are the gate and up rows of output i, which becomes
// silu(gate) * up (the two rows are reduced in lanes l and l ^ 8 for R = 8, l ^ 16 for R = 4).
// NORM: x is RMSNorm(h + delta) * w_norm (RowsNorm), rounded to bf16 as it is staged.
template <int R, int IPR, int D, bool SCALED, bool SWIGLU = false, bool NORM = false>
__global__ void __launch_bounds__(256) gemv_rows_fp4(const uint8_t* __restrict__ w, int64_t N,
                                                   const uint8_t* __restrict__ scales, const __bf16* __restrict__ x,
                                                   void* __restrict__ y, int ydt, RowsNorm nm) {
  constexpr int NI = R * IPR;  // load instructions per wave
  constexpr int K = 2048 * IPR, KB = K / 32;
  const int lane = threadIdx.x & 63;
  const int64_t r0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
  // activations: lane l needs K [2048 h + 32 l, + 32) for every half-row h
  // (loaded as pairs; the compiler merges them into 16-byte loads.  Extracting the lanes of
  // a 4-dword vector and bit-casting each to a bf16 pair was miscompiled into one repeated
  // pair by the ROCm 7.2 compiler.)
  bf16x2r xr[IPR][16];
  auto load_x = [&](const __bf16* src) __attribute__((always_inline)) {
#pragma unroll
    for (int h = 0; h < IPR; ++h) {
      const bf16x2r* xp = (const bf16x2r*)(src + 2048 * h + 32 * lane);
#pragma unroll
      for (int j = 0; j < 16; ++j) xr[h][j] = xp[j];
    }
  };
  // x reaches the waves through LDS: the workgroup reads it from memory once (IPR 16-byte
  // chunks per thread) instead of every wave reading all of it
  NormRegs<NORM ? IPR : 1> nr;
  __shared__ __attribute__((aligned(16))) __bf16 xs[K];
  __shared__ float red[4];
  u32x4r xg[NORM ? 1 : IPR];
  if constexpr (NORM) norm_issue<IPR>(nm, nr);
  else stage_issue<IPR>((const unsigned char*)x, xg);
  auto row_of = [&](int i) __attribute__((always_inline)) {
    const int64_t r = r0 + i / IPR;
    return r < N ? r : N - 1;  // rows past N re-read the last row; they are not stored
  };
  // Scales: lane l of instruction i needs the E8M0 byte of block 64 (i % IPR) + l of row
  // i / IPR.  For each instruction the wave's 64 lanes read 64 consecutive bytes, one byte
  // load per instruction issued before the weight stream (rows past N re-read the last row).
  // Loading the wave's scale bytes as 16-byte chunks and handing them out through LDS cost
  // 0.1 us more at 14336 x 4096 (the LDS round trip and its wave barrier).
  unsigned sbyte[NI];
  if constexpr (SCALED) {
#pragma unroll
    for (int i = 0; i < NI; ++i)
      sbyte[i] = __builtin_nontemporal_load(scales + row_of(i) * KB + 64 * (i % IPR) + lane);
  }
  u32x4r codes[D];
  auto load = [&](int i, int slot) __attribute__((always_inline)) {
    const int64_t r = row_of(i);
    const int h = i % IPR;
    codes[slot] = __builtin_nontemporal_load((const u32x4r*)(w + r * (K / 2) + 1024 * h + 16 * lane));
  };
#pragma unroll
  for (int i = 0; i < D; ++i) load(i, i);
  if constexpr (NORM) norm_finish<IPR>(nm, nr, xs, red);
  else stage_finish<IPR>(xg, (unsigned char*)xs);
  load_x(xs);
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int slot = i % D, h = i % IPR;
    const float s = __builtin_bit_cast(float, (SCALED ? sbyte[i] : 127u) << 23);
    float a[2] = {acc[i / IPR], 0.f};  // two chains halve the dependent-dot latency
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const unsigned cw = codes[slot][e];
      const bf16x2r p[4] = {__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(cw, s, 0),
                            __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(cw, s, 1),
                            __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(cw, s, 2),
                            __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(cw, s, 3)};
#pragma unroll
      for (int b = 0; b < 4; ++b) a[e >> 1] = __builtin_amdgcn_fdot2_f32_bf16(p[b], xr[h][4 * e + b], a[e >> 1], false);
    }
    acc[i / IPR] = a[0] + a[1];
    if (i + D < NI) load(i + D, slot);
    __builtin_amdgcn_sched_barrier(0);  // keep each refill right after the data it replaces is used
  }
  static_assert(R == 8 || R == 4, "the reduction folds 4 or 8 rows");
  const float v = reduce_rows<R>(acc, lane);
  const int64_t row = r0 + reduce_row<R>(lane);
  if constexpr (SWIGLU) {
    const float partner = R == 8 ? xor8(v) : __shfl_xor(v, 16, 64);  // row ^ 1
    if ((lane & (64 / R - 1)) == 0 && (row & 1) == 0 && row < N)
      store_from_f32(y, ydt, row >> 1, v / (1.0f + expf(-v)) * partner);
  } else {
    if ((lane & (64 / R - 1)) == 0 && row < N) store_from_f32(y, ydt, row, v);
  }
}

// ------------------------------------------------------------------ INT4 / UINT4
// Same row-streaming structure for 4-bit integer codes with fp16 activations and fp16 / bf16
// / f32 group scales (groups of 32, 64 or 128 along K).  Each code becomes an fp16 subnormal
// with one bitwise op: masking a dword with 0x000F000F leaves codes 0 and 4 at bits [3:0] of
// each half, i.e. the fp16 values u * 2^-24; masking with 0x00F000F0 leaves codes 1 and 5 as
// 16 u * 2^-24; the dword shifted right by 8 gives codes 2, 6 and 3, 7 the same way.  For
// int4 the mask is followed by an xor of bit 3 of each nibble (v_bitop3 does both), which
// stores u = code + 8, and the 8 * sum(x) this adds is taken off once per lane.  The
// activations are paired (x0, x4) (x1, x5) (x2, x6) (x3, x7) to match, once per wave.
// v_dot2_f32_f16 products of an fp16 subnormal (at most 4 significant bits) and an fp16
// activation are exact in fp32, so codes 0/2/4/6 and 1/3/5/7 accumulate in two fp32 chains
// scaled by 2^-24 and 2^-20, combined as chain0 + chain1 / 16 (exact scaling), multiplied by
// the group's scale in fp32, and the row sum is scaled back by 2^24 (exact) before storing.
// Nine VALU instructions per 8 codes: 1 shift, 4 bitop3 and 4 dot2.
typedef _Float16 half2r __attribute__((ext_vector_type(2)));

template <int SDT>
__device__ __forceinline__ float int4_scale(const unsigned char* p) {
  if constexpr (SDT == TGM_F16) return (float)*(const _Float16*)p;
  else if constexpr (SDT == TGM_BF16) return __builtin_bit_cast(float, (unsigned)*(const uint16_t*)p << 16);
  else if constexpr (SDT == TGM_F32) return *(const float*)p;
  else return 1.0f;
}

// R = 8 rows per wave; GS = log2(group size / 32); SDT = scale dtype (-1: unscaled).
template <int R, int IPR, int D, int SDT, bool NORM = false>
__global__ void __launch_bounds__(256) gemv_rows_int4(const uint8_t* __restrict__ w, int64_t N,
                                                    const uint8_t* __restrict__ scales, int GS, unsigned flip,
                                                    const _Float16* __restrict__ x, void* __restrict__ y,
                                                    int ydt, RowsNorm nm) {
  constexpr int NI = R * IPR;
  constexpr int K = 2048 * IPR;
  constexpr bool SCALED = SDT >= 0;
  constexpr int SSIZE = SDT == TGM_F32 ? 4 : 2;
  const int lane = threadIdx.x & 63;
  const int64_t r0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
  // activations K [2048 h + 32 l, + 32) as the pairs the codes come out in: dword e of
  // the lane's 16 bytes holds codes 8e .. 8e+7, paired (0,4) (1,5) (2,6) (3,7); bias[h]
  // = -8 sum(x) * 2^-24 over the lane's 32 activations of half-row h (int4; 0 for uint4)
  half2r xr[IPR][16];
  float bias[IPR];
  auto load_x = [&](const _Float16* src) __attribute__((always_inline)) {
    const half2r one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
    for (int h = 0; h < IPR; ++h) {
      const unsigned* xp = (const unsigned*)(src + 2048 * h + 32 * lane);
      float s0 = 0.f, s1 = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const unsigned p0 = xp[4 * e], p1 = xp[4 * e + 1], p2 = xp[4 * e + 2], p3 = xp[4 * e + 3];  // (0,1) (2,3) (4,5) (6,7)
        xr[h][4 * e + 0] = __builtin_bit_cast(half2r, __builtin_amdgcn_perm(p2, p0, 0x05040100u));  // x0, x4
        xr[h][4 * e + 1] = __builtin_bit_cast(half2r, __builtin_amdgcn_perm(p2, p0, 0x07060302u));  // x1, x5
        xr[h][4 * e + 2] = __builtin_bit_cast(half2r, __builtin_amdgcn_perm(p3, p1, 0x05040100u));  // x2, x6
        xr[h][4 * e + 3] = __builtin_bit_cast(half2r, __builtin_amdgcn_perm(p3, p1, 0x07060302u));  // x3, x7
        s0 = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2r, p0), one, s0, false);
        s1 = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2r, p1), one, s1, false);
        s0 = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2r, p2), one, s0, false);
        s1 = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2r, p3), one, s1, false);
      }
      bias[h] = flip ? -0x1p-21f * (s0 + s1) : 0.f;
    }
  };
  NormRegs<NORM ? IPR : 1> nr;
  __shared__ __attribute__((aligned(16))) _Float16 xs[K];
  __shared__ float red[4];
  u32x4r xg[NORM ? 1 : IPR];
  if constexpr (NORM) norm_issue<IPR>(nm, nr);  // RMSNorm(h + delta) * w_norm, rounded to fp16
  else stage_issue<IPR>((const unsigned char*)x, xg);
  auto row_of = [&](int i) __attribute__((always_inline)) {
    const int64_t r = r0 + i / IPR;
    return r < N ? r : N - 1;
  };
  // Scales: lane l of instruction i needs the scale of group (64 (i % IPR) + l) >> GS of row
  // i / IPR, read straight from memory before the weight stream (consecutive lanes read
  // consecutive scales, or the same one for groups of 64 and 128).
  const int ng = (K / 32) >> GS;  // groups per row
  float sv[NI];
  if constexpr (SCALED) {
#pragma unroll
    for (int i = 0; i < NI; ++i)
      sv[i] = int4_scale<SDT>(scales + (row_of(i) * ng + ((64 * (i % IPR) + lane) >> GS)) * SSIZE);
  }
  u32x4r codes[D];
  auto load = [&](int i, int slot) __attribute__((always_inline)) {
    const int64_t r = row_of(i);
    codes[slot] = __builtin_nontemporal_load((const u32x4r*)(w + r * (K / 2) + 1024 * (i % IPR) + 16 * lane));
  };
#pragma unroll
  for (int i = 0; i < D; ++i) load(i, i);
  if constexpr (NORM) norm_finish<IPR>(nm, nr, xs, red);
  else stage_finish<IPR>(xg, (unsigned char*)xs);
  load_x(xs);
  const unsigned xlo = flip & 0x00080008u, xhi = flip & 0x00800080u;  // bit 3 of the nibbles kept
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int slot = i % D, h = i % IPR;
    float a0 = bias[h], a1 = 0.f;  // codes 0,2,4,6 (units 2^-24) / 1,3,5,7 (units 2^-20)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const unsigned d = codes[slot][e], d8 = d >> 8;
      const half2r c0 = __builtin_bit_cast(half2r, __builtin_amdgcn_bitop3_b32(d, 0x000F000Fu, xlo, 0x6A));   // (d & m) ^ x: 0, 4
      const half2r c1 = __builtin_bit_cast(half2r, __builtin_amdgcn_bitop3_b32(d, 0x00F000F0u, xhi, 0x6A));   // 1, 5
      const half2r c2 = __builtin_bit_cast(half2r, __builtin_amdgcn_bitop3_b32(d8, 0x000F000Fu, xlo, 0x6A));  // 2, 6
      const half2r c3 = __builtin_bit_cast(half2r, __builtin_amdgcn_bitop3_b32(d8, 0x00F000F0u, xhi, 0x6A));  // 3, 7
      a0 = __builtin_amdgcn_fdot2(c0, xr[h][4 * e + 0], a0, false);
      a1 = __builtin_amdgcn_fdot2(c1, xr[h][4 * e + 1], a1, false);
      a0 = __builtin_amdgcn_fdot2(c2, xr[h][4 * e + 2], a0, false);
      a1 = __builtin_amdgcn_fdot2(c3, xr[h][4 * e + 3], a1, false);
    }
    const float part = __builtin_fmaf(a1, 0.0625f, a0);
    acc[i / IPR] = SCALED ? __builtin_fmaf(sv[i], part, acc[i / IPR]) : acc[i / IPR] + part;
    if (i + D < NI) load(i + D, slot);
    __builtin_amdgcn_sched_barrier(0);
  }
  const float v = reduce_rows<R>(acc, lane) * 0x1p24f;
  const int64_t row = r0 + reduce_row<R>(lane);
  if ((lane & (64 / R - 1)) == 0 && row < N) store_from_f32(y, ydt, row, v);
}

constexpr int kRowsPerWave = 8;

// M = 1 FP4 GEMV on the row-streaming kernel; TGM_E_UNSUPPORTED when the operands do not fit.
int launch_gemv_rows(hipStream_t s, const void* w, int fmt, int64_t n, int64_t k, const void* scales, int sdt,
                     int64_t bs, const void* x, int xdt, int64_t m, void* y, int ydt, bool swiglu) {
  if (fmt != TGM_FMT_FP4_E2M1 || m != 1 || xdt != TGM_BF16) return TGM_E_UNSUPPORTED;
  if (k % 2048 != 0 || k / 2048 > 8) return TGM_E_UNSUPPORTED;
  if (scales && (sdt != TGM_E8M0 || bs != 32)) return TGM_E_UNSUPPORTED;
  if ((uintptr_t)w % 16 || (uintptr_t)x % 16) return TGM_E_UNSUPPORTED;
  if (swiglu && (!scales || n % 2)) return TGM_E_UNSUPPORTED;
  const int ipr = (int)(k / 2048);
  // up to K = 8192 a wave takes 8 rows; longer rows (their activations fill IPR * 16 registers)
  // take 4 rows per wave.  At K = 14336 (a decoder's down projection) 8 of a wave's 28 loads in
  // flight beat 16 (batch-1 decode 0.3888 -> 0.3850 ms per step; 6 the same, 4, 12 and 20 slower)
#define TGM_ROWS(R, IPR, D)                                                                                        \
  if (ipr == IPR) {                                                                                                \
    const unsigned grid = (unsigned)((n + 4 * R - 1) / (4 * R));                                                   \
    if (swiglu)                                                                                                    \
      hipLaunchKernelGGL((gemv_rows_fp4<R, IPR, D, true, true>), dim3(grid), dim3(256), 0, s, (const uint8_t*)w,   \
                         n, (const uint8_t*)scales, (const __bf16*)x, y, ydt, RowsNorm{});                         \
    else if (scales)                                                                                               \
      hipLaunchKernelGGL((gemv_rows_fp4<R, IPR, D, true>), dim3(grid), dim3(256), 0, s, (const uint8_t*)w, n,      \
                         (const uint8_t*)scales, (const __bf16*)x, y, ydt, RowsNorm{});                            \
    else                                                                                                           \
      hipLaunchKernelGGL((gemv_rows_fp4<R, IPR, D, false>), dim3(grid), dim3(256), 0, s, (const uint8_t*)w, n,     \
                         (const uint8_t*)scales, (const __bf16*)x, y, ydt, RowsNorm{});                            \
    return TGM_OK;                                                                                                 \
  }
  TGM_ROWS(kRowsPerWave, 1, 8) TGM_ROWS(kRowsPerWave, 2, 16) TGM_ROWS(kRowsPerWave, 3, 16)
  TGM_ROWS(kRowsPerWave, 4, 16) TGM_ROWS(4, 5, 16) TGM_ROWS(4, 6, 16) TGM_ROWS(4, 7, 8) TGM_ROWS(4, 8, 16)
#undef TGM_ROWS
  return TGM_E_UNSUPPORTED;
}

// INT4 waves take 4 rows: with the subnormal decode, 8 rows per wave measured 9.1 against 8.5 us
// at 14336 x 4096 and 5.7 against 4.7 us at 4096 x 4096 (more waves hide the per-row latency).
constexpr int kRowsPerWaveInt4 = 4;

template <int IPR, int SDT>
void launch_rows_int4(unsigned grid, hipStream_t s, const void* w, int64_t n, const void* scales, int gs, bool sgn,
                      const void* x, void* y, int ydt) {
  constexpr int R = kRowsPerWaveInt4, D = R * IPR;  // every load in flight at once
  hipLaunchKernelGGL((gemv_rows_int4<R, IPR, D, SDT>), dim3(grid), dim3(256), 0, s, (const uint8_t*)w, n,
                     (const uint8_t*)scales, gs, sgn ? 0x88888888u : 0u, (const _Float16*)x, y, ydt, RowsNorm{});
}

template <int IPR>
void launch_rows_int4_sdt(int sdt, unsigned grid, hipStream_t s, const void* w, int64_t n, const void* scales, int gs,
                          bool sgn, const void* x, void* y, int ydt) {
  if (!scales) launch_rows_int4<IPR, -1>(grid, s, w, n, scales, gs, sgn, x, y, ydt);
  else if (sdt == TGM_F16) launch_rows_int4<IPR, TGM_F16>(grid, s, w, n, scales, gs, sgn, x, y, ydt);
  else if (sdt == TGM_BF16) launch_rows_int4<IPR, TGM_BF16>(grid, s, w, n, scales, gs, sgn, x, y, ydt);
  else launch_rows_int4<IPR, TGM_F32>(grid, s, w, n, scales, gs, sgn, x, y, ydt);
}

// M = 1 INT4/UINT4 x fp16 GEMV on the row-streaming kernel; TGM_E_UNSUPPORTED when it does not fit.
int launch_gemv_rows_int4(hipStream_t s, const void* w, int fmt, int64_t n, int64_t k, const void* scales, int sdt,
                          int64_t bs, const void* x, int xdt, int64_t m, void* y, int ydt) {
  if ((fmt != TGM_FMT_INT4 && fmt != TGM_FMT_UINT4) || m != 1 || xdt != TGM_F16) return TGM_E_UNSUPPORTED;
  if (k % 2048 != 0 || k / 2048 > 4) return TGM_E_UNSUPPORTED;
  int gs = 0;
  if (scales) {
    if (sdt != TGM_F16 && sdt != TGM_BF16 && sdt != TGM_F32) return TGM_E_UNSUPPORTED;
    if (bs != 32 && bs != 64 && bs != 128) return TGM_E_UNSUPPORTED;
    gs = bs == 32 ? 0 : bs == 64 ? 1 : 2;
    if ((uintptr_t)scales % 16 || (n * (k / bs) * dtype_size(sdt)) < 16) return TGM_E_UNSUPPORTED;
  }
  if ((uintptr_t)w % 16 || (uintptr_t)x % 16) return TGM_E_UNSUPPORTED;
  const unsigned grid = (unsigned)((n + 4 * kRowsPerWaveInt4 - 1) / (4 * kRowsPerWaveInt4));
  const bool sgn = fmt == TGM_FMT_INT4;
  switch (k / 2048) {
    case 1: launch_rows_int4_sdt<1>(sdt, grid, s, w, n, scales, gs, sgn, x, y, ydt); break;
    case 2: launch_rows_int4_sdt<2>(sdt, grid, s, w, n, scales, gs, sgn, x, y, ydt); break;
    case 3: launch_rows_int4_sdt<3>(sdt, grid, s, w, n, scales, gs, sgn, x, y, ydt); break;
    default: launch_rows_int4_sdt<4>(sdt, grid, s, w, n, scales, gs, sgn, x, y, ydt); break;
  }
  return TGM_OK;
}

}  // namespace tgm

namespace tgm {

// RMSNorm + one-row GEMV launches (K = 2048 or 4096).
template <int IPR>
static int launch_norm_rows(hipStream_t s, const void* w, int fmt, int64_t n, const void* scales, int sdt, int gs,
                            const RowsNorm& nm, void* y, int ydt, bool swiglu) {
  if (fmt == TGM_FMT_FP4_E2M1) {
    const unsigned grid = (unsigned)((n + 4 * kRowsPerWave - 1) / (4 * kRowsPerWave));
    constexpr int D = 8 * IPR;
    if (swiglu)
      hipLaunchKernelGGL((gemv_rows_fp4<kRowsPerWave, IPR, D, true, true, true>), dim3(grid), dim3(256), 0, s,
                         (const uint8_t*)w, n, (const uint8_t*)scales, (const __bf16*)nullptr, y, ydt, nm);
    else if (scales)
      hipLaunchKernelGGL((gemv_rows_fp4<kRowsPerWave, IPR, D, true, false, true>), dim3(grid), dim3(256), 0, s,
                         (const uint8_t*)w, n, (const uint8_t*)scales, (const __bf16*)nullptr, y, ydt, nm);
    else
      hipLaunchKernelGGL((gemv_rows_fp4<kRowsPerWave, IPR, D, false, false, true>), dim3(grid), dim3(256), 0, s,
                         (const uint8_t*)w, n, (const uint8_t*)scales, (const __bf16*)nullptr, y, ydt, nm);
    return TGM_OK;
  }
  // at K = 4096, 4 of a wave's 8 loads in flight: the norm's operand loads go first, and fewer
  // weight loads behind them measured faster in the batch-1 decode step (0.3946 -> 0.3878 ms),
  // while the plain one-row INT4 GEMV keeps all 8 (4 there cost 0.2-0.45 us per launch)
  constexpr int R = kRowsPerWaveInt4, D = IPR == 2 ? 4 : R * IPR;
  const unsigned grid = (unsigned)((n + 4 * R - 1) / (4 * R));
  const bool sgn = fmt == TGM_FMT_INT4;
#define TGM_NORM_I4(SDT)                                                                                          \
  hipLaunchKernelGGL((gemv_rows_int4<R, IPR, D, SDT, true>), dim3(grid), dim3(256), 0, s, (const uint8_t*)w, n,  \
                     (const uint8_t*)scales, gs, sgn ? 0x88888888u : 0u,                                     \
                     (const _Float16*)nullptr, y, ydt, nm)
  if (!scales) TGM_NORM_I4(-1);
  else if (sdt == TGM_F16) TGM_NORM_I4(TGM_F16);
  else if (sdt == TGM_BF16) TGM_NORM_I4(TGM_BF16);
  else TGM_NORM_I4(TGM_F32);
#undef TGM_NORM_I4
  return TGM_OK;
}

}  // namespace tgm

using namespace tgm;

extern "C" int tgm_dec_norm_gemv(const float* h, const float* delta, float* h_out, const void* norm_weight, float eps,
                                 const void* w, int fmt, int64_t n, int64_t k, const void* scales, int scale_dtype,
                                 int64_t block_size, void* y, int y_dtype, int swiglu, void* stream) {
  clear_error();
  TGM_CHECK_ARG(h && norm_weight && w && y, "null operand");
  TGM_CHECK_ARG(valid_format(fmt), "unknown packed format %d", fmt);
  TGM_CHECK_ARG(n >= 0 && k > 0 && block_size >= 1, "invalid sizes");
  TGM_CHECK_ARG(!h_out || (h_out != h && h_out != delta), "h_out must not alias h or delta");
  TGM_CHECK_ARG(!swiglu || n % 2 == 0, "swiglu needs interleaved gate and up rows (n even)");
  TGM_CHECK_ARG(y_dtype == TGM_BF16 || y_dtype == TGM_F16 || y_dtype == TGM_F32, "output must be bf16, f16 or f32");
  if (n == 0) return TGM_OK;
  if (k != 2048 && k != 4096) TGM_UNSUPPORTED("tgm_dec_norm_gemv: K must be 2048 or 4096");
  if ((uintptr_t)h % 16 || (delta && (uintptr_t)delta % 16) || (h_out && (uintptr_t)h_out % 16) ||
      (uintptr_t)norm_weight % 16 || (uintptr_t)w % 16)
    TGM_UNSUPPORTED("tgm_dec_norm_gemv: operands must be 16-byte aligned");
  int gs = 0;
  if (fmt == TGM_FMT_FP4_E2M1) {
    if (scales && (scale_dtype != TGM_E8M0 || block_size != 32))
      TGM_UNSUPPORTED("tgm_dec_norm_gemv: FP4 scales must be E8M0 per 32");
    if (swiglu && !scales) TGM_UNSUPPORTED("tgm_dec_norm_gemv: the SwiGLU epilogue needs scaled FP4 weights");
  } else if (fmt == TGM_FMT_INT4 || fmt == TGM_FMT_UINT4) {
    if (swiglu) TGM_UNSUPPORTED("tgm_dec_norm_gemv: the SwiGLU epilogue takes FP4 weights");
    if (scales) {
      if (scale_dtype != TGM_F16 && scale_dtype != TGM_BF16 && scale_dtype != TGM_F32)
        TGM_UNSUPPORTED("tgm_dec_norm_gemv: int4 scales must be f16, bf16 or f32");
      if (block_size != 32 && block_size != 64 && block_size != 128)
        TGM_UNSUPPORTED("tgm_dec_norm_gemv: int4 groups must be 32, 64 or 128");
      gs = block_size == 32 ? 0 : block_size == 64 ? 1 : 2;
      if ((uintptr_t)scales % 16 || n * (k / block_size) * dtype_size(scale_dtype) < 16)
        TGM_UNSUPPORTED("tgm_dec_norm_gemv: scales must be 16-byte aligned");
    }
  } else {
    TGM_UNSUPPORTED("tgm_dec_norm_gemv: FP4, INT4 or UINT4 weights only");
  }
  RowsNorm nm;
  nm.h = h;
  nm.delta = delta;
  nm.w = (const uint16_t*)norm_weight;
  nm.eps = eps;
  nm.h_out = h_out;
  const hipStream_t s = (hipStream_t)stream;
  const int st = k == 2048 ? launch_norm_rows<1>(s, w, fmt, n, scales, scale_dtype, gs, nm, y, y_dtype, swiglu != 0)
                           : launch_norm_rows<2>(s, w, fmt, n, scales, scale_dtype, gs, nm, y, y_dtype, swiglu != 0);
  return st == TGM_OK ? launch_status("tgm_dec_norm_gemv") : st;
}
