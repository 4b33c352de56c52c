// Streaming MX GEMV (kernel family 1, M > 1 or shapes the one-row kernels do not take),
// instantiated for FP4 E2M1, FP6 E2M3 and FP6 E3M2 weights in tgm_gemv_stream.hip.
#pragma once

#include <stdlib.h>

#include "tgm_common.h"

namespace tgm {


typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
typedef __attribute__((__vector_size__(32 * sizeof(__bf16)))) __bf16 bf16x32;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(6 * sizeof(int)))) int i32x6;
typedef __attribute__((__vector_size__(4 * sizeof(unsigned)))) unsigned u32x4;
typedef __attribute__((__vector_size__(2 * sizeof(unsigned)))) unsigned u32x2;

// ------------------------------------------------------------------ MFMA GEMV
// Operand layout.  A K "super-step" is 128 elements.  Inside a super-step, lane l (tile
// row r = l & 15, lane group q = l >> 4) owns the 32 consecutive K elements
// [32q, 32q + 32): one 16-byte load for FP4 (24 bytes for FP6) and exactly one E8M0
// scale when the block is 32.  MFMA s (s = 0..3) of the super-step consumes elements
// [32q + 8s, 32q + 8s + 8) of every lane group, so the four MFMAs together cover the
// 128 elements once.  The activation operand uses the same element order, so the
// permutation of K cancels in the dot product.
// D lane layout: lane l holds D[4q + i][l & 15], i.e. Y[m = l & 15][n0 + 4q + i].
template <int FMT>
__device__ __forceinline__ void dequant32(const unsigned* codes, float scale, bf16x8 out[4]) {
  if constexpr (FMT == TGM_FMT_FP4_E2M1) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(codes[s], scale, 0);
      bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(codes[s], scale, 1);
      bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(codes[s], scale, 2);
      bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(codes[s], scale, 3);
      out[s] = bf16x8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
    }
  } else {
    i32x6 v = {(int)codes[0], (int)codes[1], (int)codes[2], (int)codes[3], (int)codes[4], (int)codes[5]};
    bf16x32 d;
    if constexpr (FMT == TGM_FMT_FP6_E2M3) d = __builtin_amdgcn_cvt_scalef32_pk32_bf16_fp6(v, scale);
    else d = __builtin_amdgcn_cvt_scalef32_pk32_bf16_bf6(v, scale);
#pragma unroll
    for (int s = 0; s < 4; ++s)
      out[s] = bf16x8{d[8 * s + 0], d[8 * s + 1], d[8 * s + 2], d[8 * s + 3],
                      d[8 * s + 4], d[8 * s + 5], d[8 * s + 6], d[8 * s + 7]};
  }
}

// GEMV results are bf16, f16 or f32 (checked on the host); one rounding from fp32.
__device__ __forceinline__ void store_out(void* y, int ydt, int64_t i, float v) {
  if (ydt == TGM_BF16) ((uint16_t*)y)[i] = f32_to_bf16(v);
  else if (ydt == TGM_F16) ((_Float16*)y)[i] = (_Float16)v;
  else ((float*)y)[i] = v;
}

template <int FMT>
struct MfmaGemvTraits {
  static constexpr int kStepBytes = FMT == TGM_FMT_FP4_E2M1 ? 64 : 96;  // bytes per row per super-step
  static constexpr int kLaneBytes = kStepBytes / 4;                     // 16 or 24
  static constexpr int kLaneDwords = kLaneBytes / 4;                    // 4 or 6
};

// Scale layouts of the streaming GEMV.
constexpr int kScaleNone = 0, kScaleDword = 1, kScaleGroup4 = 2;

// 4-byte aligned 16-byte vector: global_load_dwordx4 needs only dword alignment on gfx950.
typedef unsigned u32x4a __attribute__((ext_vector_type(4), aligned(4)));

// Weight codes are read once per launch: non-temporal loads keep them from evicting the
// activations and scales that every workgroup reads from L2.
template <int FMT>
__device__ __forceinline__ void load_codes(const uint8_t* p, unsigned out[6]) {
  if constexpr (FMT == TGM_FMT_FP4_E2M1) {
    const u32x4 v = __builtin_nontemporal_load((const u32x4*)p);
    out[0] = v[0]; out[1] = v[1]; out[2] = v[2]; out[3] = v[3]; out[4] = 0; out[5] = 0;
  } else {
    const u32x2 a = __builtin_nontemporal_load((const u32x2*)p);
    const u32x2 b = __builtin_nontemporal_load((const u32x2*)(p + 8));
    const u32x2 c = __builtin_nontemporal_load((const u32x2*)(p + 16));
    out[0] = a[0]; out[1] = a[1]; out[2] = b[0]; out[3] = b[1]; out[4] = c[0]; out[5] = c[1];
  }
}

// Streaming MX GEMV.  A workgroup owns RPW consecutive weight rows (RPW <= 16 NT, a
// multiple of 4) and holds NT x NK waves: wave (ti, ki) owns the 16-row tile starting at
// row blockIdx.x * RPW + 16 ti (rows past the workgroup's range are clamped to its last
// row and not stored) and the ki-th of NK contiguous slices of its K super-steps, at most
// SMAX of them.  RPW below 16 NT spreads a matrix whose tile count is not a multiple of NT
// times the CU count evenly over the CUs (14336 rows: 256 workgroups of 56 rows instead of
// 224 of 64).  The slice is walked by a fully unrolled loop (all
// register indices are compile-time constants) with a ring of D super-steps of weights
// in flight: the load refilling a ring slot is issued right after the slot's MFMAs, so
// every wave keeps D x 1 KB (FP4) outstanding and consumes data in arrival order.
// Refills past the slice re-read its last super-step (same cache lines), which keeps
// every load unconditional.  EXACT: every wave's slice holds SMAX super-steps or none
// (one uniform branch); otherwise each step is guarded by a uniform branch.
// E8M0 scales (block 32) for the whole slice are loaded once, before the weights: byte
// q of scale dword t is the scale of lane group q in super-step t; with SG4 (K a
// multiple of 512) they come as dwordx4 groups.  The scale is handed to the conversion
// as the f32 bit pattern e << 23: v_cvt_scalef32_* use the exponent field with E8M0
// meaning (0 is 2^-127, 255 is NaN), so every E8M0 byte is exact.
// Activations live in LDS for the whole kernel when M x (K + 8) bf16 fit (XV > 0: XV
// straight-line 16-byte loads per thread, then a loop).  Otherwise (XV = 0) each lane's
// 64 activation bytes of a super-step ride in the ring beside its weights: they are loaded
// with the super-step's codes, D steps ahead, so that waiting for them (the vector memory
// counter retires in order) never drains the weight loads behind them.  Lanes whose B
// column c >= M read activation row 0: those D columns are never stored and MFMA columns
// do not mix, so they need no zeroing.  The NK partial tiles of a weight tile are summed
// through LDS.
// K slices (gridDim.y > 1): workgroup row blockIdx.y takes K elements [blockIdx.y K, + K) of
// rows whose packed bytes are row_bytes apart (the scale rows nblk blocks apart, the
// activation rows ldx elements apart) and writes its partial product to y + blockIdx.y
// part_stride; one slice (gridDim.y = 1) is the whole product.
template <int FMT, int NT, int NK, int RING, int SMAX, bool EXACT, int XV, int SC>
__global__ void __launch_bounds__(NT * NK * 64) gemv_stream(const uint8_t* __restrict__ w, int64_t N, int64_t K,
                                                          const uint8_t* __restrict__ scales, int64_t nblk,
                                                          const __bf16* __restrict__ x, int M, int64_t ldx,
                                                          void* __restrict__ y, int ydt, int64_t ldy, int swiglu,
                                                          int rpw, int64_t row_bytes, int64_t part_stride) {
  static_assert(SMAX % 4 == 0, "scale groups");
  constexpr int D = RING < SMAX ? RING : SMAX;  // ring depth
  constexpr bool SCALED = SC != kScaleNone, SG4 = SC == kScaleGroup4, XLDS = XV > 0;
  using T = MfmaGemvTraits<FMT>;
  constexpr int NW = NT * NK;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  float* partial = (float*)smem;                                   // [NW][64][4] when NK > 1
  __bf16* xs = (__bf16*)(smem + (NK > 1 ? NW * 64 * 4 * 4 : 0));   // [M][K + 8] when XLDS
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: keeps K control flow scalar
  const int ti = wave % NT, ki = wave / NT;
  const int r = lane & 15, q = lane >> 4;
  const int64_t wg0 = (int64_t)blockIdx.x * rpw;
  const int64_t wg_end = wg0 + rpw < N ? wg0 + rpw : N;  // rows of this workgroup: [wg0, wg_end)
  const int64_t n0 = wg0 + 16 * ti;
  const int64_t row = n0 + r < wg_end ? n0 + r : wg_end - 1;  // clamped rows are computed but not stored
  if (gridDim.y > 1) {  // this workgroup's K slice (uniform offsets)
    w += (int64_t)blockIdx.y * (K * format_info(FMT).bits / 8);
    scales += (int64_t)blockIdx.y * (K / 32);
    x += (int64_t)blockIdx.y * K;
    y = (char*)y + (int64_t)blockIdx.y * part_stride * dtype_size(ydt);
  }
  const unsigned* srow = (const unsigned*)(scales + row * nblk);  // dereferenced only when SCALED
  const int S = (int)(K / 128);
  const int per = SG4 ? ((S + NK - 1) / NK + 3) / 4 * 4 : (S + NK - 1) / NK;  // <= SMAX (host)
  const int t_begin = ki * per < S ? ki * per : S;
  const int t_end = t_begin + per < S ? t_begin + per : S;
  const int nsteps = t_end - t_begin;  // uniform; EXACT: SMAX or 0
  const int t_last = nsteps > 0 ? t_end - 1 : 0;
  // Weights are addressed as a uniform base plus a 32-bit per-lane offset (the host keeps
  // the packed matrix under 4 GiB), so a refill costs no 64-bit vector arithmetic.
  const unsigned woff = (unsigned)(row * row_bytes) + (unsigned)(q * T::kLaneBytes);
  auto wptr = [&](int t) __attribute__((always_inline)) { return w + (int64_t)t * T::kStepBytes + woff; };
  const int c = lane & 15;
  const int xr = c < M ? c : 0;  // activation row feeding B column c
  const int64_t xstride = K + 8;

  // Activation loads go first so that the LDS copy waits only for them.  Element
  // e = tid * 8 + i * XSTEP sits at (row m_i, column k_i): one division gives (m_0, k_0)
  // and each pass adds XSTEP = xa * K + xb with one carry.  Threads past the end read row
  // M - 1 (loads stay unconditional: a conditional load would be waited for at once) and
  // store nothing.
  constexpr int XN = XV > 0 ? XV : 1;
  constexpr int XSTEP = NW * 64 * 8;
  const unsigned xtotal = (unsigned)M * (unsigned)K;  // < 2^30 (checked on the host)
  const unsigned uk = (unsigned)K;
  unsigned xm[XN], xk[XN];
  u32x4 xv[XN];
  if constexpr (XLDS) {
    const unsigned xa = XSTEP / uk, xb = XSTEP - xa * uk;
    const unsigned e0 = threadIdx.x * 8u;
    unsigned m = e0 / uk, kk = e0 - m * uk;
#pragma unroll
    for (int i = 0; i < XV; ++i) {
      xm[i] = m;
      xk[i] = kk;
      kk += xb;
      const bool carry = kk >= uk;
      kk = carry ? kk - uk : kk;
      m += xa + (carry ? 1u : 0u);
    }
#pragma unroll
    for (int i = 0; i < XV; ++i) {
      const unsigned mm = xm[i] < (unsigned)M ? xm[i] : (unsigned)M - 1u;
      xv[i] = *(const u32x4*)(x + (mm * (unsigned)ldx + xk[i]));  // 32-bit offset (host: M * ldx < 2^30)
    }
  }
  // Scales of the whole slice, then the first D weight slots.
  unsigned sc[SMAX];
  if constexpr (SCALED) {
#pragma unroll
    for (int g = 0; g < SMAX / 4; ++g) {
      if constexpr (SG4) {
        const int tg = t_begin + 4 * g < t_end - 4 ? t_begin + 4 * g : (t_end >= 4 ? t_end - 4 : 0);
        const u32x4a v = *(const u32x4a*)(srow + tg);
        sc[4 * g] = v[0]; sc[4 * g + 1] = v[1]; sc[4 * g + 2] = v[2]; sc[4 * g + 3] = v[3];
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = t_begin + 4 * g + i < t_last ? t_begin + 4 * g + i : t_last;
          sc[4 * g + i] = srow[t];
        }
      }
    }
  }
  const __bf16* xg = x + (int64_t)xr * ldx + (int64_t)t_begin * 128 + q * 32;
  unsigned buf[D][6];
  bf16x8 xq[XLDS ? 1 : D][4];  // XV = 0: the ring's activations
  auto load_x = [&](int t, int slot) __attribute__((always_inline)) {
    if constexpr (!XLDS) {
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) xq[slot][s4] = *(const bf16x8*)(xg + (int64_t)(t - t_begin) * 128 + 8 * s4);
    }
  };
#pragma unroll
  for (int j = 0; j < D; ++j) {
    const int t = t_begin + j < t_last ? t_begin + j : t_last;
    load_codes<FMT>(wptr(t), buf[j]);
    load_x(t, j);
  }
  if constexpr (XLDS) {
#pragma unroll
    for (int i = 0; i < XV; ++i)
      if (xm[i] < (unsigned)M) *(u32x4*)(xs + xm[i] * xstride + xk[i]) = xv[i];
    for (unsigned e = threadIdx.x * 8u + (unsigned)XV * XSTEP; e < xtotal; e += XSTEP) {
      const unsigned m = e / uk, kk = e - m * uk;
      *(u32x4*)(xs + m * xstride + kk) = *(const u32x4*)(x + (m * (unsigned)ldx + kk));
    }
    __syncthreads();
  }
  const __bf16* xl = xs + (int64_t)xr * xstride + (int64_t)t_begin * 128 + q * 32;
  f32x4 acc[4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
  auto step = [&](int j) __attribute__((always_inline)) {
    const unsigned sdw = SCALED ? sc[j] : 0x7F7F7F7Fu;  // 2^0 in every byte when unscaled
    bf16x8 a[4];
    dequant32<FMT>(buf[j % D], bits_f32(((sdw >> (8 * q)) & 0xFFu) << 23), a);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int kk = j * 128 + 8 * s;
      const bf16x8 b = XLDS ? *(const bf16x8*)(xl + kk) : xq[XLDS ? 0 : j % D][s];
      acc[s] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[s], b, acc[s], 0, 0, 0);
    }
  };
  auto refill = [&](int j) __attribute__((always_inline)) {
    if (j + D < SMAX) {  // compile-time: refill slot j % D with step j + D
      const int t = t_begin + j + D < t_last ? t_begin + j + D : t_last;
      load_codes<FMT>(wptr(t), buf[j % D]);
      load_x(t, j % D);
    }
  };
  if constexpr (EXACT) {
    if (nsteps > 0) {
#pragma unroll
      for (int j = 0; j < SMAX; ++j) {
        step(j);
        refill(j);
        __builtin_amdgcn_sched_barrier(0);  // keep each refill right after its slot's MFMAs
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < SMAX; ++j) {
      if (j < nsteps) step(j);
      refill(j);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  f32x4 sum;
#pragma unroll
  for (int i = 0; i < 4; ++i) sum[i] = (acc[0][i] + acc[1][i]) + (acc[2][i] + acc[3][i]);
  if constexpr (NK > 1) {
#pragma unroll
    for (int i = 0; i < 4; ++i) partial[(wave * 64 + lane) * 4 + i] = sum[i];
    __syncthreads();
    if (ki != 0) return;
#pragma unroll
    for (int kk = 1; kk < NK; ++kk)
#pragma unroll
      for (int i = 0; i < 4; ++i) sum[i] += partial[((kk * NT + ti) * 64 + lane) * 4 + i];
  }
  // Lane (c, q) holds Y[c][n0 + 4q .. n0 + 4q + 3]: one 8- or 16-byte store when whole.
  // swiglu: rows 2 i and 2 i + 1 are the gate and up rows of output column i, so the lane
  // holds two whole pairs and writes silu(gate) * up to columns (n0 + 4q) / 2 + {0, 1}.
  if (swiglu) {
    if (c < M) {
      const int64_t nb = n0 + 4 * q;
#pragma unroll
      for (int i = 0; i < 2; ++i)
        if (nb + 2 * i + 1 < wg_end) {
          const float g = sum[2 * i], u = sum[2 * i + 1];
          store_out(y, ydt, (int64_t)c * ldy + nb / 2 + i, g / (1.0f + expf(-g)) * u);
        }
    }
    return;
  }
  if (c < M) {
    const int64_t nb = n0 + 4 * q;
    const int64_t o = (int64_t)c * ldy + nb;
    if (nb + 3 < wg_end && (o & 3) == 0) {
      if (ydt == TGM_F32) {
        *(f32x4*)((float*)y + o) = sum;
      } else {
        unsigned lo, hi;
        if (ydt == TGM_BF16) {
          lo = f32_to_bf16(sum[0]) | ((unsigned)f32_to_bf16(sum[1]) << 16);
          hi = f32_to_bf16(sum[2]) | ((unsigned)f32_to_bf16(sum[3]) << 16);
        } else {
          lo = __builtin_bit_cast(unsigned short, (_Float16)sum[0]) |
               ((unsigned)__builtin_bit_cast(unsigned short, (_Float16)sum[1]) << 16);
          hi = __builtin_bit_cast(unsigned short, (_Float16)sum[2]) |
               ((unsigned)__builtin_bit_cast(unsigned short, (_Float16)sum[3]) << 16);
        }
        *(u32x2*)((uint16_t*)y + o) = u32x2{lo, hi};
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (nb + i < wg_end) store_out(y, ydt, o + i, sum[i]);
    }
  }
}

constexpr int kGemvRing = 8;            // super-steps of weights in flight per wave
constexpr int kGemvRingX = 4;           // the same when the activations ride in the ring
constexpr size_t kMaxLds = 160 * 1024;  // LDS per workgroup on gfx950

// Compute units of the current device (cached per device; 0 if the query fails).
inline int device_cus() {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cached[dev] == 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cached[dev] = v;
  }
  return cached[dev];
}

// Launch shape of the streaming GEMV: eight waves per workgroup, NT 16-row tiles x NK
// slices of K, at most 32 super-steps per wave.  Shapes are tried in an order that
// keeps 1500+ waves in flight for the tile count; a shape whose slices all hold exactly
// SMAX super-steps (or none) runs the unguarded kernel.
struct GemvShape {
  int nt, nk, smax;
  bool exact;
};

// From kGemvWideTiles tiles (28672 rows) up, eight tiles x the whole K per workgroup: every
// workgroup stages X once for 128 rows, one round of 224 workgroups instead of two rounds of
// 512 with 56 rows each (at 8-16 activation rows the staging traffic, each workgroup reading
// all of X from its XCD's L2, is what grows with M).
constexpr int64_t kGemvWideTiles = 1792;

inline GemvShape gemv_shape(int64_t tiles, int64_t S, bool sg4) {
  static const int order_wide[4][2] = {{8, 1}, {4, 2}, {2, 4}, {1, 8}};
  static const int order_big[4][2] = {{4, 2}, {2, 4}, {1, 8}, {1, 8}};
  static const int order_mid[4][2] = {{2, 4}, {1, 8}, {4, 2}, {4, 2}};
  static const int order_small[4][2] = {{1, 8}, {2, 4}, {4, 2}, {4, 2}};
  const int(*order)[2] = tiles >= kGemvWideTiles ? order_wide
                         : tiles >= 768 ? order_big : tiles >= 384 ? order_mid : order_small;
  for (int i = 0; i < 4; ++i) {
    const int nt = order[i][0], nk = order[i][1];
    int64_t per = (S + nk - 1) / nk;
    if (sg4) per = (per + 3) / 4 * 4;
    if (per > 32) continue;
    // exact kernels exist for block-32 E8M0 scales in groups of four
    const bool exact = sg4 && S % per == 0 && (per == 4 || per == 8 || per == 16 || per == 28 || per == 32);
    return GemvShape{nt, nk, exact ? (int)per : 32, exact};
  }
  return GemvShape{0, 0, 0, false};
}

// The launch description of one streaming GEMV: grid.x row groups x grid.y K slices.
struct StreamLaunch {
  unsigned grid, slices;
  int64_t row_bytes, part_stride;
};

template <int FMT, int NT, int NK, int SMAX, bool EXACT, int XV, int SC>
int launch_stream(const StreamLaunch& L, size_t lds, hipStream_t s, const void* w, int64_t n, int64_t k, const void* scales,
                  int64_t nblk, const void* x, int64_t m, int64_t ldx, void* y, int ydt, int64_t ldy, int swiglu, int rpw) {
  // slices of 8 super-steps keep 6 in flight rather than all 8: 0.45-0.9 us less per launch on
  // every shape (the decoder's K-slice down projection: batch-8 decode 0.583 -> 0.573 ms per step)
  constexpr int RING = XV == 0 ? kGemvRingX : SMAX == 8 ? 6 : kGemvRing;
  auto kernel = gemv_stream<FMT, NT, NK, RING, SMAX, EXACT, XV, SC>;
  if (lds > 64 * 1024) {
    static bool raised = false;  // per instantiation
    if (!raised) {
      hipError_t err = hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxLds);
      if (err != hipSuccess) {
        set_error("tgm_gemv: cannot raise the LDS limit: %s", hipGetErrorString(err));
        return (int)err;
      }
      raised = true;
    }
  }
  hipLaunchKernelGGL(kernel, dim3(L.grid, L.slices), dim3(NT * NK * 64), lds, s, (const uint8_t*)w, n, k,
                     (const uint8_t*)scales, nblk, (const __bf16*)x, (int)m, ldx, y, ydt, ldy, swiglu, rpw, L.row_bytes,
                     L.part_stride);
  return TGM_OK;
}

// xv: 2, 8 or 16 straight-line activation passes, 0 for activations in the load ring.
template <int FMT, int NT, int NK, int SMAX, bool EXACT, int SC>
int launch_stream_xv(int xv, const StreamLaunch& L, size_t lds, hipStream_t s, const void* w, int64_t n, int64_t k,
                     const void* scales, int64_t nblk, const void* x, int64_t m, int64_t ldx, void* y, int ydt,
                     int64_t ldy, int swiglu, int rpw) {
  if (xv == 2) return launch_stream<FMT, NT, NK, SMAX, EXACT, 2, SC>(L, lds, s, w, n, k, scales, nblk, x, m, ldx, y, ydt, ldy, swiglu, rpw);
  if (xv == 8) return launch_stream<FMT, NT, NK, SMAX, EXACT, 8, SC>(L, lds, s, w, n, k, scales, nblk, x, m, ldx, y, ydt, ldy, swiglu, rpw);
  if (xv == 16) return launch_stream<FMT, NT, NK, SMAX, EXACT, 16, SC>(L, lds, s, w, n, k, scales, nblk, x, m, ldx, y, ydt, ldy, swiglu, rpw);
  return launch_stream<FMT, NT, NK, SMAX, EXACT, 0, SC>(L, lds, s, w, n, k, scales, nblk, x, m, ldx, y, ydt, ldy, swiglu, rpw);
}

template <int FMT, int NT, int NK>
int launch_stream_shape(const GemvShape& g, int sc, int xv, const StreamLaunch& L, size_t lds, hipStream_t s, const void* w,
                        int64_t n, int64_t k, const void* scales, int64_t nblk, const void* x, int64_t m, int64_t ldx,
                        void* y, int ydt, int64_t ldy, int swiglu, int rpw) {
  if (g.exact) {  // block-32 E8M0 scales in groups of four, slices of exactly SMAX super-steps
#define TGM_EXACT(SMAX) \
    if (g.smax == SMAX) return launch_stream_xv<FMT, NT, NK, SMAX, true, kScaleGroup4>(xv, L, lds, s, w, n, k, scales, nblk, x, m, ldx, y, ydt, ldy, swiglu, rpw);
    TGM_EXACT(4) TGM_EXACT(8) TGM_EXACT(16) TGM_EXACT(28) TGM_EXACT(32)
#undef TGM_EXACT
    return TGM_E_UNSUPPORTED;
  }
  if (sc == kScaleGroup4) return launch_stream_xv<FMT, NT, NK, 32, false, kScaleGroup4>(xv, L, lds, s, w, n, k, scales, nblk, x, m, ldx, y, ydt, ldy, swiglu, rpw);
  if (sc == kScaleDword) return launch_stream_xv<FMT, NT, NK, 32, false, kScaleDword>(xv, L, lds, s, w, n, k, scales, nblk, x, m, ldx, y, ydt, ldy, swiglu, rpw);
  return launch_stream_xv<FMT, NT, NK, 32, false, kScaleNone>(xv, L, lds, s, w, n, k, scales, nblk, x, m, ldx, y, ydt, ldy, swiglu, rpw);
}

// swiglu: the weight rows interleave gate and up rows; y gets silu(gate) * up (N / 2 columns).
// slices > 1: K is cut into ``slices`` equal parts (k a multiple of 128 slices) and the product
// over part z goes to y + z part_stride (the caller sums the parts); the workgroups then take
// the widest row groups, so that each stages its slice of X for as many rows as it can.
template <int FMT>
int launch_gemv_stream(hipStream_t s, const void* w, int64_t n, int64_t k, const void* scales, const void* x,
                       int64_t m, int64_t ldx, void* y, int ydt, int64_t ldy, int swiglu = 0, int slices = 1,
                       int64_t part_stride = 0) {
  if (slices < 1 || k % (128 * (int64_t)slices) != 0) return TGM_E_UNSUPPORTED;
  const int64_t ks = k / slices;  // K of one slice
  const int64_t tiles = (n + 15) / 16;
  const int sc = scales == nullptr ? kScaleNone : (ks % 512 == 0 ? kScaleGroup4 : kScaleDword);
  const GemvShape g = gemv_shape(slices > 1 && tiles < 768 ? 768 : tiles, ks / 128, sc == kScaleGroup4);
  if (g.nt == 0) return TGM_E_UNSUPPORTED;
  const size_t part = (size_t)g.nt * g.nk * 64 * 16;
  const size_t xbytes = (size_t)m * (size_t)(ks + 8) * 2;
  const bool xlds = part + xbytes <= kMaxLds;
  const int64_t passes = (m * ks + 8 * 64 * 8 - 1) / (8 * 64 * 8);  // XSTEP of an 8-wave workgroup
  // every staging load is issued before the weight ring up to 16 passes: a load in the
  // staging loop after it waits for the whole ring (the vector memory counter retires in order)
  const int xv = !xlds ? 0 : passes <= 2 ? 2 : passes <= 8 ? 8 : 16;
  const size_t lds = part + (xlds ? xbytes : 0);
  const int64_t nblk = k / 32;  // scale row stride (blocks of the whole row)
  // Rows per workgroup: 16 NT, unless the workgroups would leave part of the last round of
  // CUs idle; then the rows are spread evenly over whole rounds (a multiple of 4 rows each).
  // With K slices each slice counts on its share of the CUs.
  int rpw = 16 * g.nt;
  int64_t wgs = (n + rpw - 1) / rpw;
  const int cus = device_cus() / slices;
  if (cus > 0 && wgs % cus != 0) {
    const int64_t rounds = (wgs + cus - 1) / cus;
    const int64_t even = ((n + rounds * cus - 1) / (rounds * cus) + 3) / 4 * 4;
    if (even > 16 * (g.nt - 1) && even < rpw) {  // every tile of the shape keeps rows
      rpw = (int)even;
      wgs = (n + rpw - 1) / rpw;
    }
  }
  const StreamLaunch L{(unsigned)wgs, (unsigned)slices, k * format_info(FMT).bits / 8, part_stride};
  if (g.nt == 8) return launch_stream_shape<FMT, 8, 1>(g, sc, xv, L, lds, s, w, n, ks, scales, nblk, x, m, ldx, y, ydt, ldy, swiglu, rpw);
  if (g.nt == 4) return launch_stream_shape<FMT, 4, 2>(g, sc, xv, L, lds, s, w, n, ks, scales, nblk, x, m, ldx, y, ydt, ldy, swiglu, rpw);
  if (g.nt == 2) return launch_stream_shape<FMT, 2, 4>(g, sc, xv, L, lds, s, w, n, ks, scales, nblk, x, m, ldx, y, ydt, ldy, swiglu, rpw);
  return launch_stream_shape<FMT, 1, 8>(g, sc, xv, L, lds, s, w, n, ks, scales, nblk, x, m, ldx, y, ydt, ldy, swiglu, rpw);
}

// Instantiated per format in tgm_gemv_stream.hip.
int launch_gemv_stream_fp4(hipStream_t s, const void* w, int64_t n, int64_t k, const void* scales, const void* x,
                           int64_t m, int64_t ldx, void* y, int ydt, int64_t ldy, int swiglu = 0, int slices = 1,
                           int64_t part_stride = 0);
int launch_gemv_stream_fp6(hipStream_t s, const void* w, int64_t n, int64_t k, const void* scales, const void* x,
                           int64_t m, int64_t ldx, void* y, int ydt, int64_t ldy, int swiglu = 0, int slices = 1,
                           int64_t part_stride = 0);
int launch_gemv_stream_bf6(hipStream_t s, const void* w, int64_t n, int64_t k, const void* scales, const void* x,
                           int64_t m, int64_t ldx, void* y, int ydt, int64_t ldy, int swiglu = 0, int slices = 1,
                           int64_t part_stride = 0);

}  // namespace tgm
