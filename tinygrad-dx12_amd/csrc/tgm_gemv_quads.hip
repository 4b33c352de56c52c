// Kernel family 1 for 2 <= M <= 4 activation rows: FP4 E2M1 weights with E8M0 block-32 (or no)
// scales, bf16 activations, K a multiple of 2048 up to 8192 ("row-quad" GEMV).
//
// Replaces, like the other GEMVs, the reference's matvec / N <= 16 matmul over decoded weights
// (alexandreteles/tinygrad-dx12 src/tinygrad_dx12/renderer/linalg.py:127-166,
// codegen/linalg.py:244-245).
//
// One v_mfma_f32_16x16x32_bf16 multiplies 16 A rows by 16 B columns over four lane groups
// g = lane >> 4 of 8 K elements each.  Lane l (j = l & 15, quad q = j >> 2, rr = j & 3) feeds
//   A: weight row rr of the wave's current row-quad, chunk c = 4 g + q of the instruction's 256
//      bytes of that row (32 codes, one MX block; sub-step s takes codes 8 s .. 8 s + 7);
//   B: activation row m = rr, the same chunk and sub-step.
// A rows 4q .. 4q+3 and B columns 4q .. 4q+3 therefore see the same K positions (chunks 4 g + q,
// g = 0..3), and D's 4x4 diagonal block q holds the partial dot products of the 4 weight rows
// with the 4 activation rows over those chunks; the 12 other blocks pair different positions and
// are ignored.  So one MFMA per 8 codes of a lane serves every activation row, and each wave
// streams its rows in address order with all of its loads issued up front, as the M = 1 kernel
// does: lanes with the same rr cover 256 contiguous bytes of their row per instruction.
//
// Dequantisation is exact (code * 2^(e-127) in bf16 via v_cvt_scalef32_pk_bf16_fp4), every
// bf16 x bf16 product is exact in fp32, and sums are fp32: only the summation order differs
// from the reference's fp32 GEMV over decoded weights.
//
// A workgroup holds 4 waves, one K slice of K / 4 each, over the same 4 RQ rows, so a wave loads
// only its slice of the activations (4 KB per 512 codes of slice) and the slices meet in LDS.
#include "tgm_gemv_stream.h"  // device_cus

namespace tgm {
namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 qbf16x8;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 qbf16x2;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float qf32x4;
typedef unsigned qu32x4 __attribute__((ext_vector_type(4)));

constexpr int kQuadSlices = 4;  // waves per workgroup, one K slice each

// RQ row-quads per workgroup; IPS 512-code instructions per row and slice (K = 2048 IPS);
// D load instructions in flight per wave (a ring when D < RQ IPS).
template <int RQ, int IPS, int D, bool SCALED>
__global__ void __launch_bounds__(256) gemv_quads_fp4(const uint8_t* __restrict__ w, int64_t N,
                                                    const uint8_t* __restrict__ scales,
                                                    const __bf16* __restrict__ x, int M, int64_t ldx,
                                                    void* __restrict__ y, int ydt, int64_t ldy) {
  constexpr int NI = RQ * IPS;              // load instructions per wave
  constexpr int K = kQuadSlices * IPS * 512;
  constexpr int KB = K / 32;                // E8M0 bytes per row
  const int lane = threadIdx.x & 63;
  const int z = threadIdx.x >> 6;           // K slice of this wave
  const int j = lane & 15, g = lane >> 4, q = j >> 2, rr = j & 3;
  const int c = 4 * g + q;                  // 16-byte chunk of the instruction's 256 bytes per row
  const int64_t r0 = (int64_t)blockIdx.x * (4 * RQ);
  const int slice = z * (IPS * 512);        // first code of the slice
  auto row_of = [&](int p) __attribute__((always_inline)) {
    const int64_t r = r0 + 4 * p + rr;
    return r < N ? r : N - 1;               // rows past N re-read the last row and are not stored
  };
  // Activations first: waiting for them then does not wait for the weights (the vector memory
  // counter retires in order).  B columns with m >= M read row 0 and are not stored.
  const int m = rr < M ? rr : 0;
  const __bf16* xp = x + (int64_t)m * ldx + slice + 32 * c;
  qbf16x8 xb[IPS][4];
#pragma unroll
  for (int t = 0; t < IPS; ++t)
#pragma unroll
    for (int s = 0; s < 4; ++s) xb[t][s] = *(const qbf16x8*)(xp + 512 * t + 8 * s);
  __builtin_amdgcn_sched_barrier(0);  // keep the load groups in this order, ahead of the arithmetic
  // Instruction i = t RQ + p: slice instruction t of row-quad p.
  unsigned sb[NI];
  if constexpr (SCALED) {
#pragma unroll
    for (int i = 0; i < NI; ++i)
      sb[i] = __builtin_nontemporal_load(scales + row_of(i % RQ) * KB + slice / 32 + 16 * (i / RQ) + c);
  }
  __builtin_amdgcn_sched_barrier(0);
  qu32x4 codes[D];
  auto load = [&](int i) __attribute__((always_inline)) {
    codes[i % D] = __builtin_nontemporal_load(
        (const qu32x4*)(w + row_of(i % RQ) * (K / 2) + slice / 2 + 256 * (i / RQ) + 16 * c));
  };
#pragma unroll
  for (int i = 0; i < D; ++i) load(i);
  __builtin_amdgcn_sched_barrier(0);
  qf32x4 acc[RQ];
#pragma unroll
  for (int p = 0; p < RQ; ++p) acc[p] = qf32x4{0.f, 0.f, 0.f, 0.f};
  // instructions in load order, one accumulator chain per row-quad
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int t = i / RQ, p = i % RQ;
    const float sc = bits_f32((SCALED ? sb[i] : 127u) << 23);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const unsigned cw = codes[i % D][s];
      const qbf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(cw, sc, 0);
      const qbf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(cw, sc, 1);
      const qbf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(cw, sc, 2);
      const qbf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(cw, sc, 3);
      const qbf16x8 a = {p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
      acc[p] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, xb[t][s], acc[p], 0, 0, 0);
    }
    if (i + D < NI) load(i + D);  // compile-time condition: refill the slot just consumed
    __builtin_amdgcn_sched_barrier(0);
  }
  // D layout: lane l holds D[4 (l >> 4) + v][l & 15], v = 0..3.  The diagonal blocks are in the
  // lanes with l >> 4 == q, i.e. g == q: D[4q + v][4q + rr] = rows 4p + v, activation row rr.
  __shared__ float red[kQuadSlices][RQ][4][16];  // [slice][row-quad][q][4 v + m]
  if (g == q) {
#pragma unroll
    for (int p = 0; p < RQ; ++p)
#pragma unroll
      for (int v = 0; v < 4; ++v) red[z][p][q][4 * v + rr] = acc[p][v];
  }
  __syncthreads();
  const int tid = threadIdx.x;
  if (tid < 16 * RQ) {
    const int p = tid >> 4, vm = tid & 15, v = vm >> 2, mm = vm & 3;
    float sum = 0.f;
#pragma unroll
    for (int zz = 0; zz < kQuadSlices; ++zz)
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) sum += red[zz][p][qq][vm];
    const int64_t row = r0 + 4 * p + v;
    if (mm < M && row < N) store_from_f32(y, ydt, (int64_t)mm * ldy + row, sum);
  }
}

template <int RQ, int IPS, int D>
void launch_quads(hipStream_t s, const void* w, int64_t n, const void* scales, const void* x, int64_t m,
                  int64_t ldx, void* y, int ydt, int64_t ldy) {
  const unsigned grid = (unsigned)((n + 4 * RQ - 1) / (4 * RQ));
  if (scales)
    hipLaunchKernelGGL((gemv_quads_fp4<RQ, IPS, D, true>), dim3(grid), dim3(256), 0, s, (const uint8_t*)w, n,
                       (const uint8_t*)scales, (const __bf16*)x, (int)m, ldx, y, ydt, ldy);
  else
    hipLaunchKernelGGL((gemv_quads_fp4<RQ, IPS, D, false>), dim3(grid), dim3(256), 0, s, (const uint8_t*)w, n,
                       (const uint8_t*)scales, (const __bf16*)x, (int)m, ldx, y, ydt, ldy);
}

}  // namespace

template <int IPS>
void launch_quads_rows(int rq, hipStream_t s, const void* w, int64_t n, const void* scales, const void* x, int64_t m,
                       int64_t ldx, void* y, int ydt, int64_t ldy) {
  constexpr int D = 12;  // loads in flight per wave (measured: 8-12 best, 16 and all-in-flight slower)
  if (rq == 14) launch_quads<14, IPS, (14 * IPS < D ? 14 * IPS : D)>(s, w, n, scales, x, m, ldx, y, ydt, ldy);
  else if (rq == 7) launch_quads<7, IPS, (7 * IPS < D ? 7 * IPS : D)>(s, w, n, scales, x, m, ldx, y, ydt, ldy);
  else if (rq == 4) launch_quads<4, IPS, (4 * IPS < D ? 4 * IPS : D)>(s, w, n, scales, x, m, ldx, y, ydt, ldy);
  else launch_quads<2, IPS, 2 * IPS>(s, w, n, scales, x, m, ldx, y, ydt, ldy);
}

// The caller has checked the operands as for the streaming GEMV (FP4 weights 16-byte aligned,
// E8M0 block-32 or no scales, bf16 x 16-byte aligned with ldx % 8 == 0, 32-bit offsets); this
// covers 2 <= M <= 4 and K in {2048, 4096, 6144, 8192}.  Rows per workgroup: the most (56, 28,
// 16 or 8) that still gives every CU a workgroup.  Each wave loads M x its K slice of
// activations for 4 RQ weight rows, so fewer rows per workgroup cost activation traffic (28
// rows: 9.3 against 8.3 us at 14336 x 4096, M = 4).
int launch_gemv_quads_fp4(hipStream_t s, const void* w, int64_t n, int64_t k, const void* scales, const void* x,
                          int64_t m, int64_t ldx, void* y, int ydt, int64_t ldy) {
  if (m < 2 || m > 4 || k % 2048 != 0 || k > 8192 || n < 1) return TGM_E_UNSUPPORTED;
  const int64_t cus = device_cus() > 0 ? device_cus() : 256;
  int rq = 2;
  for (const int cand : {14, 7, 4})
    if ((n + 4 * cand - 1) / (4 * cand) >= cus) {
      rq = cand;
      break;
    }
  switch (k / 2048) {
    case 1: launch_quads_rows<1>(rq, s, w, n, scales, x, m, ldx, y, ydt, ldy); break;
    case 2: launch_quads_rows<2>(rq, s, w, n, scales, x, m, ldx, y, ydt, ldy); break;
    case 3: launch_quads_rows<3>(rq, s, w, n, scales, x, m, ldx, y, ydt, ldy); break;
    default: launch_quads_rows<4>(rq, s, w, n, scales, x, m, ldx, y, ydt, ldy); break;
  }
  return TGM_OK;
}

}  // namespace tgm
