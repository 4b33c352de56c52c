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

// Transpose 4 x 4 dwords across the four 16-lane rows of a wave: on return register r of
// lane row g holds what register g of lane row r held.  A lane that loaded 16 bytes (block
// g = its row, dwords 0..3) then holds dword g of blocks 0..3, one per MFMA.
__device__ __forceinline__ void transpose4(unsigned& r0, unsigned& r1, unsigned& r2, unsigned& r3) {
  swap32(r0, r2);  // rows 2,3 of r0 <-> rows 0,1 of r2
  swap32(r1, r3);
  swap16(r0, r1);  // odd rows of r0 <-> even rows of r1
  swap16(r2, r3);
}

// A workgroup holds NT x NK waves: wave (ti, ki) owns weight tile blockIdx.x * NT + ti (16
// rows) and the ki-th of NK contiguous slices of its 128-element super-steps (at most
// SMAX).  Each super-step lane (c, q) loads 16 bytes of row c -- block q of the four -- and
// the row's scales of the super-step's blocks (4 / G groups, one vector load); a lane-row
// transpose hands each MFMA u the dword q of block u.  D super-steps are in flight;
// refills past the slice re-read its last super-step, so every load is unconditional.  The
// activations are copied to LDS once ([M][K + 8] fp16) and each step's operands are read
// one step ahead.  G = blocks per scale group (1, 2 or 4).
template <int NT, int NK, int SMAX, int G, int SDT, int XP>
__global__ void __launch_bounds__(NT * NK * 64) gemv_int4(const uint8_t* __restrict__ w, int64_t N, int64_t K,
                                                        const uint8_t* __restrict__ scales, int64_t ngroups,
                                                        unsigned flip, float bias, const _Float16* __restrict__ x,
                                                        int M, int64_t ldx, void* __restrict__ y, int ydt, int64_t ldy) {
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
  const int64_t n0 = ((int64_t)blockIdx.x * NT + ti) * 16;
  const int64_t row = n0 + c < N ? n0 + c : N - 1;  // clamped: rows >= N are computed, not stored
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
  if (n0 + c < N) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = 4 * q + v;
      if (m < M) store_from_f32(y, ydt, (int64_t)m * ldy + n0 + c, acc[v]);
    }
  }
}

template <int NT, int NK, int G, int SDT>
int launch_int4_shape(unsigned grid, hipStream_t s, const void* w, int64_t n, int64_t k, const void* scales,
                      int64_t ngroups, bool sgn, const void* x, int64_t m, int64_t ldx, void* y, int ydt, int64_t ldy,
                      int per) {
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
                       sgn ? 1032.0f : 1024.0f, (const _Float16*)x, (int)m, ldx, y, ydt, ldy);                      \
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
  // Split K until about 2048 waves are in flight (or a slice is 2 super-steps): 8 waves per
  // workgroup as NT tiles x NK slices.
  int nk = 1;
  while (nk < 8 && tiles * nk < 2048 && (S + 2 * nk - 1) / (2 * nk) >= 2) nk *= 2;
  const int per = (int)((S + nk - 1) / nk);
  if (per > 16) return TGM_E_UNSUPPORTED;
  const int nt = 8 / nk;
  const unsigned grid = (unsigned)((tiles + nt - 1) / nt);
  switch (nk) {
    case 1: return launch_int4_shape<8, 1, G, SDT>(grid, s, w, n, k, scales, ngroups, sgn, x, m, ldx, y, ydt, ldy, per);
    case 2: return launch_int4_shape<4, 2, G, SDT>(grid, s, w, n, k, scales, ngroups, sgn, x, m, ldx, y, ydt, ldy, per);
    case 4: return launch_int4_shape<2, 4, G, SDT>(grid, s, w, n, k, scales, ngroups, sgn, x, m, ldx, y, ydt, ldy, per);
    default: return launch_int4_shape<1, 8, G, SDT>(grid, s, w, n, k, scales, ngroups, sgn, x, m, ldx, y, ydt, ldy, per);
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
#define TGM_SDT(SDT)                                                                                                 \
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
