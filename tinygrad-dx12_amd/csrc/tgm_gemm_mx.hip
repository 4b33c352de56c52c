// Kernel family 2, block-scaled path: FP4 (E2M1) x FP4 GEMM on gfx950 scaled MFMA.
//
// Replaces the reference's collective LinAlg GEMM (alexandreteles/tinygrad-dx12
// src/tinygrad_dx12/renderer/linalg.py:38-124) for two packed operands.  The reference
// first decodes both operands to the fp32 intermediate (codegen/decomp/dx12.py:115-138,
// 49-106) and multiplies those; here the packed codes and their E8M0 scales feed
// v_mfma_scale_f32_32x32x64_f8f6f4 directly.  FP4 x FP4 products with power-of-two
// scales are exact in fp32, so only the summation order differs from the reference.
//
//   C[m, n] = sum_k deq(A)[m, k] * deq(B)[n, k]
//
// A [M, K] and B [N, K] are stored K-contiguous, two codes per byte (low nibble first),
// with one E8M0 scale byte per 32 K-elements ([M, K/32], [N, K/32]).
//
// MFMA operand layout (32x32x64): lane l supplies row (l % 32) of its operand and the 32
// consecutive K elements [32 * (l / 32), +32) of the 64-element K step -- 16 bytes of
// packed codes, i.e. one MX block, and that block's scale in byte 0 of its scale VGPR.
// D layout: lane l holds column l % 32 and rows 8 * (v / 4) + 4 * (l / 32) + v % 4.
//
// Workgroup: 256 x 256 output tile, four waves in 2 x 2, each wave 128 x 128 = 4 x 4
// MFMA tiles (256 fp32 accumulators per lane).  K advances in steps of 256 elements
// (128 bytes per row and operand): each step's A and B panels (32 KB each) are staged
// from global memory through registers into a double-buffered LDS tile whose rows are
// padded to 144 bytes, so the 32 rows read by one ds_read_b128 fall in distinct banks.
// The next step's global loads are in flight while the current step's MFMAs run.
// Tiles are mapped XCD-aware: consecutive hardware workgroup ids go to different XCDs,
// so the id is permuted to give each XCD a contiguous range of tiles, walked in groups
// of 8 row-panels so that concurrently running tiles share A and B panels in its L2.
#include "tgm_common.h"

namespace tgm {

typedef __attribute__((__vector_size__(8 * sizeof(int)))) int i32x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(unsigned)))) unsigned u32x4;
typedef __attribute__((__vector_size__(2 * sizeof(unsigned)))) unsigned u32x2;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;

constexpr int kBM = 256, kBN = 256;  // output tile
constexpr int kBK = 256;             // K elements per step
constexpr int kRowBytes = kBK / 2;   // FP4 bytes per row and step
constexpr int kLdsRow = kRowBytes + 16;
constexpr int kPanel = kBM * kLdsRow;            // one operand, one buffer (36 KB)
constexpr int kLdsBytes = 2 * 2 * kPanel;        // A and B, double buffered (144 KB)
constexpr int kGroupM = 8;

__device__ __forceinline__ void tile_of(int pid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int ntiles = tiles_m * tiles_n;
  if (ntiles % 8 == 0) pid = (pid % 8) * (ntiles / 8) + pid / 8;  // contiguous range per XCD
  const int per_group = kGroupM * tiles_n;
  const int group = pid / per_group;
  const int first_m = group * kGroupM;
  const int gsize = tiles_m - first_m < kGroupM ? tiles_m - first_m : kGroupM;
  const int in_group = pid - group * per_group;
  tm = first_m + in_group % gsize;
  tn = in_group / gsize;
}

__device__ __forceinline__ void store_c(void* c, int cdt, int64_t i, float v) {
  if (cdt == TGM_BF16) ((uint16_t*)c)[i] = f32_to_bf16(v);
  else if (cdt == TGM_F16) ((_Float16*)c)[i] = (_Float16)v;
  else ((float*)c)[i] = v;
}

__global__ void __launch_bounds__(256) gemm_mx_fp4(const uint8_t* __restrict__ a, const uint8_t* __restrict__ sa,
                                                   const uint8_t* __restrict__ b, const uint8_t* __restrict__ sb,
                                                   int M, int N, int K, void* __restrict__ c, int cdt, int64_t ldc) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int tiles_m = (M + kBM - 1) / kBM, tiles_n = (N + kBN - 1) / kBN;
  int tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * kBM, n0 = tn * kBN;
  const int nsteps = K / kBK;

  // Global -> LDS staging: chunk g = i * 256 + tid of a 256-row x 128-byte panel is row
  // i * 32 + tid / 8, 16-byte column tid % 8 (a wave covers 8 whole 128-byte rows per
  // load).  Offsets are 32-bit (the host keeps each operand under 4 GiB) and recomputed
  // per step, which costs a few VALU next to the step's 64 MFMAs and keeps registers for
  // the accumulators.  Rows past M or N re-read the last row; their results are dropped.
  const int srow = tid >> 3, scol = (tid & 7) * 16;
  const int lds_base = srow * kLdsRow + scol;
  const unsigned kb = (unsigned)(K / 2);
  auto a_off = [&](int i, int s) __attribute__((always_inline)) {
    const int r = m0 + i * 32 + srow;
    return (unsigned)(r < M ? r : M - 1) * kb + (unsigned)(scol + s * kRowBytes);
  };
  auto b_off = [&](int i, int s) __attribute__((always_inline)) {
    const int r = n0 + i * 32 + srow;
    return (unsigned)(r < N ? r : N - 1) * kb + (unsigned)(scol + s * kRowBytes);
  };
  // Scale rows of this lane: A rows wm*128 + t*32 + l%32, B rows wn*128 + t*32 + l%32.
  const unsigned kblk = (unsigned)(K / 32);
  auto sa_off = [&](int t, int s) __attribute__((always_inline)) {
    const int r = m0 + wm * 128 + t * 32 + (lane & 31);
    return (unsigned)(r < M ? r : M - 1) * kblk + (unsigned)(s * 8);
  };
  auto sb_off = [&](int t, int s) __attribute__((always_inline)) {
    const int r = n0 + wn * 128 + t * 32 + (lane & 31);
    return (unsigned)(r < N ? r : N - 1) * kblk + (unsigned)(s * 8);
  };

  u32x4 stage_a[8], stage_b[8];
  u32x2 scl_a[4], scl_b[4], nscl_a[4], nscl_b[4];
  auto load_step = [&](int s) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      stage_a[i] = *(const u32x4*)(a + a_off(i, s));
      stage_b[i] = *(const u32x4*)(b + b_off(i, s));
    }
  };
  auto load_scales = [&](int s) __attribute__((always_inline)) {  // into nscl_*
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      nscl_a[t] = *(const u32x2*)(sa + sa_off(t, s));
      nscl_b[t] = *(const u32x2*)(sb + sb_off(t, s));
    }
  };
  auto store_step = [&](int buf) __attribute__((always_inline)) {
    unsigned char* la = smem + buf * 2 * kPanel + lds_base;
    unsigned char* lb = la + kPanel;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      *(u32x4*)(la + i * 32 * kLdsRow) = stage_a[i];
      *(u32x4*)(lb + i * 32 * kLdsRow) = stage_b[i];
    }
  };

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};

  // Scales live in scl_* for the current step and nscl_* for the next one.
  load_step(0);
  load_scales(0);
  store_step(0);
#pragma unroll
  for (int t = 0; t < 4; ++t) { scl_a[t] = nscl_a[t]; scl_b[t] = nscl_b[t]; }
  load_step(nsteps > 1 ? 1 : 0);
  load_scales(nsteps > 1 ? 1 : 0);
  __syncthreads();

  const int half = lane >> 5;  // K half of the 64-element MFMA step
  const int frag_off_a = (wm * 128 + (lane & 31)) * kLdsRow + half * 16;
  const int frag_off_b = (wn * 128 + (lane & 31)) * kLdsRow + half * 16;
  // Fragments of one 64-element K substep: rows t*32 + l%32 of the wave's A and B panels.
  struct Frags {
    u32x4 a[4], b[4];
  };
  auto read_frags = [&](Frags& f, int buf, int u) __attribute__((always_inline)) {
    const unsigned char* la = smem + buf * 2 * kPanel;
    const unsigned char* lb = la + kPanel;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      f.a[t] = *(const u32x4*)(la + frag_off_a + t * 32 * kLdsRow + u * 32);
      f.b[t] = *(const u32x4*)(lb + frag_off_b + t * 32 * kLdsRow + u * 32);
    }
  };
  auto mfmas = [&](const Frags& f, int u) __attribute__((always_inline)) {
    // scale of block 2u + half of this step: byte (2u + half) % 4 of word (2u + half) / 4
    const int blk = 2 * u + half;
    int xa[4], xb[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      xa[t] = (int)((u < 2 ? scl_a[t][0] : scl_a[t][1]) >> (8 * (blk & 3)));
      xb[t] = (int)((u < 2 ? scl_b[t][0] : scl_b[t][1]) >> (8 * (blk & 3)));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const i32x8 fa = {(int)f.a[i][0], (int)f.a[i][1], (int)f.a[i][2], (int)f.a[i][3], 0, 0, 0, 0};
        const i32x8 fb = {(int)f.b[j][0], (int)f.b[j][1], (int)f.b[j][2], (int)f.b[j][3], 0, 0, 0, 0};
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa, fb, acc[i][j], 4, 4, 0, xa[i], 0, xb[j]);
      }
  };
  // Per step: the fragments of substep u + 1 are read while substep u's MFMAs run; the
  // next step's panels go to the other LDS buffer during substep 1 (that buffer was last
  // read in the previous step, before its barrier) and the step after next is fetched
  // from global memory during substep 2, so its loads overlap two substeps of MFMAs.
  // The body has no branches (past the last step the loads re-read step nsteps - 1 and the
  // stores fill the buffer nobody reads again), so the instruction interleaving asked for
  // by the scheduling barriers holds: one LDS or global instruction between MFMAs.
  Frags f0, f1;
  for (int s = 0; s < nsteps; ++s) {
    const int buf = s & 1;
    const int s2 = s + 2 < nsteps ? s + 2 : nsteps - 1;
    read_frags(f0, buf, 0);
    read_frags(f1, buf, 1);
    mfmas(f0, 0);
    __builtin_amdgcn_sched_barrier(0);
    store_step(buf ^ 1);
    read_frags(f0, buf, 2);
    mfmas(f1, 1);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x200, 2, 0);  // DS write
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
    }
    __builtin_amdgcn_sched_barrier(0);
    load_step(s2);
    read_frags(f1, buf, 3);
    mfmas(f0, 2);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);  // VMEM read
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    mfmas(f1, 3);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < 4; ++t) { scl_a[t] = nscl_a[t]; scl_b[t] = nscl_b[t]; }
    load_scales(s2);
    __syncthreads();
  }

  // Epilogue: each 32 x 32 accumulator tile goes through a per-wave LDS block (rows
  // padded to 36 floats) so that lane l then holds row l / 2, columns 16 * (l % 2) .. +16,
  // rounded once from fp32 and written as 16-byte row segments.
  float* ep = (float*)smem + wave * 32 * 36;
  const int er = lane >> 1, ec = (lane & 1) * 16;
  auto out_tile = [&](const f32x16 t, int i, int j) __attribute__((always_inline)) {
#pragma unroll
    for (int v = 0; v < 16; ++v) ep[(8 * (v >> 2) + 4 * half + (v & 3)) * 36 + (lane & 31)] = t[v];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float vals[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const f32x4 f = *(const f32x4*)(ep + er * 36 + ec + 4 * q);
      vals[4 * q] = f[0]; vals[4 * q + 1] = f[1]; vals[4 * q + 2] = f[2]; vals[4 * q + 3] = f[3];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int row = m0 + wm * 128 + i * 32 + er;
    const int col = n0 + wn * 128 + j * 32 + ec;
    if (row < M) {
      const int64_t o = (int64_t)row * ldc + col;
      if (col + 15 < N && (o & 7) == 0 && cdt != TGM_F32) {
        unsigned pk[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          if (cdt == TGM_BF16)
            pk[q] = f32_to_bf16(vals[2 * q]) | ((unsigned)f32_to_bf16(vals[2 * q + 1]) << 16);
          else
            pk[q] = __builtin_bit_cast(unsigned short, (_Float16)vals[2 * q]) |
                    ((unsigned)__builtin_bit_cast(unsigned short, (_Float16)vals[2 * q + 1]) << 16);
        }
        *(u32x4*)((uint16_t*)c + o) = u32x4{pk[0], pk[1], pk[2], pk[3]};
        *(u32x4*)((uint16_t*)c + o + 8) = u32x4{pk[4], pk[5], pk[6], pk[7]};
      } else if (col + 15 < N && (o & 3) == 0 && cdt == TGM_F32) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *(f32x4*)((float*)c + o + 4 * q) = f32x4{vals[4 * q], vals[4 * q + 1], vals[4 * q + 2], vals[4 * q + 3]};
      } else {
#pragma unroll
        for (int q = 0; q < 16; ++q)
          if (col + q < N) store_c(c, cdt, o + q, vals[q]);
      }
    }
  };
  // literal indices keep the accumulators in registers
  out_tile(acc[0][0], 0, 0); out_tile(acc[0][1], 0, 1); out_tile(acc[0][2], 0, 2); out_tile(acc[0][3], 0, 3);
  out_tile(acc[1][0], 1, 0); out_tile(acc[1][1], 1, 1); out_tile(acc[1][2], 1, 2); out_tile(acc[1][3], 1, 3);
  out_tile(acc[2][0], 2, 0); out_tile(acc[2][1], 2, 1); out_tile(acc[2][2], 2, 2); out_tile(acc[2][3], 2, 3);
  out_tile(acc[3][0], 3, 0); out_tile(acc[3][1], 3, 1); out_tile(acc[3][2], 3, 2); out_tile(acc[3][3], 3, 3);
}

}  // namespace tgm

using namespace tgm;

extern "C" int tgm_gemm_w(const void* a, int a_dtype, int64_t m, int64_t lda, const void* w, int fmt, int64_t n,
                          int64_t k, const void* scales, int scale_dtype, int64_t block_size, void* c, int c_dtype,
                          int64_t ldc, void* stream) {
  clear_error();
  TGM_UNSUPPORTED("tgm_gemm_w: no MFMA kernel for this combination");
}

extern "C" int tgm_gemm_mx(const void* a, int a_fmt, const void* a_scales, int64_t m, const void* b, int b_fmt,
                           const void* b_scales, int64_t n, int64_t k, void* c, int c_dtype, int64_t ldc,
                           void* stream) {
  clear_error();
  TGM_CHECK_ARG(valid_format(a_fmt) && valid_format(b_fmt), "unknown packed format");
  TGM_CHECK_ARG(m >= 0 && n >= 0 && k >= 0, "invalid gemm sizes");
  TGM_CHECK_ARG(a_scales && b_scales, "block-scaled GEMM needs E8M0 scales for both operands");
  TGM_CHECK_ARG(c_dtype == TGM_BF16 || c_dtype == TGM_F16 || c_dtype == TGM_F32, "output must be bf16, f16 or f32");
  TGM_CHECK_ARG(m <= 1 || ldc >= n, "ldc smaller than N");
  if (m == 0 || n == 0) return TGM_OK;
  if (a_fmt != TGM_FMT_FP4_E2M1 || b_fmt != TGM_FMT_FP4_E2M1)
    TGM_UNSUPPORTED("tgm_gemm_mx: only FP4 x FP4 has a scaled-MFMA kernel");
  if (k == 0 || k % kBK != 0) TGM_UNSUPPORTED("tgm_gemm_mx: K must be a positive multiple of %d", kBK);
  if (m >= (1ll << 31) || n >= (1ll << 31) || m * (k / 2) >= (1ll << 32) || n * (k / 2) >= (1ll << 32))
    TGM_UNSUPPORTED("tgm_gemm_mx: operands must be under 4 GiB (32-bit offsets)");
  if ((uintptr_t)a % 16 || (uintptr_t)b % 16 || (uintptr_t)a_scales % 8 || (uintptr_t)b_scales % 8)
    TGM_UNSUPPORTED("tgm_gemm_mx: operands must be 16-byte and scales 8-byte aligned");
  static bool raised = false;
  if (!raised) {
    hipError_t err = hipFuncSetAttribute((const void*)gemm_mx_fp4, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
    if (err != hipSuccess) {
      set_error("tgm_gemm_mx: cannot raise the LDS limit: %s", hipGetErrorString(err));
      return (int)err;
    }
    raised = true;
  }
  const int64_t tiles = ((m + kBM - 1) / kBM) * ((n + kBN - 1) / kBN);
  hipLaunchKernelGGL(gemm_mx_fp4, dim3((unsigned)tiles), dim3(256), kLdsBytes, (hipStream_t)stream, (const uint8_t*)a,
                     (const uint8_t*)a_scales, (const uint8_t*)b, (const uint8_t*)b_scales, (int)m, (int)n, (int)k, c,
                     c_dtype, ldc);
  return launch_status("tgm_gemm_mx");
}
