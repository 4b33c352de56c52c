// Pieces shared by the MFMA GEMM kernels: vector typedefs, direct global -> LDS loads,
// buffer resources, the XCD-aware tile order and the output store.
#pragma once

#include <math.h>

#include "tgm_common.h"

namespace tgm {

typedef __attribute__((__vector_size__(8 * sizeof(int)))) int i32x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(unsigned)))) unsigned u32x4;
typedef __attribute__((__vector_size__(2 * sizeof(unsigned)))) unsigned u32x2;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;

typedef int i32x4v __attribute__((ext_vector_type(4)));

// Direct global -> LDS loads through a buffer resource (bounds-checked: offsets past the
// resource's size read zeros).  The 16 (or 4) bytes of lane l land at LDS address
// lds_addr + 16 l (4 l).  They are issued as inline assembly so that the compiler does not
// order later LDS reads of the *other* buffer behind them; completion is awaited
// explicitly (s_waitcnt vmcnt(0)) before the barrier that publishes a buffer.  M0 is set
// inside each statement and nothing else in the kernel uses it.
__device__ __forceinline__ void lds_dma16(i32x4v rsrc, unsigned lds_addr, unsigned voff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" : : "s"(lds_addr), "v"(voff), "s"(rsrc) : "memory");
}
__device__ __forceinline__ void lds_dma4(i32x4v rsrc, unsigned lds_addr, unsigned voff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds" : : "s"(lds_addr), "v"(voff), "s"(rsrc) : "memory");
}
__device__ __forceinline__ void wait_lds_dma() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Raw buffer resource (stride 0, num_records = bytes) for a global pointer.
__device__ __forceinline__ i32x4v buffer_rsrc(const void* p, unsigned bytes) {
  const unsigned long long a = (unsigned long long)p;
  return i32x4v{(int)(unsigned)a, (int)((unsigned)(a >> 32) & 0xFFFFu), (int)bytes, 0x00020000};
}

// Tile order: consecutive hardware workgroup ids go to different XCDs, so the id is permuted
// to give each XCD a contiguous range of tiles (when the count divides by 8), walked in
// groups of ``group_m`` row panels so that concurrently running tiles share operand panels
// in that XCD's L2.
__device__ __forceinline__ void tile_of(int pid, int tiles_m, int tiles_n, int group_m, int& tm, int& tn) {
  const int ntiles = tiles_m * tiles_n;
  if (ntiles % 8 == 0) pid = (pid % 8) * (ntiles / 8) + pid / 8;  // contiguous range per XCD
  const int per_group = group_m * tiles_n;
  const int group = pid / per_group;
  const int first_m = group * group_m;
  const int gsize = tiles_m - first_m < group_m ? tiles_m - first_m : group_m;
  const int in_group = pid - group * per_group;
  tm = first_m + in_group % gsize;
  tn = in_group / gsize;
}

__device__ __forceinline__ void store_c(void* c, int cdt, int64_t i, float v) {
  if (cdt == TGM_BF16) ((uint16_t*)c)[i] = f32_to_bf16(v);
  else if (cdt == TGM_F16) ((_Float16*)c)[i] = (_Float16)v;
  else ((float*)c)[i] = v;
}

// Store one 32 x 32 fp32 accumulator tile in the 32x32 MFMA D layout (lane l holds column
// l % 32, rows 8 (v / 4) + 4 (l / 32) + v % 4) to C rows r0 .. r0 + 31, columns c0 .. c0 + 31.
// The tile goes through the wave's own LDS block ``ep`` (32 rows padded to 36 floats) so
// that lane l then holds row l / 2, columns 16 (l % 2) .. + 16, rounded once from fp32 and
// written as 16-byte row segments; rows past M and columns past N are not written.
// Lane l gets row l / 2, columns 16 (l % 2) .. + 16 of a 32 x 32 accumulator tile.
__device__ __forceinline__ void tile32_row_values(const f32x16& t, float* ep, int lane, float (&vals)[16]) {
  const int half = lane >> 5, er = lane >> 1, ec = (lane & 1) * 16;
#pragma unroll
  for (int v = 0; v < 16; ++v) ep[(8 * (v >> 2) + 4 * half + (v & 3)) * 36 + (lane & 31)] = t[v];
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const f32x4 f = *(const f32x4*)(ep + er * 36 + ec + 4 * q);
    vals[4 * q] = f[0]; vals[4 * q + 1] = f[1]; vals[4 * q + 2] = f[2]; vals[4 * q + 3] = f[3];
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ void store_tile32(const f32x16& t, float* ep, int lane, int r0, int c0, int M, int N,
                                             void* c, int cdt, int64_t ldc) {
  const int er = lane >> 1, ec = (lane & 1) * 16;
  float vals[16];
  tile32_row_values(t, ep, lane, vals);
  const int row = r0 + er, col = c0 + ec;
  if (row >= M) return;
  const int64_t o = (int64_t)row * ldc + col;
  if (col + 15 < N && (o & 7) == 0 && cdt != TGM_F32) {
    unsigned pk[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      if (cdt == TGM_BF16)
        pk[q] = bf16x2_bits(vals[2 * q], vals[2 * q + 1]);
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

// SwiGLU epilogue of a product whose columns interleave gate (even) and up (odd) rows: column
// pair (2 i, 2 i + 1) of a row becomes output column i, silu(gate) * up = gate / (1 +
// exp(-gate)) * up in fp32, rounded once.  N is the product's (even) column count and ldc
// counts output elements; a lane's 16 columns are 8 whole pairs.
__device__ __forceinline__ void store_tile32_swiglu(const f32x16& t, float* ep, int lane, int r0, int c0, int M,
                                                    int N, void* c, int cdt, int64_t ldc) {
  const int er = lane >> 1, ec = (lane & 1) * 16;
  float vals[16];
  tile32_row_values(t, ep, lane, vals);
  const int row = r0 + er, col = c0 + ec;
  if (row >= M) return;
  float y[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const float g = vals[2 * q], u = vals[2 * q + 1];
    y[q] = g / (1.0f + expf(-g)) * u;
  }
  const int64_t o = (int64_t)row * ldc + col / 2;
  if (col + 15 < N && (o & 7) == 0 && cdt != TGM_F32) {
    unsigned pk[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (cdt == TGM_BF16)
        pk[q] = bf16x2_bits(y[2 * q], y[2 * q + 1]);
      else
        pk[q] = __builtin_bit_cast(unsigned short, (_Float16)y[2 * q]) |
                ((unsigned)__builtin_bit_cast(unsigned short, (_Float16)y[2 * q + 1]) << 16);
    }
    *(u32x4*)((uint16_t*)c + o) = u32x4{pk[0], pk[1], pk[2], pk[3]};
  } else {
#pragma unroll
    for (int q = 0; q < 8; ++q)
      if (col + 2 * q + 1 < N) store_c(c, cdt, o + q, y[q]);
  }
}

// Scaled-MFMA GEMM over an FP6 / FP4 operand pair (tgm_gemm_f8f6f4.hip): operand type codes
// ta / tb (f8f6f4_code_of_format), row strides in bytes, scales E8M0 per 32 K-elements or null.
// Returns a TGM_* status (TGM_E_UNSUPPORTED with the reason set, E3M2 x E3M2 included).
int f8f6f4_code_of_format(int fmt);
int launch_f8f6f4(hipStream_t s, int ta, const void* a, int64_t lda, const void* sa, int64_t m, int tb,
                  const void* b, int64_t ldb, const void* sb, int64_t n, int64_t k, void* c, int cdt, int64_t ldc,
                  const char* who);

}  // namespace tgm
