// Kernel family 1: fused unpack + dequant GEMV / skinny GEMM (decode), gfx950.
//
// Replaces the reference's thread-scope LinAlg matvec (alexandreteles/tinygrad-dx12
// src/tinygrad_dx12/renderer/linalg.py:127-166) and the N=1 collective matmul that
// matvec(thread=None) lowers to (codegen/linalg.py:244-245), which in the reference
// runs after a separate decode kernel has written the fp32 weights to memory
// (codegen/decomp/dx12.py:49-106).  Here the packed bytes are the only weight traffic.
//
//   Y[m, n] = sum_k X[m, k] * deq(W)[n, k],   M <= 16
//
// Two kernels:
//  * gemv_mfma  -- FP4/FP6 weights with E8M0 (or no) scales, bf16 activations.  Each
//    dequantised weight code*2^(e-127) is exact in bf16, every bf16*bf16 product is
//    exact in fp32, so v_mfma_f32_16x16x32_bf16 with fp32 accumulation computes the
//    reference's products exactly; only the summation order differs.
//  * gemv_valu  -- every other combination: fp32 dequant (code*scale rounded in fp32,
//    dx12.py:105) and fp32 FMA, one wave per output row.
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

// ------------------------------------------------------------------ VALU GEMV
// One wave per output row n; lanes stride over K.  Exact fp32 dequant per element.
template <int MB>
__global__ void __launch_bounds__(256) gemv_valu(const uint8_t* __restrict__ w, int64_t wbytes, int fmt, int64_t N,
                                                 int64_t K, const void* __restrict__ scales, int sdt, int64_t nblk,
                                                 int64_t bs, const void* __restrict__ x, int xdt, int M, int64_t ldx,
                                                 void* __restrict__ y, int ydt, int64_t ldy) {
  const int lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const FormatInfo f = format_info(fmt);
  float acc[MB];
#pragma unroll
  for (int m = 0; m < MB; ++m) acc[m] = 0.f;
  const int64_t row0 = n * K;
  for (int64_t kk = lane; kk < K; kk += 64) {
    const uint32_t p = payload_at(w, wbytes, row0 + kk, f.bits);
    float v = is_int_format(fmt) ? (float)decode_int(p, fmt) : decode_float(p, f);
    if (scales) v = v * load_f32(scales, sdt, n * nblk + kk / bs);
#pragma unroll
    for (int m = 0; m < MB; ++m)
      if (m < M) acc[m] = __builtin_fmaf(load_f32(x, xdt, (int64_t)m * ldx + kk), v, acc[m]);
  }
#pragma unroll
  for (int m = 0; m < MB; ++m) {
    float v = acc[m];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    if (lane == 0 && m < M) store_from_f32(y, ydt, (int64_t)m * ldy + n, v);
  }
}

// ------------------------------------------------------------------ MFMA GEMV
// Inside a 128-element K super-step, lane l (row r = l & 15 of the tile, lane group q = l >> 4) owns
// the 32 consecutive K elements [32q, 32q+32) of the super-step: one 16-byte load for
// FP4 (24 bytes for FP6) and exactly one E8M0 scale (block 32).  MFMA s (s = 0..3) of
// the super-step consumes elements [32q + 8s, 32q + 8s + 8) of every lane group, so
// the four MFMAs together cover the 128 elements once.  The activation operand uses
// the same element order, so the permutation of K cancels in the dot product.
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

template <int FMT>
__device__ __forceinline__ void load_codes(const uint8_t* p, unsigned out[6]) {
  if constexpr (FMT == TGM_FMT_FP4_E2M1) {
    const u32x4 v = *(const u32x4*)p;
    out[0] = v[0]; out[1] = v[1]; out[2] = v[2]; out[3] = v[3]; out[4] = 0; out[5] = 0;
  } else {
    const u32x2 a = *(const u32x2*)p;
    const u32x2 b = *(const u32x2*)(p + 8);
    const u32x2 c = *(const u32x2*)(p + 16);
    out[0] = a[0]; out[1] = a[1]; out[2] = b[0]; out[3] = b[1]; out[4] = c[0]; out[5] = c[1];
  }
}

// Work decomposition: one workgroup of NW waves per 16 weight rows; the K axis is cut
// into 128-element super-steps and wave w owns a contiguous range of them.  Each wave
// walks its range in chunks of PF super-steps: every weight and scale load of the next
// chunk is issued before the MFMAs of the current chunk, so a wave keeps PF x 16 bytes
// (FP4) per lane in flight.  Activations (M rows) are staged once per workgroup in LDS
// when they fit (XLDS); the NW partial tiles are summed through LDS at the end.
// Loads are unconditional: rows past N and super-steps past the wave's range read a
// clamped (valid) address and their results are discarded, so no load sits behind a
// branch and every load of a chunk is in flight before the first wait.
template <int FMT, int PF>
__device__ __forceinline__ void load_chunk(const uint8_t* wrow, const uint8_t* srow, int sshift, int q, int t0,
                                           int t_last, unsigned codes[PF][6], uint32_t sraw[PF]) {
  using T = MfmaGemvTraits<FMT>;
#pragma unroll
  for (int j = 0; j < PF; ++j) {
    const int t = t0 + j < t_last ? t0 + j : t_last;
    load_codes<FMT>(wrow + (int64_t)t * T::kStepBytes, codes[j]);
  }
  if (srow) {
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const int t = t0 + j < t_last ? t0 + j : t_last;
      sraw[j] = srow[(t * 128 + q * 32) >> sshift];
    }
  } else {
#pragma unroll
    for (int j = 0; j < PF; ++j) sraw[j] = 127u;  // 2^0
  }
}

template <int FMT, int NW, int PF, bool XLDS>
__global__ void __launch_bounds__(NW * 64) gemv_mfma(const uint8_t* __restrict__ w, int64_t N, int64_t K,
                                                     const uint8_t* __restrict__ scales, int64_t nblk, int sshift,
                                                     const __bf16* __restrict__ x, int M, int64_t ldx,
                                                     void* __restrict__ y, int ydt, int64_t ldy) {
  using T = MfmaGemvTraits<FMT>;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  float* partial = (float*)smem;                     // [NW][64][4]
  __bf16* xs = (__bf16*)(smem + NW * 64 * 4 * 4);    // [M + 1][K + 8] when XLDS; row M is zero
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int64_t n0 = (int64_t)blockIdx.x * 16;
  const int64_t row = n0 + r < N ? n0 + r : N - 1;  // clamped: rows >= N are computed but not stored
  const int64_t row_bytes = K * format_info(FMT).bits / 8;
  const uint8_t* wrow = w + row * row_bytes + q * T::kLaneBytes;
  const uint8_t* srow = scales ? scales + row * nblk : nullptr;
  const int S = (int)(K / 128);
  const int per = (S + NW - 1) / NW;
  const int t_begin = wave * per < S ? wave * per : S;
  const int t_end = t_begin + per < S ? t_begin + per : S;
  const int c = lane & 15;  // activation row of this lane in the B operand
  const bool x_ok = c < M;
  const int64_t xstride = K + 8;
  const int t_last = t_end > t_begin ? t_end - 1 : t_begin < S ? t_begin : S - 1;

  unsigned cur[PF][6];
  uint32_t s_cur[PF];
  load_chunk<FMT, PF>(wrow, srow, sshift, q, t_begin, t_last, cur, s_cur);
  const __bf16* xrow = x + (int64_t)(x_ok ? c : 0) * ldx;
  if constexpr (XLDS) {
    const int64_t total = (int64_t)M * K;
    for (int64_t e = (int64_t)threadIdx.x * 8; e < total; e += NW * 64 * 8) {
      const int64_t m = e / K, kk = e - m * K;
      *(u32x4*)(xs + m * xstride + kk) = *(const u32x4*)(x + m * ldx + kk);
    }
    for (int64_t kk = (int64_t)threadIdx.x * 8; kk < K; kk += NW * 64 * 8)
      *(u32x4*)(xs + (int64_t)M * xstride + kk) = u32x4{0, 0, 0, 0};
    __syncthreads();
  }
  const __bf16* xl = xs + (int64_t)(x_ok ? c : M) * xstride;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int t0 = t_begin; t0 < t_end; t0 += PF) {
    unsigned nxt[PF][6];
    uint32_t s_nxt[PF];
    const bool more = t0 + PF < t_end;
    if (more) load_chunk<FMT, PF>(wrow, srow, sshift, q, t0 + PF, t_last, nxt, s_nxt);
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const int t = t0 + j;
      if (t < t_end) {
        bf16x8 a[4];
        dequant32<FMT>(cur[j], e8m0_to_float(s_cur[j]), a);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int64_t kk = (int64_t)t * 128 + q * 32 + 8 * s;
          bf16x8 b;
          if constexpr (XLDS) {
            b = *(const bf16x8*)(xl + kk);
          } else {
            b = *(const bf16x8*)(xrow + kk);
            if (!x_ok) b = bf16x8{};
          }
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[s], b, acc, 0, 0, 0);
        }
      }
    }
    if (more) {
#pragma unroll
      for (int j = 0; j < PF; ++j) {
        s_cur[j] = s_nxt[j];
#pragma unroll
        for (int d = 0; d < 6; ++d) cur[j][d] = nxt[j][d];
      }
    }
  }
  if constexpr (NW == 1) {
    if (c < M) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t n = n0 + 4 * q + i;
        if (n < N) store_out(y, ydt, (int64_t)c * ldy + n, acc[i]);
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) partial[(wave * 64 + lane) * 4 + i] = acc[i];
  __syncthreads();
  if (wave == 0) {
    f32x4 sum = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ww = 0; ww < NW; ++ww)
#pragma unroll
      for (int i = 0; i < 4; ++i) sum[i] += partial[(ww * 64 + lane) * 4 + i];
    if (c < M) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t n = n0 + 4 * q + i;
        if (n < N) store_out(y, ydt, (int64_t)c * ldy + n, sum[i]);
      }
    }
  }
}

}  // namespace tgm

using namespace tgm;

static int gemv_waves() {
  static int cached = 0;
  if (!cached) {
    const char* v = getenv("TGM_GEMV_WAVES");
    const int n = v ? atoi(v) : 4;
    cached = (n == 1 || n == 2 || n == 4 || n == 8) ? n : 4;
  }
  return cached;
}

template <int FMT, int NW, bool XLDS>
static void launch_gemv_variant(unsigned grid, size_t lds, hipStream_t s, const void* w, int64_t n, int64_t k,
                                const void* scales, int64_t nblk, int64_t bs, const void* x, int64_t m, int64_t ldx,
                                void* y, int ydt, int64_t ldy) {
  constexpr int PF = 8;
  const int sshift = __builtin_ctzll((unsigned long long)bs);
  hipLaunchKernelGGL((gemv_mfma<FMT, NW, PF, XLDS>), dim3(grid), dim3(NW * 64), lds, s, (const uint8_t*)w, n, k,
                     (const uint8_t*)scales, nblk, sshift, (const __bf16*)x, (int)m, ldx, y, ydt, ldy);
}

template <int FMT>
static int launch_gemv_mfma(int nw, bool xlds, unsigned grid, size_t lds, hipStream_t s, const void* w, int64_t n,
                            int64_t k, const void* scales, int64_t nblk, int64_t bs, const void* x, int64_t m,
                            int64_t ldx, void* y, int ydt, int64_t ldy) {
#define TGM_GEMV_CASE(NW)                                                                                       \
  if (nw == NW) {                                                                                               \
    if (xlds) launch_gemv_variant<FMT, NW, true>(grid, lds, s, w, n, k, scales, nblk, bs, x, m, ldx, y, ydt, ldy);  \
    else launch_gemv_variant<FMT, NW, false>(grid, lds, s, w, n, k, scales, nblk, bs, x, m, ldx, y, ydt, ldy);      \
    return TGM_OK;                                                                                              \
  }
  TGM_GEMV_CASE(1)
  TGM_GEMV_CASE(2)
  TGM_GEMV_CASE(4)
  TGM_GEMV_CASE(8)
#undef TGM_GEMV_CASE
  return TGM_E_INVALID;
}

static bool mfma_gemv_ok(const void* w, int fmt, int64_t k, const void* scales, int sdt, int64_t bs, const void* x,
                         int xdt, int64_t ldx, int ydt) {
  if (fmt != TGM_FMT_FP4_E2M1 && fmt != TGM_FMT_FP6_E2M3 && fmt != TGM_FMT_FP6_E3M2) return false;
  if (xdt != TGM_BF16 || k % 128 != 0 || ldx % 8 != 0) return false;
  if (scales && (sdt != TGM_E8M0 || bs < 32 || (bs & (bs - 1)) != 0)) return false;
  if (k >= (1ll << 30)) return false;
  if (ydt != TGM_BF16 && ydt != TGM_F16 && ydt != TGM_F32) return false;
  const uintptr_t align = fmt == TGM_FMT_FP4_E2M1 ? 16 : 8;
  if ((uintptr_t)w % align || (uintptr_t)x % 16) return false;
  return true;
}

extern "C" int tgm_gemv(const void* w, int fmt, int64_t n, int64_t k, const void* scales, int scale_dtype,
                        int64_t block_size, const void* x, int x_dtype, int64_t m, int64_t ldx, void* y,
                        int y_dtype, int64_t ldy, void* stream) {
  clear_error();
  TGM_CHECK_ARG(valid_format(fmt), "unknown packed format %d", fmt);
  TGM_CHECK_ARG(n >= 0 && k >= 0 && m >= 0 && m <= 16 && block_size >= 1, "invalid gemv sizes (M must be <= 16)");
  TGM_CHECK_ARG(m <= 1 || ldx >= k, "ldx smaller than K");
  TGM_CHECK_ARG(m <= 1 || ldy >= n, "ldy smaller than N");
  TGM_CHECK_ARG(x_dtype == TGM_BF16 || x_dtype == TGM_F16 || x_dtype == TGM_F32, "gemv activations must be bf16, f16 or f32");
  TGM_CHECK_ARG(y_dtype == TGM_BF16 || y_dtype == TGM_F16 || y_dtype == TGM_F32, "gemv output must be bf16, f16 or f32");
  TGM_CHECK_ARG(!scales || (scale_dtype != TGM_F64 && dtype_size(scale_dtype) > 0), "gemv scales must not be f64");
  if (n == 0 || m == 0) return TGM_OK;
  hipStream_t s = (hipStream_t)stream;
  const int64_t nblk = (k + block_size - 1) / block_size;
  if (k == 0) {
    TGM_UNSUPPORTED("K == 0 has no gemv kernel");
  }
  if (mfma_gemv_ok(w, fmt, k, scales, scale_dtype, block_size, x, x_dtype, ldx, y_dtype)) {
    const unsigned grid = (unsigned)((n + 15) / 16);
    const int64_t xlds_bytes = (m + 1) * (k + 8) * 2;
    const bool xlds = xlds_bytes <= 48 * 1024;
    const int nw = gemv_waves();
    const size_t lds = (size_t)nw * 64 * 4 * 4 + (xlds ? (size_t)xlds_bytes : 0);
    int st = TGM_OK;
    switch (fmt) {
      case TGM_FMT_FP4_E2M1: st = launch_gemv_mfma<TGM_FMT_FP4_E2M1>(nw, xlds, grid, lds, s, w, n, k, scales, nblk, block_size, x, m, ldx, y, y_dtype, ldy); break;
      case TGM_FMT_FP6_E2M3: st = launch_gemv_mfma<TGM_FMT_FP6_E2M3>(nw, xlds, grid, lds, s, w, n, k, scales, nblk, block_size, x, m, ldx, y, y_dtype, ldy); break;
      default: st = launch_gemv_mfma<TGM_FMT_FP6_E3M2>(nw, xlds, grid, lds, s, w, n, k, scales, nblk, block_size, x, m, ldx, y, y_dtype, ldy); break;
    }
    if (st != TGM_OK) return st;
    return launch_status("tgm_gemv(mfma)");
  }
  const int64_t wbytes = (n * k * format_info(fmt).bits + 7) / 8;
  const unsigned grid = (unsigned)((n + 3) / 4);
#define TGM_LAUNCH_VALU(MB)                                                                                         \
  hipLaunchKernelGGL(gemv_valu<MB>, dim3(grid), dim3(256), 0, s, (const uint8_t*)w, wbytes, fmt, n, k, scales,       \
                     scale_dtype, nblk, block_size, x, x_dtype, (int)m, ldx, y, y_dtype, ldy)
  if (m <= 1) TGM_LAUNCH_VALU(1);
  else if (m <= 4) TGM_LAUNCH_VALU(4);
  else TGM_LAUNCH_VALU(16);
#undef TGM_LAUNCH_VALU
  return launch_status("tgm_gemv(valu)");
}
