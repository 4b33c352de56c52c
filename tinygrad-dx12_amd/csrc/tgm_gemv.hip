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
// Five kernels:
//  * gemv_rows_fp4 / gemv_rows_int4 -- M = 1 with K a multiple of 2048: FP4 weights with
//    E8M0 (or no) scales x bf16 activations, or INT4/UINT4 weights with fp16/bf16/f32 group
//    scales (32, 64, 128) x fp16 activations; each wave streams 8 whole rows in address
//    order and reduces on the VALU (tgm_gemv_rows.hip).
//  * gemv_int4   -- INT4/UINT4 weights with fp16/bf16/f32/E8M0 group scales (groups of 32,
//    64 or 128), fp16 activations: one f16 MFMA per 32-element block, scale applied to the
//    block's exact partial sum (tgm_gemv_int4.hip).
//  * gemv_quads_fp4 -- 2 <= M <= 4, FP4 weights with E8M0 (or no) scales, bf16 activations,
//    K = 2048 .. 8192 in steps of 2048: four weight rows and the activation rows share K
//    positions in one bf16 MFMA, whose 4x4 diagonal blocks are the dot products
//    (tgm_gemv_quads.hip).
//  * gemv_stream -- FP4/FP6 weights with E8M0 (or no) scales, bf16 activations.  Each
//    dequantised weight code*2^(e-127) is exact in bf16, every bf16*bf16 product is
//    exact in fp32, so v_mfma_f32_16x16x32_bf16 with fp32 accumulation computes the
//    reference's products exactly; only the summation order differs.
//  * gemv_valu  -- every other combination: fp32 dequant (code*scale rounded in fp32,
//    dx12.py:105) and fp32 FMA, one wave per output row.
#include "tgm_gemv_stream.h"

namespace tgm {
// 2 <= M <= 4 FP4 GEMV over row-quads (tgm_gemv_quads.hip).
int launch_gemv_quads_fp4(hipStream_t s, const void* w, int64_t n, int64_t k, const void* scales, const void* x,
                          int64_t m, int64_t ldx, void* y, int ydt, int64_t ldy);
// M = 1 FP4 GEMV streamed row-contiguously (tgm_gemv_rows.hip).
int launch_gemv_rows(hipStream_t s, const void* w, int fmt, int64_t n, int64_t k, const void* scales, int sdt,
                     int64_t bs, const void* x, int xdt, int64_t m, void* y, int ydt, bool swiglu = false);
int launch_gemv_rows_int4(hipStream_t s, const void* w, int fmt, int64_t n, int64_t k, const void* scales, int sdt,
                          int64_t bs, const void* x, int xdt, int64_t m, void* y, int ydt);
// INT4/UINT4 weights x fp16 activations on f16 MFMA (tgm_gemv_int4.hip).
int launch_gemv_int4(hipStream_t s, const void* w, int fmt, int64_t n, int64_t k, const void* scales, int sdt,
                     int64_t bs, const void* x, int xdt, int64_t m, int64_t ldx, void* y, int ydt, int64_t ldy);

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

}  // namespace tgm

using namespace tgm;

static bool mfma_gemv_ok(const void* w, int fmt, int64_t n, int64_t k, const void* scales, int sdt, int64_t bs, const void* x,
                         int xdt, int64_t m, int64_t ldx, int ydt) {
  if (fmt != TGM_FMT_FP4_E2M1 && fmt != TGM_FMT_FP6_E2M3 && fmt != TGM_FMT_FP6_E3M2) return false;
  if (xdt != TGM_BF16 || k % 128 != 0 || ldx % 8 != 0) return false;
  if (scales && (sdt != TGM_E8M0 || bs != 32 || (uintptr_t)scales % 4)) return false;
  if (k >= (1ll << 26) || m * ldx >= (1ll << 30)) return false;  // 32-bit activation indexing
  if (n * (k * format_info(fmt).bits / 8) >= (1ll << 32)) return false;  // 32-bit weight offsets
  if (ydt != TGM_BF16 && ydt != TGM_F16 && ydt != TGM_F32) return false;
  const uintptr_t align = fmt == TGM_FMT_FP4_E2M1 ? 16 : 8;
  if ((uintptr_t)w % align || (uintptr_t)x % 16) return false;
  return true;
}

extern "C" int tgm_gemv_swiglu(const void* w, int fmt, int64_t n, int64_t k, const void* scales, int scale_dtype,
                               int64_t block_size, const void* x, int x_dtype, int64_t m, int64_t ldx, void* y,
                               int y_dtype, int64_t ldy, void* stream) {
  clear_error();
  TGM_CHECK_ARG(valid_format(fmt), "unknown packed format %d", fmt);
  TGM_CHECK_ARG(n >= 0 && n % 2 == 0 && k >= 0 && block_size >= 1, "n must be even (gate and up rows interleaved)");
  TGM_CHECK_ARG(m >= 0 && m <= 16, "M must be <= 16");
  TGM_CHECK_ARG(m <= 1 || ldx >= k, "ldx smaller than K");
  TGM_CHECK_ARG(m <= 1 || ldy >= n / 2, "ldy smaller than N / 2");
  TGM_CHECK_ARG(y_dtype == TGM_BF16 || y_dtype == TGM_F16 || y_dtype == TGM_F32, "output must be bf16, f16 or f32");
  if (n == 0 || m == 0) return TGM_OK;
  if (k == 0 || n * (k / 2) >= (1ll << 40)) TGM_UNSUPPORTED("tgm_gemv_swiglu: no kernel for this size");
  const hipStream_t s = (hipStream_t)stream;
  if (m == 1) {
    const int st = launch_gemv_rows(s, w, fmt, n, k, scales, scale_dtype, block_size, x, x_dtype, 1, y, y_dtype, true);
    if (st == TGM_E_UNSUPPORTED)
      TGM_UNSUPPORTED("tgm_gemv_swiglu: one row needs FP4 weights with E8M0/32 scales, bf16 x, K a multiple of 2048 "
                      "up to 16384");
    return st == TGM_OK ? launch_status("tgm_gemv_swiglu") : st;
  }
  if (!mfma_gemv_ok(w, fmt, n, k, scales, scale_dtype, block_size, x, x_dtype, m, ldx, y_dtype))
    TGM_UNSUPPORTED("tgm_gemv_swiglu: 2-16 rows need FP4/FP6 weights with E8M0/32 (or no) scales, bf16 x, K %% 128 == 0");
  int st;
  switch (fmt) {
    case TGM_FMT_FP4_E2M1: st = launch_gemv_stream_fp4(s, w, n, k, scales, x, m, ldx, y, y_dtype, ldy, 1); break;
    case TGM_FMT_FP6_E2M3: st = launch_gemv_stream_fp6(s, w, n, k, scales, x, m, ldx, y, y_dtype, ldy, 1); break;
    default: st = launch_gemv_stream_bf6(s, w, n, k, scales, x, m, ldx, y, y_dtype, ldy, 1); break;
  }
  if (st == TGM_E_UNSUPPORTED) TGM_UNSUPPORTED("tgm_gemv_swiglu: no streaming shape for K = %lld", (long long)k);
  return st == TGM_OK ? launch_status("tgm_gemv_swiglu") : st;
}

extern "C" int tgm_dec_gemv_parts(const void* w, int fmt, int64_t n, int64_t k, const void* scales, int scale_dtype,
                                  int64_t block_size, const void* x, int x_dtype, int64_t m, int64_t ldx, float* parts,
                                  int64_t ldp, int64_t slices, void* stream) {
  clear_error();
  TGM_CHECK_ARG(valid_format(fmt), "unknown packed format %d", fmt);
  TGM_CHECK_ARG(w && x && parts, "null operand");
  TGM_CHECK_ARG(n >= 0 && k >= 0 && block_size >= 1 && m >= 1 && m <= 16, "invalid gemv sizes (1 <= M <= 16)");
  TGM_CHECK_ARG(slices >= 1 && slices <= 64 && k % (128 * slices) == 0, "K must be a multiple of 128 x slices (1 .. 64)");
  TGM_CHECK_ARG(ldx >= k && ldp >= n, "ldx smaller than K or ldp smaller than N");
  if (n == 0) return TGM_OK;
  // (a slice is a multiple of 128 elements, so its scale bytes start dword-aligned)
  if (!mfma_gemv_ok(w, fmt, n, k, scales, scale_dtype, block_size, x, x_dtype, m, ldx, TGM_F32) || (uintptr_t)parts % 4)
    TGM_UNSUPPORTED("tgm_dec_gemv_parts: FP4/FP6 weights with E8M0/32 (or no) scales, bf16 x, K %% 128 == 0");
  const hipStream_t s = (hipStream_t)stream;
  const int64_t stride = m * ldp;  // floats per part
  int st;
  switch (fmt) {
    case TGM_FMT_FP4_E2M1: st = launch_gemv_stream_fp4(s, w, n, k, scales, x, m, ldx, parts, TGM_F32, ldp, 0, (int)slices, stride); break;
    case TGM_FMT_FP6_E2M3: st = launch_gemv_stream_fp6(s, w, n, k, scales, x, m, ldx, parts, TGM_F32, ldp, 0, (int)slices, stride); break;
    default: st = launch_gemv_stream_bf6(s, w, n, k, scales, x, m, ldx, parts, TGM_F32, ldp, 0, (int)slices, stride); break;
  }
  if (st == TGM_E_UNSUPPORTED) TGM_UNSUPPORTED("tgm_dec_gemv_parts: no streaming shape for K / slices = %lld", (long long)(k / slices));
  return st == TGM_OK ? launch_status("tgm_dec_gemv_parts") : st;
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
  if (m == 1 && n * (k / 2) < (1ll << 40)) {
    int st = launch_gemv_rows(s, w, fmt, n, k, scales, scale_dtype, block_size, x, x_dtype, m, y, y_dtype);
    if (st == TGM_E_UNSUPPORTED)
      st = launch_gemv_rows_int4(s, w, fmt, n, k, scales, scale_dtype, block_size, x, x_dtype, m, y, y_dtype);
    if (st == TGM_OK) return launch_status("tgm_gemv(rows)");
    if (st != TGM_E_UNSUPPORTED) return st;
  }
  if (fmt == TGM_FMT_INT4 || fmt == TGM_FMT_UINT4) {
    const int st = launch_gemv_int4(s, w, fmt, n, k, scales, scale_dtype, block_size, x, x_dtype, m, ldx, y, y_dtype, ldy);
    if (st == TGM_OK) return launch_status("tgm_gemv(int4 mfma)");
    if (st != TGM_E_UNSUPPORTED) return st;
  }
  if (mfma_gemv_ok(w, fmt, n, k, scales, scale_dtype, block_size, x, x_dtype, m, ldx, y_dtype)) {
    if (fmt == TGM_FMT_FP4_E2M1) {
      const int sq = launch_gemv_quads_fp4(s, w, n, k, scales, x, m, ldx, y, y_dtype, ldy);
      if (sq == TGM_OK) return launch_status("tgm_gemv(quads)");
    }
    int st;
    switch (fmt) {
      case TGM_FMT_FP4_E2M1: st = launch_gemv_stream_fp4(s, w, n, k, scales, x, m, ldx, y, y_dtype, ldy); break;
      case TGM_FMT_FP6_E2M3: st = launch_gemv_stream_fp6(s, w, n, k, scales, x, m, ldx, y, y_dtype, ldy); break;
      default: st = launch_gemv_stream_bf6(s, w, n, k, scales, x, m, ldx, y, y_dtype, ldy); break;
    }
    if (st == TGM_OK) return launch_status("tgm_gemv(mfma)");
    if (st != TGM_E_UNSUPPORTED) return st;
    clear_error();  // no streaming shape for this K: the VALU kernel below covers it
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
