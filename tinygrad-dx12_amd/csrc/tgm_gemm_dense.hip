// Kernel family 2, ordinary operands: bf16 x bf16 or f16 x f16 GEMM on 32x32x16 MFMA, and FP8 x
// FP8 (E4M3 / E5M2) decoded to bf16 in registers on the same MFMA (tgm_gemm_fp8).
//
// The reference lowers an ordinary scheduled matrix product to its collective LinAlg GEMM
// (alexandreteles/tinygrad-dx12 src/tinygrad_dx12/codegen/matmul.py:156-246, source from
// renderer/linalg.py:38-124).  This is that product on gfx950:
//
//   C[m, n] = sum_k A[m, k] * B[n, k]      A [M, K] (row stride lda), B [N, K] (row stride ldb)
//
// i.e. A @ B^T with both operands K-contiguous (batched over blockIdx.y with per-operand
// strides; consecutive batches may share B); a row-major B [K, N] is first transposed by
// tgm_transpose16 (the caller's staging copy, as the reference stages operands it cannot
// bind directly, matmul.py:218-226).  Products of two bf16 or two f16 values are exact in
// fp32; accumulation is fp32 and the output is rounded once.
//
// Workgroup: 128 (M) x 256 (N) output tile, eight waves in 2 x 4 (64 x 64 each, 2 x 2 MFMA
// tiles).  K advances 64 elements per step: the A panel (128 rows x 128 B) and B panel (256 rows
// x 128 B) go straight from global memory into a double-buffered LDS stage (buffer_load ... lds,
// zero-filled past M and N), 16-byte columns XOR-swizzled by (row / 2) % 8 so that the 32 rows a
// fragment read touches fall in distinct banks.  MFMA j of a step takes K [16 j + 8 h, + 8) for
// lane half h.  Loads of step s + 2 run while step s + 1 computes.
#include <type_traits>

#include "tgm_mfma_common.h"

namespace tgm {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 dn_bf16x8;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 dn_f16x8;

constexpr int kDM = 128, kDN = 256, kDK = 64;        // tile and K step
constexpr int kDRow = kDK * 2;                        // bytes per panel row and step
constexpr int kDStage = (kDM + kDN) * kDRow;          // 48 KB
constexpr int kDGroupM = 8;

// FP8 operands (E4M3 / E5M2) decoded to bf16 in registers: every FP8 value is exact in bf16, so
// the bf16 MFMA multiplies exactly the FP8 values.  (The gfx950 FP8 MFMA sums its 64-element
// products at reduced precision, measured ~2e-4 of sum |products|; the bf16 MFMA keeps fp32.)
template <bool E5M2>
__device__ __forceinline__ dn_bf16x8 fp8x8_to_bf16(u32x2 q) {
  typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 b2;
  b2 p[4];
  if constexpr (E5M2) {
    p[0] = __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(q[0], 1.0f, false);
    p[1] = __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(q[0], 1.0f, true);
    p[2] = __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(q[1], 1.0f, false);
    p[3] = __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(q[1], 1.0f, true);
  } else {
    p[0] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q[0], 1.0f, false);
    p[1] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q[0], 1.0f, true);
    p[2] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q[1], 1.0f, false);
    p[3] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q[1], 1.0f, true);
  }
  return dn_bf16x8{p[0][0], p[0][1], p[1][0], p[1][1], p[2][0], p[2][1], p[3][0], p[3][1]};
}

// Batched: blockIdx.y = z selects A + z * sa, B + (z / b_group) * sb and
// C + (z / c_group) * scg + (z % c_group) * sc (elements).  TA / TB: operand dtypes (TGM_BF16 /
// TGM_F16 on both sides, or TGM_FP8E4M3 / TGM_FP8E5M2 on each side).  A step is 128 bytes of
// each row: 64 16-bit or 128 FP8 elements.  alpha_a / alpha_b: optional fp32 device factors on
// the sums before the output rounding.
template <int TA, int TB>
__global__ void __launch_bounds__(512) gemm_dense(const uint8_t* __restrict__ a, unsigned lda_bytes,
                                                  const uint8_t* __restrict__ b, unsigned ldb_bytes, int M, int N,
                                                  int K, void* __restrict__ c, int cdt, int64_t ldc, int64_t sa,
                                                  int64_t sb, int64_t sc, int b_group, int c_group, int64_t scg,
                                                  const float* __restrict__ alpha_a, const float* __restrict__ alpha_b) {
  constexpr bool FP8 = TA == TGM_FP8E4M3 || TA == TGM_FP8E5M2;
  constexpr int ES = FP8 ? 1 : 2;   // bytes per element
  constexpr int KS = kDRow / ES;    // elements per step
  constexpr int FA = 2, FB = 2;
  const int z = blockIdx.y;
  a += z * sa * ES;
  b += (z / b_group) * sb * ES;
  c = (uint8_t*)c + ((int64_t)(z / c_group) * scg + (int64_t)(z % c_group) * sc) * dtype_size(cdt);
  __shared__ __attribute__((aligned(16))) unsigned char lds[2 * kDStage];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  const int tiles_m = (M + kDM - 1) / kDM, tiles_n = (N + kDN - 1) / kDN;
  int tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, kDGroupM, tm, tn);
  const int m0 = tm * kDM, n0 = tn * kDN;
  const int nsteps = K / KS;
  const i32x4v ra = buffer_rsrc(a, (unsigned)(M - 1) * lda_bytes + (unsigned)K * ES);
  const i32x4v rb = buffer_rsrc(b, (unsigned)(N - 1) * ldb_bytes + (unsigned)K * ES);
  const unsigned lds_base = (unsigned)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)lds;
  // Load instruction i fills rows 8 i .. 8 i + 7 of a panel: lane l writes slot l % 8 of row
  // 8 i + l / 8, which holds logical column (l % 8) ^ ((row / 2) % 8).  A: instructions
  // 2 wave, 2 wave + 1; B: 4 wave .. 4 wave + 3.
  unsigned voa[2], vob[4];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int row = 8 * (2 * wave + q) + (lane >> 3);
    voa[q] = (unsigned)(m0 + row) * lda_bytes + (unsigned)((lane & 7) ^ ((row >> 1) & 7)) * 16u;
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int row = 8 * (4 * wave + q) + (lane >> 3);
    vob[q] = (unsigned)(n0 + row) * ldb_bytes + (unsigned)((lane & 7) ^ ((row >> 1) & 7)) * 16u;
  }
  auto dma_step = [&](int s, int buf) __attribute__((always_inline)) {
    const unsigned st = lds_base + (unsigned)(buf * kDStage);
#pragma unroll
    for (int q = 0; q < 2; ++q) lds_dma16(ra, st + (unsigned)(2 * wave + q) * 1024u, voa[q] + (unsigned)s * kDRow);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      lds_dma16(rb, st + (unsigned)(kDM * kDRow) + (unsigned)(4 * wave + q) * 1024u, vob[q] + (unsigned)s * kDRow);
  };
  const int half = lane >> 5;
  const int a_row = wm * 64 + (lane & 31), b_row = wn * 64 + (lane & 31);
  using V = typename std::conditional<TA == TGM_F16, dn_f16x8, dn_bf16x8>::type;  // the MFMA operand type
  // MFMA j of a step takes K [16 j + 8 h, + 8) for lane half h: 16 bytes at logical column
  // 2 j + h (16-bit), or 8 bytes at byte 8 h of column j (FP8, decoded to bf16)
  auto frag = [&](const unsigned char* panel, int row, int j, auto tag) __attribute__((always_inline)) {
    if constexpr (FP8) {
      const u32x2 q = *(const u32x2*)(panel + row * kDRow + ((j ^ ((row >> 1) & 7)) * 16) + 8 * half);
      return fp8x8_to_bf16<decltype(tag)::value == TGM_FP8E5M2>(q);
    } else {
      return *(const V*)(panel + row * kDRow + (((2 * j + half) ^ ((row >> 1) & 7)) * 16));
    }
  };
  f32x16 acc[FA][FB];
#pragma unroll
  for (int i = 0; i < FA; ++i)
#pragma unroll
    for (int j = 0; j < FB; ++j) acc[i][j] = f32x16{};

  const int s1 = nsteps > 1 ? 1 : 0;
  dma_step(0, 0);
  dma_step(s1, 1);
  wait_lds_dma();
  __syncthreads();
  for (int s = 0; s < nsteps; ++s) {
    const int cur = s & 1;
    const int s2 = s + 2 < nsteps ? s + 2 : nsteps - 1;
    const unsigned char* pa = lds + cur * kDStage;
    const unsigned char* pb = pa + kDM * kDRow;
#pragma unroll
    for (int j = 0; j < KS / 16; ++j) {
      V fa[FA], fb[FB];
#pragma unroll
      for (int t = 0; t < FA; ++t) fa[t] = frag(pa, a_row + 32 * t, j, std::integral_constant<int, TA>{});
#pragma unroll
      for (int t = 0; t < FB; ++t) fb[t] = frag(pb, b_row + 32 * t, j, std::integral_constant<int, TB>{});
#pragma unroll
      for (int ta = 0; ta < FA; ++ta)
#pragma unroll
        for (int tb = 0; tb < FB; ++tb) {
          if constexpr (TA == TGM_F16)
            acc[ta][tb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[ta], fb[tb], acc[ta][tb], 0, 0, 0);
          else
            acc[ta][tb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[ta], fb[tb], acc[ta][tb], 0, 0, 0);
        }
    }
    wait_lds_dma();   // this wave's loads of step s + 1
    __syncthreads();  // every wave is done with this buffer; step s + 1 is complete in the other
    dma_step(s2, cur);
  }
  wait_lds_dma();
  __syncthreads();  // the epilogue reuses the LDS
  if (alpha_a || alpha_b) {
    const float alpha = (alpha_a ? *alpha_a : 1.0f) * (alpha_b ? *alpha_b : 1.0f);
#pragma unroll
    for (int i = 0; i < FA; ++i)
#pragma unroll
      for (int j = 0; j < FB; ++j) acc[i][j] *= alpha;
  }
  float* ep = (float*)lds + wave * 32 * 36;
#pragma unroll
  for (int i = 0; i < FA; ++i)
#pragma unroll
    for (int j = 0; j < FB; ++j)
      store_tile32(acc[i][j], ep, lane, m0 + wm * 64 + i * 32, n0 + wn * 64 + j * 32, M, N, c, cdt, ldc);
}

// out[j, i] = in[i, j] through padded 64 x 64 LDS tiles; T = uint16_t (bf16 / f16) or uint8_t (fp8).
template <typename T>
__global__ void __launch_bounds__(256) transpose_t(const T* __restrict__ in, int rows, int cols, int64_t ld_in,
                                                   T* __restrict__ out, int64_t ld_out) {
  __shared__ T t[64][65];
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int i = ty; i < 64; i += 4) {
    const int r = r0 + i, cc = c0 + tx;
    if (r < rows && cc < cols) t[i][tx] = in[(int64_t)r * ld_in + cc];
  }
  __syncthreads();
  for (int i = ty; i < 64; i += 4) {
    const int cc = c0 + i, r = r0 + tx;
    if (cc < cols && r < rows) out[(int64_t)cc * ld_out + r] = t[tx][i];
  }
}

}  // namespace tgm

using namespace tgm;

extern "C" int tgm_gemm_dense_batched(const void* a, int a_dtype, int64_t m, int64_t lda, int64_t stride_a,
                                      const void* b, int b_dtype, int64_t n, int64_t ldb, int64_t stride_b,
                                      int64_t b_group, int64_t k, void* c, int c_dtype, int64_t ldc, int64_t stride_c,
                                      int64_t c_group, int64_t stride_c_group,
                                      int64_t batch, void* stream) {
  clear_error();
  TGM_CHECK_ARG(a && b && c, "null operand");
  TGM_CHECK_ARG(m >= 0 && n >= 0 && k >= 0 && batch >= 0 && b_group >= 1 && c_group >= 1 && b_group < (1ll << 31) &&
                    c_group < (1ll << 31),
                "invalid gemm sizes");
  TGM_CHECK_ARG(m <= 1 || lda >= k, "lda smaller than K");
  TGM_CHECK_ARG(n <= 1 || ldb >= k, "ldb smaller than K");
  TGM_CHECK_ARG(m <= 1 || ldc >= n, "ldc smaller than N");
  TGM_CHECK_ARG(stride_a >= 0 && stride_b >= 0 && stride_c >= 0 && stride_c_group >= 0, "negative batch stride");
  TGM_CHECK_ARG(c_dtype == TGM_BF16 || c_dtype == TGM_F16 || c_dtype == TGM_F32, "output must be bf16, f16 or f32");
  if (m == 0 || n == 0 || batch == 0) return TGM_OK;
  if (a_dtype != b_dtype || (a_dtype != TGM_BF16 && a_dtype != TGM_F16))
    TGM_UNSUPPORTED("tgm_gemm_dense: operands must both be bf16 or both f16");
  if (k == 0 || k % kDK != 0) TGM_UNSUPPORTED("tgm_gemm_dense: K must be a positive multiple of %d", kDK);
  const int64_t lda_eff = m > 1 ? lda : k, ldb_eff = n > 1 ? ldb : k;
  if ((lda_eff * 2) % 16 || (ldb_eff * 2) % 16 || (uintptr_t)a % 16 || (uintptr_t)b % 16 ||
      (batch > 1 && ((stride_a * 2) % 16 || (stride_b * 2) % 16)))
    TGM_UNSUPPORTED("tgm_gemm_dense: operands and their rows must be 16-byte aligned");
  if (m >= (1ll << 31) || n >= (1ll << 31) || (m - 1) * lda_eff * 2 + k * 2 >= (1ll << 32) ||
      (n - 1) * ldb_eff * 2 + k * 2 >= (1ll << 32) || batch > 65535)
    TGM_UNSUPPORTED("tgm_gemm_dense: operands must be under 4 GiB (32-bit offsets), at most 65535 batches");
  const int64_t tiles = ((m + kDM - 1) / kDM) * ((n + kDN - 1) / kDN);
  const hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)tiles, (unsigned)batch);
  if (a_dtype == TGM_BF16)
    hipLaunchKernelGGL((gemm_dense<TGM_BF16, TGM_BF16>), grid, dim3(512), 0, st, (const uint8_t*)a,
                       (unsigned)(lda_eff * 2), (const uint8_t*)b, (unsigned)(ldb_eff * 2), (int)m, (int)n, (int)k, c,
                       c_dtype, ldc, stride_a, stride_b, stride_c, (int)b_group, (int)c_group, stride_c_group,
                       (const float*)nullptr, (const float*)nullptr);
  else
    hipLaunchKernelGGL((gemm_dense<TGM_F16, TGM_F16>), grid, dim3(512), 0, st, (const uint8_t*)a,
                       (unsigned)(lda_eff * 2), (const uint8_t*)b, (unsigned)(ldb_eff * 2), (int)m, (int)n, (int)k, c,
                       c_dtype, ldc, stride_a, stride_b, stride_c, (int)b_group, (int)c_group, stride_c_group,
                       (const float*)nullptr, (const float*)nullptr);
  return launch_status("tgm_gemm_dense");
}

extern "C" int tgm_gemm_fp8(const void* a, int a_dtype, int64_t lda, int64_t m, const void* b, int b_dtype,
                            int64_t ldb, int64_t n, int64_t k, const float* scale_a, const float* scale_b, void* c,
                            int c_dtype, int64_t ldc, void* stream) {
  clear_error();
  TGM_CHECK_ARG(a && b && c, "null operand");
  TGM_CHECK_ARG(m >= 0 && n >= 0 && k >= 0, "invalid gemm sizes");
  TGM_CHECK_ARG(m <= 1 || lda >= k, "lda smaller than K");
  TGM_CHECK_ARG(n <= 1 || ldb >= k, "ldb smaller than K");
  TGM_CHECK_ARG(m <= 1 || ldc >= n, "ldc smaller than N");
  TGM_CHECK_ARG(c_dtype == TGM_BF16 || c_dtype == TGM_F16 || c_dtype == TGM_F32, "output must be bf16, f16 or f32");
  const bool fa = a_dtype == TGM_FP8E4M3 || a_dtype == TGM_FP8E5M2, fb = b_dtype == TGM_FP8E4M3 || b_dtype == TGM_FP8E5M2;
  TGM_CHECK_ARG(fa && fb, "tgm_gemm_fp8 takes FP8 E4M3 / E5M2 operands");
  if (m == 0 || n == 0) return TGM_OK;
  if (k == 0 || k % kDRow != 0) TGM_UNSUPPORTED("tgm_gemm_fp8: K must be a positive multiple of %d", kDRow);
  const int64_t lda_eff = m > 1 ? lda : k, ldb_eff = n > 1 ? ldb : k;
  if (lda_eff % 16 || ldb_eff % 16 || (uintptr_t)a % 16 || (uintptr_t)b % 16)
    TGM_UNSUPPORTED("tgm_gemm_fp8: operands and their rows must be 16-byte aligned");
  if (m >= (1ll << 31) || n >= (1ll << 31) || k >= (1ll << 31) || (m - 1) * lda_eff + k >= (1ll << 32) ||
      (n - 1) * ldb_eff + k >= (1ll << 32))
    TGM_UNSUPPORTED("tgm_gemm_fp8: operands must be under 4 GiB (32-bit offsets)");
  const int64_t tiles = ((m + kDM - 1) / kDM) * ((n + kDN - 1) / kDN);
  const hipStream_t st = (hipStream_t)stream;
#define TGM_FP8_PAIR(A, B)                                                                                       \
  if (a_dtype == A && b_dtype == B) {                                                                            \
    hipLaunchKernelGGL((gemm_dense<A, B>), dim3((unsigned)tiles), dim3(512), 0, st, (const uint8_t*)a,           \
                       (unsigned)lda_eff, (const uint8_t*)b, (unsigned)ldb_eff, (int)m, (int)n, (int)k, c, c_dtype, \
                       ldc, (int64_t)0, (int64_t)0, (int64_t)0, 1, 1, (int64_t)0, scale_a, scale_b);           \
    return launch_status("tgm_gemm_fp8");                                                                        \
  }
  TGM_FP8_PAIR(TGM_FP8E4M3, TGM_FP8E4M3) TGM_FP8_PAIR(TGM_FP8E4M3, TGM_FP8E5M2)
  TGM_FP8_PAIR(TGM_FP8E5M2, TGM_FP8E4M3) TGM_FP8_PAIR(TGM_FP8E5M2, TGM_FP8E5M2)
#undef TGM_FP8_PAIR
  return TGM_E_UNSUPPORTED;
}

extern "C" int tgm_gemm_dense(const void* a, int a_dtype, int64_t m, int64_t lda, const void* b, int b_dtype, int64_t n,
                              int64_t ldb, int64_t k, void* c, int c_dtype, int64_t ldc, void* stream) {
  return tgm_gemm_dense_batched(a, a_dtype, m, lda, 0, b, b_dtype, n, ldb, 0, 1, k, c, c_dtype, ldc, 0, 1, 0, 1, stream);
}

extern "C" int tgm_transpose16(const void* in, int64_t rows, int64_t cols, int64_t ld_in, void* out, int64_t ld_out,
                               void* stream) {
  clear_error();
  TGM_CHECK_ARG(in && out, "null operand");
  TGM_CHECK_ARG(rows >= 0 && cols >= 0 && rows < (1ll << 31) && cols < (1ll << 31), "invalid sizes");
  TGM_CHECK_ARG(rows <= 1 || ld_in >= cols, "ld_in smaller than cols");
  TGM_CHECK_ARG(cols <= 1 || ld_out >= rows, "ld_out smaller than rows");
  if (rows == 0 || cols == 0) return TGM_OK;
  const dim3 grid((unsigned)((cols + 63) / 64), (unsigned)((rows + 63) / 64));
  if (grid.y > 65535) TGM_UNSUPPORTED("tgm_transpose16: too many rows");
  hipLaunchKernelGGL(transpose_t<uint16_t>, grid, dim3(256), 0, (hipStream_t)stream, (const uint16_t*)in, (int)rows,
                     (int)cols, ld_in, (uint16_t*)out, ld_out);
  return launch_status("tgm_transpose16");
}

extern "C" int tgm_transpose8(const void* in, int64_t rows, int64_t cols, int64_t ld_in, void* out, int64_t ld_out,
                              void* stream) {
  clear_error();
  TGM_CHECK_ARG(in && out, "null operand");
  TGM_CHECK_ARG(rows >= 0 && cols >= 0 && rows < (1ll << 31) && cols < (1ll << 31), "invalid sizes");
  TGM_CHECK_ARG(rows <= 1 || ld_in >= cols, "ld_in smaller than cols");
  TGM_CHECK_ARG(cols <= 1 || ld_out >= rows, "ld_out smaller than rows");
  if (rows == 0 || cols == 0) return TGM_OK;
  const dim3 grid((unsigned)((cols + 63) / 64), (unsigned)((rows + 63) / 64));
  if (grid.y > 65535) TGM_UNSUPPORTED("tgm_transpose8: too many rows");
  hipLaunchKernelGGL(transpose_t<uint8_t>, grid, dim3(256), 0, (hipStream_t)stream, (const uint8_t*)in, (int)rows,
                     (int)cols, ld_in, (uint8_t*)out, ld_out);
  return launch_status("tgm_transpose8");
}
