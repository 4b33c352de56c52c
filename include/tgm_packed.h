/*
 * tgm_packed.h -- C ABI of the MI355X (gfx950) packed low-bit matmul library
 * (libtgm_mi355x.so).
 *
 * Every entry point takes plain device pointers, element counts and strides, and an
 * opaque HIP stream (hipStream_t passed as void*; NULL = the legacy default stream).
 * Kernels are enqueued asynchronously on that stream; no entry point synchronises
 * except where stated.  Entry points return TGM_OK (0) on success, a negative TGM_E_*
 * code for argument errors, or a positive hipError_t for runtime failures; the text of
 * the last failure on the calling thread is available from tgm_last_error().
 *
 * The packed storage contract is the reference's: a continuous little-endian bit
 * stream over the flattened logical array (alexandreteles/tinygrad-dx12
 * src/tinygrad_dx12/codegen/decomp/dx12.py:69-77, ARCHITECTURE.md:594-658).  Scales
 * are numeric tensors of shape shape[:-1] + (ceil(K/block),) (dx12.py:44-47); an
 * E8M0 scale tensor is one byte per scale holding 2^(e-127).
 *
 * The reference binds nothing below Python: its packed path is
 * PackedTensor.unpack + linalg.matmul/matvec -> LinAlg HLSL kernels.  The Python
 * package tinygrad_mi355x binds this header with ctypes (runtime/kernels.py); each
 * declaration names the reference interface it replaces.
 */
#ifndef TGM_PACKED_H
#define TGM_PACKED_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TGM_ABI_VERSION 1

/* Packed formats, FORMATS of dx12.py:10. */
enum tgm_format {
  TGM_FMT_INT4 = 0,
  TGM_FMT_UINT4 = 1,
  TGM_FMT_FP4_E2M1 = 2,
  TGM_FMT_FP6_E2M3 = 3,
  TGM_FMT_FP6_E3M2 = 4,
};

/* Element types of ordinary (unpacked) operands, scales and results. */
enum tgm_dtype {
  TGM_BOOL = 0,
  TGM_I8 = 1,
  TGM_U8 = 2,
  TGM_I16 = 3,
  TGM_U16 = 4,
  TGM_I32 = 5,
  TGM_U32 = 6,
  TGM_I64 = 7,
  TGM_U64 = 8,
  TGM_FP8E4M3 = 9, /* OCP E4M3FN */
  TGM_FP8E5M2 = 10,
  TGM_F16 = 11,
  TGM_BF16 = 12,
  TGM_F32 = 13,
  TGM_F64 = 14,
  TGM_E8M0 = 15, /* OCP MX shared scale: 2^(e-127), 0xFF = NaN */
  TGM_NONE = -1,
};

enum tgm_status {
  TGM_OK = 0,
  TGM_E_INVALID = -1,     /* bad argument (maps to ValueError) */
  TGM_E_UNSUPPORTED = -2, /* no kernel for this combination (caller picks another family) */
};

/* ABI version; lets the binding reject a stale library. */
int tgm_abi_version(void);

/* Message of the last failure on this thread ("" if none). */
const char* tgm_last_error(void);

/*
 * The gcnArchName of HIP device ``ordinal`` (e.g. "gfx950:sramecc+:xnack-"), written to out
 * (at most len bytes, NUL-terminated).  Replaces the reference's adapter description query
 * (runtime/support/dx12.py:298-336) for the plugin's renderer target, so the runtime needs no
 * other library to learn the architecture.  Returns a hipError_t on failure.
 */
int tgm_device_arch(int ordinal, char* out, int64_t len);

/*
 * Decode ``count`` packed elements to ``out_dtype`` (replaces PackedTensor.unpack,
 * dx12.py:49-106).  ``k`` is the logical last dimension (scales index
 * [i / k, (i % k) / block]).  ``scales`` may be NULL (scale_dtype ignored).
 * Multiplication happens in f64 when scale_dtype or out_dtype is F64, else f32, then
 * the value is cast to out_dtype (RNE for float narrowing, truncation for integers).
 * Unscaled FP4/FP6 with an exact FP8 out_dtype (FP8_CANDIDATES, dx12.py:11) use the
 * direct re-encode of dx12.py:78-92.
 */
int tgm_unpack(const void* data, int64_t nbytes, int fmt, int64_t count, int64_t k,
               const void* scales, int scale_dtype, int64_t block_size,
               void* out, int out_dtype, void* stream);

/*
 * Kernel family 1 -- fused unpack+dequant GEMV / skinny GEMM for decode
 * (replaces the LinAlg thread-scope matvec thread_source, renderer/linalg.py:127-166,
 * and the N=1 use of linalg_source through linalg.py:244-245).
 *
 *   Y[m, n] = sum_k X[m, k] * deq(W)[n, k]      0 <= m < M <= 16, 0 <= n < N
 *
 * W is packed [N, K] (K contiguous) with optional scales [N, ceil(K/block)].
 * X element (m, k) lives at x + m*ldx + k (elements of x_dtype: BF16, F16 or F32).
 * Y element (m, n) lives at y + m*ldy + n (y_dtype: BF16, F16 or F32).  Accumulation
 * is fp32; the result is rounded once to y_dtype.
 */
int tgm_gemv(const void* w, int fmt, int64_t n, int64_t k,
             const void* scales, int scale_dtype, int64_t block_size,
             const void* x, int x_dtype, int64_t m, int64_t ldx,
             void* y, int y_dtype, int64_t ldy, void* stream);

/*
 * Family 1 with a SwiGLU epilogue (the gate / up projection of a decoder's feed-forward
 * block; no reference counterpart, where the activation would be a separate tinygrad op):
 *
 *   y[m, i] = silu(g) * u,  g = sum_k x[m, k] deq(W)[2 i, k],  u = sum_k x[m, k] deq(W)[2 i + 1, k]
 *
 * W packed [n, k] with gate and up rows interleaved, n even; m <= 16 activation rows x (BF16,
 * row stride ldx); y has n / 2 columns (row stride ldy).  silu(g) = g / (1 + exp(-g)) in
 * fp32, rounded once.  M = 1 runs the FP4 + E8M0/32 row-streaming kernel (K a multiple of
 * 2048, at most 16384); 2 <= M <= 16 the streaming MFMA GEMV (FP4 / FP6, E8M0/32 or no
 * scales, K a multiple of 128); otherwise TGM_E_UNSUPPORTED.
 */
int tgm_gemv_swiglu(const void* w, int fmt, int64_t n, int64_t k, const void* scales, int scale_dtype,
                    int64_t block_size, const void* x, int x_dtype, int64_t m, int64_t ldx, void* y, int y_dtype,
                    int64_t ldy, void* stream);

/*
 * Kernel family 2 -- prefill GEMM with packed weights and 16-bit activations
 * (replaces the collective LinAlg GEMM linalg_source, renderer/linalg.py:38-124,
 * for a packed weight operand; linalg.py:175-218).
 *
 *   C[m, n] = sum_k A[m, k] * deq(W)[n, k]
 *
 * W packed [N, K] with scales [N, ceil(K/block)]; C (c_dtype BF16, F16 or F32) with
 * row stride ldc; A [M, K] with row stride lda.  K must be a multiple of 128.
 *   - FP4 / FP6 weights: A is BF16, scales E8M0 per 32 (or none).  The codes are
 *     dequantised in registers to bf16 (exact) and fed to bf16 MFMA.
 *   - INT4 / UINT4 weights: A is F16, scales F16, BF16 or F32 per 32, 64 or 128 K-elements
 *     (or none).  The codes become exact f16 values, f16 MFMA sums each scale group's
 *     products in fp32 and the group sum is multiplied by its fp32 scale.
 * Accumulation is fp32; the result is rounded once.  Other combinations return
 * TGM_E_UNSUPPORTED.
 */
int tgm_gemm_w(const void* a, int a_dtype, int64_t m, int64_t lda,
               const void* w, int fmt, int64_t n, int64_t k,
               const void* scales, int scale_dtype, int64_t block_size,
               void* c, int c_dtype, int64_t ldc, void* stream);

/*
 * tgm_gemm_w with K split over up to `splits` groups of workgroups, for products with too few
 * output tiles to fill the chip (few rows, or N of a few thousand): each group writes fp32
 * partial products to `workspace` ([splits][M][N]), and a reduction sums them in group
 * order (deterministic) and rounds once to c_dtype.  The effective split count makes every
 * group hold at least one 128-wide K step; with one group, or N % 4 != 0, this is exactly
 * tgm_gemm_w and needs no workspace.  Otherwise workspace (16-byte aligned) must hold
 * tgm_gemm_w_split_workspace(m, n, splits) bytes.  The reference has no split-K (its GEMM is a
 * single D3D12 dispatch, renderer/linalg.py:38-124).
 */
int64_t tgm_gemm_w_split_workspace(int64_t m, int64_t n, int64_t splits);
int tgm_gemm_w_split(const void* a, int a_dtype, int64_t m, int64_t lda, const void* w, int fmt, int64_t n, int64_t k,
                     const void* scales, int scale_dtype, int64_t block_size, void* c, int c_dtype, int64_t ldc,
                     int64_t splits, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * tgm_gemm_w_split without a workspace argument: the same kernels, the same split choice and
 * bit-identical results, with the fp32 partials in a static array of device memory that the
 * library holds on each GPU it runs on (tgm_gemm_w_split_noalloc_capacity() bytes, 32 MiB) from
 * the code object's load until the process ends.  No counterpart in the reference.  It is for
 * callers that cannot allocate device memory: code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc.  It calls no hipMalloc, hipFree or allocating library
 * routine.  A product whose partials exceed the capacity (splits x M x N x 4 bytes) is rejected
 * with TGM_E_INVALID.  All calls on one GPU share its array and each call overwrites it, so
 * calls that overlap in time on one GPU (other streams, other threads) race: the caller orders
 * them.  The first call on each device looks up that device's address of the array
 * (hipGetSymbolAddress); make that first call outside graph capture.  The stream must launch
 * on the calling thread's current device (the null and legacy / per-thread default streams
 * do): a stream of another device is rejected with TGM_E_INVALID before any GPU work.
 */
int64_t tgm_gemm_w_split_noalloc_capacity(void);
int tgm_gemm_w_split_noalloc(const void* a, int a_dtype, int64_t m, int64_t lda, const void* w, int fmt, int64_t n,
                             int64_t k, const void* scales, int scale_dtype, int64_t block_size, void* c, int c_dtype,
                             int64_t ldc, int64_t splits, void* stream);

/*
 * tgm_gemm_w for FP4 weights whose rows interleave the gate (row 2 i) and up (row 2 i + 1)
 * projections of a SwiGLU block, with the activation in the epilogue:
 *
 *   C[m, i] = silu(G[m, 2 i]) * G[m, 2 i + 1],  G = A . deq(W)^T,  silu(g) = g / (1 + exp(-g))
 *
 * in fp32, rounded once to c_dtype; C has N / 2 columns (row stride ldc).  The gate and up
 * products never reach memory.  The reference has no fused activation (a tinygrad caller
 * applies silu to the matmul's output); tgm_gemv_swiglu is the one-token form.
 */
int tgm_gemm_w_swiglu(const void* a, int a_dtype, int64_t m, int64_t lda, const void* w, int fmt, int64_t n, int64_t k,
                      const void* scales, int scale_dtype, int64_t block_size, void* c, int c_dtype, int64_t ldc,
                      void* stream);

/*
 * Kernel family 2 -- FP4/FP6 x FP4/FP6 GEMM on gfx950 scaled MFMA
 * (replaces linalg_source for two packed operands, renderer/linalg.py:38-124; the
 * reference decodes both to their common intermediate first -- FP8 when both are
 * unscaled, fp32 when either is scaled -- dx12.py:115-138).
 *
 *   C[m, n] = sum_k deq(A)[m, k] * deq(B)[n, k]
 *
 * A packed [M, K], B packed [N, K] (FP4 E2M1, FP6 E2M3 or FP6 E3M2), both K contiguous,
 * each with E8M0 scales per 32 K-elements ([M, K/32] / [N, K/32]) or NULL (unscaled:
 * every scale 1).  C (BF16, F16 or F32) row stride ldc; fp32 accumulation.  FP4 x FP4
 * with both scales and K a multiple of 256 runs the 256 x 256-tile FP4 kernel; every
 * other pair needs K a multiple of 128.  INT4 / UINT4 and FP6 E3M2 x E3M2 (whose MFMA
 * sums are not exact on gfx950) give TGM_E_UNSUPPORTED.
 */
int tgm_gemm_mx(const void* a, int a_fmt, const void* a_scales, int64_t m,
                const void* b, int b_fmt, const void* b_scales, int64_t n, int64_t k,
                void* c, int c_dtype, int64_t ldc, void* stream);

/*
 * Kernel family 2 -- ordinary FP8 x FP8 GEMM: both operands decoded to bf16 in registers (every
 * FP8 value is exact in bf16) on the bf16 MFMA of tgm_gemm_dense (the reference's LinAlg
 * lowering takes FP8 operands as they are, renderer/linalg.py:12-13, through the
 * scheduled-matmul rewrite, codegen/matmul.py:51-128).
 *
 *   C[m, n] = (sum_k A[m, k] * B[n, k]) * scale_a * scale_b
 *
 * A [M, K] and B [N, K] of dtype FP8E4M3 or FP8E5M2 (the two may differ), K contiguous, row
 * strides lda / ldb in elements (multiples of 16, rows 16-byte aligned); scale_a / scale_b are
 * optional fp32 device scalars (NULL = 1; torch._scaled_mm's per-tensor scales) applied to the
 * fp32 sum before it is rounded to C (BF16, F16 or F32, row stride ldc).  Products are exact in
 * fp32, accumulation fp32.  K must be a multiple of 128; otherwise TGM_E_UNSUPPORTED.  (The
 * gfx950 FP8 MFMA is not used: it sums at ~2e-4 of sum |products|, measured.)
 */
int tgm_gemm_fp8(const void* a, int a_dtype, int64_t lda, int64_t m, const void* b, int b_dtype, int64_t ldb,
                 int64_t n, int64_t k, const float* scale_a, const float* scale_b, void* c, int c_dtype,
                 int64_t ldc, void* stream);

/*
 * Kernel family 2 -- ordinary bf16 x bf16 or f16 x f16 GEMM on MFMA (the reference's LinAlg
 * lowering of a scheduled ordinary matrix product, codegen/matmul.py:156-246 with
 * renderer/linalg.py:38-124).
 *
 *   C[m, n] = sum_k A[m, k] * B[n, k]
 *
 * A [M, K] (row stride lda) and B [N, K] (row stride ldb) of one dtype, both K-contiguous;
 * C (BF16, F16 or F32) with row stride ldc.  Products are exact in fp32, accumulation fp32.
 * K must be a multiple of 64 and rows 16-byte aligned; otherwise TGM_E_UNSUPPORTED.
 */
int tgm_gemm_dense(const void* a, int a_dtype, int64_t m, int64_t lda, const void* b, int b_dtype, int64_t n,
                   int64_t ldb, int64_t k, void* c, int c_dtype, int64_t ldc, void* stream);

/*
 * The same product for ``batch`` independent matrices (the reference's tinygrad lowering
 * handles one scheduled matrix reduction per kernel; a batch here is one launch): batch z uses
 * A + z * stride_a, B + (z / b_group) * stride_b and
 * C + (z / c_group) * stride_c_group + (z % c_group) * stride_c (element offsets), so b_group
 * consecutive batches can share one B (grouped-query attention's shared keys) and the outputs
 * of c_group consecutive batches can interleave (heads side by side in one token row).
 * c_group = batch with stride_c_group = 0 gives plain C + z * stride_c.  At most 65535 batches.
 */
int tgm_gemm_dense_batched(const void* a, int a_dtype, int64_t m, int64_t lda, int64_t stride_a, const void* b,
                           int b_dtype, int64_t n, int64_t ldb, int64_t stride_b, int64_t b_group, int64_t k, void* c,
                           int c_dtype, int64_t ldc, int64_t stride_c, int64_t c_group, int64_t stride_c_group,
                           int64_t batch, void* stream);

/*
 * out[j, i] = in[i, j] for 16-bit elements: in is [rows, cols] (row stride ld_in), out is
 * [cols, rows] (row stride ld_out).  Stages a row-major [K, N] operand as [N, K] for
 * tgm_gemm_dense (the reference stages operands it cannot bind directly, matmul.py:218-226).
 */
int tgm_transpose16(const void* in, int64_t rows, int64_t cols, int64_t ld_in, void* out, int64_t ld_out,
                    void* stream);

/* The same for 8-bit elements: stages a row-major FP8 [K, N] operand as [N, K] for tgm_gemm_fp8. */
int tgm_transpose8(const void* in, int64_t rows, int64_t cols, int64_t ld_in, void* out, int64_t ld_out,
                   void* stream);

/*
 * Exact-width GEMM for operands the families above do not cover (the reference's
 * fallback lhs.matmul(rhs, dtype=...), linalg.py:169-174 and :219-223, with products
 * formed at accumulator width as the DX12 device does, test_linalg.py:221-230).
 *
 *   C[m, n] = cast_c( sum_k acc(A[m, k]) * acc(B[k, n]) )
 *
 * Element (i, j) of A is at a + i*sa0 + j*sa1 (element strides), same for B and C.
 * acc_dtype is one of F32, F64, I32, U32, I64, U64.
 */
int tgm_gemm_plain(const void* a, int a_dtype, int64_t sa0, int64_t sa1,
                   const void* b, int b_dtype, int64_t sb0, int64_t sb1,
                   void* c, int c_dtype, int64_t sc0, int64_t sc1,
                   int64_t m, int64_t n, int64_t k, int acc_dtype, void* stream);

/*
 * Tensor-level pack with block scales (no reference counterpart: the reference only
 * accepts pre-packed bytes, dx12.py:26-30; its packers are benchmark_dtypes.py:129-152).
 * Quantises x [rows, k] (BF16, F16 or F32) along k to an MX float format with one
 * E8M0 scale per ``block_size`` elements: shared exponent floor(log2(amax)) -
 * emax_elem, elements rounded to nearest even and saturated.  Writes the packed
 * bit stream (rows*k elements) to ``data`` and rows*ceil(k/block) bytes to ``scales``.
 */
int tgm_quantize_mx(const void* x, int x_dtype, int64_t rows, int64_t k, int fmt,
                    int64_t block_size, void* data, void* scales, void* stream);

/*
 * Pack ``count`` payload codes (one per byte, low ``bits`` bits used) into the
 * LSB-first bit stream (pack_payload, benchmark_dtypes.py:129-152).  ``out`` must hold
 * ceil(count*bits/8) bytes; padding bits are zero.
 */
int tgm_pack_codes(const void* codes, int64_t count, int bits, void* out, void* stream);

/*
 * Measurement probes (no reference counterpart; bench.py reports them beside the kernels they
 * bound).  tgm_probe_read reads ``nbytes`` (a multiple of 16) with the decode GEMV's access
 * shape -- contiguous 8 KB per wave, 16-byte non-temporal loads, all in flight -- and discards
 * them: the single-launch read ceiling for that many bytes.  tgm_probe_mfma_fp4 runs ``blocks``
 * workgroups of 8 waves, each wave ``iters`` rounds of 8 FP4 v_mfma_scale_f32_32x32x64_f8f6f4
 * from registers with operand bits changing every round: the FP4 MFMA ceiling with no data
 * movement (2^20 flops per wave and round).  ``sink`` is a 4-byte device scratch word.
 */
int tgm_probe_read(const void* p, int64_t nbytes, void* sink, void* stream);
int tgm_probe_mfma_fp4(int64_t blocks, int64_t iters, void* sink, void* stream);
/* tgm_probe_launch launches an empty kernel of ``groups`` x ``threads`` (threads <= 1024): the
 * fixed cost of one launch of that grid with no work, the floor under any kernel's time. */
int tgm_probe_launch(int64_t groups, int64_t threads, void* sink, void* stream);
/* tgm_probe_bf16_rounding converts the fp32 bit patterns first .. first + count - 1 (both even,
 * first + count <= 2^32) to bf16 with the instruction the bf16 epilogues use, in both halves of a
 * packed pair, and compares each with integer round-to-nearest-even (NaN -> quiet NaN).  ``bad``
 * (2 x uint32, set by the caller to 0 and 0xFFFFFFFF) receives the mismatch count and the
 * smallest mismatching pattern; ``bits`` (nullable, count x uint16) the converted patterns. */
int tgm_probe_bf16_rounding(uint32_t first, int64_t count, void* bits, void* bad, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TGM_PACKED_H */
