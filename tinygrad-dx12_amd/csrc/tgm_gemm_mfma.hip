// Kernel family 2 (prefill GEMM) entry points.  Kernels land in later revisions; until
// then the entry points report TGM_E_UNSUPPORTED so callers take the exact-width path.
#include "tgm_common.h"

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
  TGM_UNSUPPORTED("tgm_gemm_mx: no scaled-MFMA kernel for this combination");
}
