// Streaming MX GEMV instantiated for TGM_FMT_FP6_E2M3 weights (one translation unit per format
// so that the instantiations compile in parallel).
#include "tgm_gemv_stream.h"

namespace tgm {

int launch_gemv_stream_fp6(hipStream_t s, const void* w, int64_t n, int64_t k, const void* scales, const void* x,
                           int64_t m, int64_t ldx, void* y, int ydt, int64_t ldy, int swiglu) {
  return launch_gemv_stream<TGM_FMT_FP6_E2M3>(s, w, n, k, scales, x, m, ldx, y, ydt, ldy, swiglu);
}

}  // namespace tgm
