// The streaming MX GEMV (tgm_gemv_stream.h) instantiated for the three MX weight formats:
// FP4 E2M1, FP6 E2M3 and FP6 E3M2.  tgm_gemv.hip picks one of these launchers by format.
#include "tgm_gemv_stream.h"

namespace tgm {

int launch_gemv_stream_fp4(hipStream_t s, const void* w, int64_t n, int64_t k, const void* scales, const void* x,
                           int64_t m, int64_t ldx, void* y, int ydt, int64_t ldy, int swiglu, int slices,
                           int64_t part_stride) {
  return launch_gemv_stream<TGM_FMT_FP4_E2M1>(s, w, n, k, scales, x, m, ldx, y, ydt, ldy, swiglu, slices, part_stride);
}

int launch_gemv_stream_fp6(hipStream_t s, const void* w, int64_t n, int64_t k, const void* scales, const void* x,
                           int64_t m, int64_t ldx, void* y, int ydt, int64_t ldy, int swiglu, int slices,
                           int64_t part_stride) {
  return launch_gemv_stream<TGM_FMT_FP6_E2M3>(s, w, n, k, scales, x, m, ldx, y, ydt, ldy, swiglu, slices, part_stride);
}

int launch_gemv_stream_bf6(hipStream_t s, const void* w, int64_t n, int64_t k, const void* scales, const void* x,
                           int64_t m, int64_t ldx, void* y, int ydt, int64_t ldy, int swiglu, int slices,
                           int64_t part_stride) {
  return launch_gemv_stream<TGM_FMT_FP6_E3M2>(s, w, n, k, scales, x, m, ldx, y, ydt, ldy, swiglu, slices, part_stride);
}

}  // namespace tgm
