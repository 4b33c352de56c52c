// Host-side plumbing shared by the C-ABI entry points: error reporting, dtype helpers
// and element load/store used by the generic (non-MFMA) kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "tgm_formats.h"

namespace tgm {

// Thread-local text of the last failure (tgm_last_error).
void set_error(const char* fmt, ...);
void clear_error();

#define TGM_CHECK_ARG(cond, ...)          \
  do {                                    \
    if (!(cond)) {                        \
      ::tgm::set_error(__VA_ARGS__);      \
      return TGM_E_INVALID;               \
    }                                     \
  } while (0)

#define TGM_UNSUPPORTED(...)              \
  do {                                    \
    ::tgm::set_error(__VA_ARGS__);        \
    return TGM_E_UNSUPPORTED;             \
  } while (0)

// Launch status after an asynchronous kernel launch.
int launch_status(const char* what);

// Compute units of the device ``stream`` launches on (the current device for the null and
// legacy / per-thread default streams), looked up once per device; 0 when unknown.
int stream_cu_count(hipStream_t stream);

__host__ __device__ inline int dtype_size(int dt) {
  switch (dt) {
    case TGM_BOOL: case TGM_I8: case TGM_U8: case TGM_FP8E4M3: case TGM_FP8E5M2: case TGM_E8M0: return 1;
    case TGM_I16: case TGM_U16: case TGM_F16: case TGM_BF16: return 2;
    case TGM_I32: case TGM_U32: case TGM_F32: return 4;
    case TGM_I64: case TGM_U64: case TGM_F64: return 8;
    default: return 0;
  }
}

__host__ __device__ inline bool valid_format(int fmt) { return fmt >= TGM_FMT_INT4 && fmt <= TGM_FMT_FP6_E3M2; }

// ------------------------------------------------------------------ element access
// Value of element ``i`` of a ``dt`` array as double (exact for every type but the
// 64-bit integers beyond 2^53, which callers read through load_i64 instead).
__device__ __forceinline__ double load_f64(const void* p, int dt, int64_t i) {
  switch (dt) {
    case TGM_BOOL: return ((const uint8_t*)p)[i] ? 1.0 : 0.0;
    case TGM_I8: return (double)((const int8_t*)p)[i];
    case TGM_U8: return (double)((const uint8_t*)p)[i];
    case TGM_I16: return (double)((const int16_t*)p)[i];
    case TGM_U16: return (double)((const uint16_t*)p)[i];
    case TGM_I32: return (double)((const int32_t*)p)[i];
    case TGM_U32: return (double)((const uint32_t*)p)[i];
    case TGM_I64: return (double)((const int64_t*)p)[i];
    case TGM_U64: return (double)((const uint64_t*)p)[i];
    case TGM_FP8E4M3: return fp8_bits_to_double(((const uint8_t*)p)[i], 3, 7, true);
    case TGM_FP8E5M2: return fp8_bits_to_double(((const uint8_t*)p)[i], 2, 15, false);
    case TGM_F16: return (double)f16_bits_to_f32(((const uint16_t*)p)[i]);
    case TGM_BF16: return (double)bf16_to_f32(((const uint16_t*)p)[i]);
    case TGM_F32: return (double)((const float*)p)[i];
    case TGM_F64: return ((const double*)p)[i];
    case TGM_E8M0: return (double)e8m0_to_float(((const uint8_t*)p)[i]);
    default: return 0.0;
  }
}

__device__ __forceinline__ float load_f32(const void* p, int dt, int64_t i) {
  switch (dt) {
    case TGM_F32: return ((const float*)p)[i];
    case TGM_F16: return f16_bits_to_f32(((const uint16_t*)p)[i]);
    case TGM_BF16: return bf16_to_f32(((const uint16_t*)p)[i]);
    case TGM_E8M0: return e8m0_to_float(((const uint8_t*)p)[i]);
    default: return (float)load_f64(p, dt, i);
  }
}

__device__ __forceinline__ int64_t load_i64(const void* p, int dt, int64_t i) {
  switch (dt) {
    case TGM_I64: return ((const int64_t*)p)[i];
    case TGM_U64: return (int64_t)((const uint64_t*)p)[i];
    case TGM_BOOL: case TGM_I8: case TGM_U8: case TGM_I16: case TGM_U16: case TGM_I32: case TGM_U32:
      return (int64_t)load_f64(p, dt, i);
    default: return (int64_t)load_f64(p, dt, i);
  }
}

// Store a floating value with a single rounding to ``dt``.
__device__ __forceinline__ void store_from_f64(void* p, int dt, int64_t i, double v) {
  switch (dt) {
    case TGM_BOOL: ((uint8_t*)p)[i] = v != 0.0; break;
    case TGM_I8: ((int8_t*)p)[i] = (int8_t)(int64_t)v; break;
    case TGM_U8: ((uint8_t*)p)[i] = (uint8_t)(int64_t)v; break;
    case TGM_I16: ((int16_t*)p)[i] = (int16_t)(int64_t)v; break;
    case TGM_U16: ((uint16_t*)p)[i] = (uint16_t)(int64_t)v; break;
    case TGM_I32: ((int32_t*)p)[i] = (int32_t)(int64_t)v; break;
    case TGM_U32: ((uint32_t*)p)[i] = (uint32_t)(int64_t)v; break;
    case TGM_I64: ((int64_t*)p)[i] = (int64_t)v; break;
    case TGM_U64: ((uint64_t*)p)[i] = v < 0 ? (uint64_t)(int64_t)v : (uint64_t)v; break;
    case TGM_FP8E4M3: ((uint8_t*)p)[i] = to_fp8e4m3(v); break;
    case TGM_FP8E5M2: ((uint8_t*)p)[i] = to_fp8e5m2(v); break;
    case TGM_F16: ((uint16_t*)p)[i] = to_f16_bits(v); break;
    case TGM_BF16: ((uint16_t*)p)[i] = (uint16_t)narrow_rne(v, 8, 7, 127, false); break;
    case TGM_F32: ((float*)p)[i] = (float)v; break;
    case TGM_F64: ((double*)p)[i] = v; break;
    default: break;
  }
}

__device__ __forceinline__ void store_from_f32(void* p, int dt, int64_t i, float v) {
  switch (dt) {
    case TGM_F32: ((float*)p)[i] = v; break;
    case TGM_BF16: ((uint16_t*)p)[i] = f32_to_bf16(v); break;
    case TGM_F16: ((_Float16*)p)[i] = (_Float16)v; break;
    default: store_from_f64(p, dt, i, (double)v); break;
  }
}

__device__ __forceinline__ void store_from_i64(void* p, int dt, int64_t i, int64_t v) {
  switch (dt) {
    case TGM_BOOL: ((uint8_t*)p)[i] = v != 0; break;
    case TGM_I8: ((int8_t*)p)[i] = (int8_t)v; break;
    case TGM_U8: ((uint8_t*)p)[i] = (uint8_t)v; break;
    case TGM_I16: ((int16_t*)p)[i] = (int16_t)v; break;
    case TGM_U16: ((uint16_t*)p)[i] = (uint16_t)v; break;
    case TGM_I32: ((int32_t*)p)[i] = (int32_t)v; break;
    case TGM_U32: ((uint32_t*)p)[i] = (uint32_t)v; break;
    case TGM_I64: ((int64_t*)p)[i] = v; break;
    case TGM_U64: ((uint64_t*)p)[i] = (uint64_t)v; break;
    default: store_from_f64(p, dt, i, (double)v); break;
  }
}

__host__ __device__ inline bool is_float_dtype(int dt) {
  return dt == TGM_F16 || dt == TGM_BF16 || dt == TGM_F32 || dt == TGM_F64 || dt == TGM_FP8E4M3 ||
         dt == TGM_FP8E5M2 || dt == TGM_E8M0;
}

}  // namespace tgm
