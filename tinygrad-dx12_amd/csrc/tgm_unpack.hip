// Packed decode (PackedTensor.unpack, alexandreteles/tinygrad-dx12
// src/tinygrad_dx12/codegen/decomp/dx12.py:49-106) and the library's error plumbing.
//
// One thread decodes eight consecutive logical elements of the flattened array.  The
// payload of element i is read straight from the bit stream (two bytes cover any
// 4- or 6-bit payload), so rows that do not start on a byte boundary (odd K for
// 4-bit, K % 4 != 0 for 6-bit) decode exactly like the reference's flat word view.
#include <atomic>

#include "tgm_common.h"

namespace tgm {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_last_error[0] = 0; }

int launch_status(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("%s launch failed: %s (%d)", what, hipGetErrorString(err), (int)err);
    return (int)err;
  }
  return TGM_OK;
}

int stream_cu_count(hipStream_t stream) {
  static std::atomic<int> counts[64];  // per device, 0 = not looked up yet
  int device = -1;
  if (stream != nullptr && stream != hipStreamLegacy && stream != hipStreamPerThread) {
    hipDevice_t d = -1;
    if (hipStreamGetDevice(stream, &d) != hipSuccess) return 0;
    device = (int)d;
  } else if (hipGetDevice(&device) != hipSuccess) {
    return 0;
  }
  if (device < 0 || device >= 64) return 0;
  int n = counts[device].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || n < 0) return 0;
    counts[device].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Value of one element in the multiplication type of dx12.py:103 and its final cast.
template <typename MT>
__device__ __forceinline__ void decode_store(uint32_t p, int fmt, FormatInfo f, bool has_scale, MT scale,
                                             void* out, int odt, int64_t i) {
  if (is_int_format(fmt)) {
    const int32_t v = decode_int(p, fmt);
    if (has_scale) {
      store_from_f64(out, odt, i, (double)((MT)v * scale));
    } else if (odt == TGM_F32 || odt == TGM_F16 || odt == TGM_BF16) {
      store_from_f32(out, odt, i, (float)v);
    } else {
      store_from_i64(out, odt, i, (int64_t)v);
    }
  } else {
    const float v = decode_float(p, f);
    if (has_scale) {
      const MT prod = (MT)v * scale;
      if (sizeof(MT) == 4) store_from_f32(out, odt, i, (float)prod);
      else store_from_f64(out, odt, i, (double)prod);
    } else {
      store_from_f32(out, odt, i, v);
    }
  }
}

template <typename MT>
__global__ void __launch_bounds__(256) unpack_kernel(const uint8_t* __restrict__ data, int64_t nbytes, int fmt,
                                                     int64_t count, int64_t k, const void* __restrict__ scales,
                                                     int sdt, int64_t nblk, int64_t bs, void* __restrict__ out,
                                                     int odt, int fp8_target) {
  const FormatInfo f = format_info(fmt);
  const int64_t stride = (int64_t)gridDim.x * blockDim.x * 8;
  for (int64_t base = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8; base < count; base += stride) {
    int64_t row = base / k, col = base - row * k;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t i = base + j;
      if (i >= count) break;
      const uint32_t p = payload_at(data, nbytes, i, f.bits);
      if (fp8_target) {
        ((uint8_t*)out)[i] = fp8_target == 1 ? fp8_direct(p, f, 3, 7) : fp8_direct(p, f, 2, 15);
      } else if (scales) {
        const int64_t si = row * nblk + col / bs;
        MT s;
        if (sizeof(MT) == 8) s = (MT)load_f64(scales, sdt, si);
        else s = (MT)load_f32(scales, sdt, si);
        decode_store<MT>(p, fmt, f, true, s, out, odt, i);
      } else {
        decode_store<MT>(p, fmt, f, false, (MT)1, out, odt, i);
      }
      if (++col == k) { col = 0; ++row; }
    }
  }
}

}  // namespace tgm

using namespace tgm;

extern "C" int tgm_abi_version(void) { return TGM_ABI_VERSION; }

extern "C" const char* tgm_last_error(void) { return g_last_error; }

extern "C" int tgm_device_arch(int ordinal, char* out, int64_t len) {
  clear_error();
  TGM_CHECK_ARG(out && len > 0, "null output");
  hipDeviceProp_t prop;
  const hipError_t e = hipGetDeviceProperties(&prop, ordinal);
  if (e != hipSuccess) {
    set_error("hipGetDeviceProperties(%d) failed: %s", ordinal, hipGetErrorString(e));
    return (int)e;
  }
  snprintf(out, (size_t)len, "%s", prop.gcnArchName);
  return TGM_OK;
}

extern "C" int tgm_unpack(const void* data, int64_t nbytes, int fmt, int64_t count, int64_t k, const void* scales,
                          int scale_dtype, int64_t block_size, void* out, int out_dtype, void* stream) {
  clear_error();
  TGM_CHECK_ARG(valid_format(fmt), "unknown packed format %d", fmt);
  TGM_CHECK_ARG(count >= 0 && k >= 1 && block_size >= 1 && nbytes >= 0, "invalid unpack sizes");
  const int bits = format_info(fmt).bits;
  TGM_CHECK_ARG(nbytes >= (count * bits + 7) / 8, "packed storage is smaller than the declared shape");
  TGM_CHECK_ARG(dtype_size(out_dtype) > 0 && out_dtype != TGM_E8M0, "invalid output dtype %d", out_dtype);
  TGM_CHECK_ARG(!scales || (dtype_size(scale_dtype) > 0), "invalid scale dtype %d", scale_dtype);
  if (count == 0) return TGM_OK;
  int fp8_target = 0;
  if (!scales && !is_int_format(fmt)) {
    // FP8_CANDIDATES (dx12.py:11): fp4 -> {e4m3, e5m2}; e2m3 -> {e4m3}; e3m2 -> {e4m3, e5m2}
    if (out_dtype == TGM_FP8E4M3) fp8_target = 1;
    if (out_dtype == TGM_FP8E5M2 && fmt != TGM_FMT_FP6_E2M3) fp8_target = 2;
  }
  const int64_t nblk = (k + block_size - 1) / block_size;
  const bool wide = scales && (scale_dtype == TGM_F64 || out_dtype == TGM_F64);
  const int64_t threads = (count + 7) / 8;
  int64_t blocks = (threads + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipStream_t s = (hipStream_t)stream;
  if (wide)
    hipLaunchKernelGGL(unpack_kernel<double>, dim3((unsigned)blocks), dim3(256), 0, s, (const uint8_t*)data, nbytes,
                       fmt, count, k, scales, scale_dtype, nblk, block_size, out, out_dtype, fp8_target);
  else
    hipLaunchKernelGGL(unpack_kernel<float>, dim3((unsigned)blocks), dim3(256), 0, s, (const uint8_t*)data, nbytes,
                       fmt, count, k, scales, scale_dtype, nblk, block_size, out, out_dtype, fp8_target);
  return launch_status("tgm_unpack");
}
