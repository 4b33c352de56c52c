// Tensor-level pack: MX block quantisation and the LSB-first code packer.
//
// The reference accepts only pre-packed bytes (alexandreteles/tinygrad-dx12
// src/tinygrad_dx12/codegen/decomp/dx12.py:26-30); its only packers live in the
// harness and tests (scripts/benchmark_dtypes.py:129-152, test/backend/test_packed.py:81-84)
// and pack payload codes least-significant bit first.  tgm_pack_codes produces that
// byte stream; tgm_quantize_mx adds the OCP MX quantiser that the reference lacks.
#include "tgm_common.h"

namespace tgm {

// Largest-normal exponent of each MX element format.
__device__ __forceinline__ int emax_elem(int fmt) { return fmt == TGM_FMT_FP6_E3M2 ? 4 : 2; }

// One thread per (row, block): amax -> shared exponent -> RNE codes -> packed bytes.
// Requires rows and blocks to start on byte boundaries (checked on the host).
__global__ void __launch_bounds__(256) quantize_mx_kernel(const void* __restrict__ x, int xdt, int64_t rows, int64_t k,
                                                          int fmt, int64_t bs, int64_t nblk,
                                                          uint8_t* __restrict__ data, uint8_t* __restrict__ scales) {
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= rows * nblk) return;
  const int64_t row = id / nblk, blk = id - row * nblk;
  const int64_t c0 = blk * bs;
  const int64_t c1 = c0 + bs < k ? c0 + bs : k;
  const FormatInfo f = format_info(fmt);
  const int64_t base = row * k;
  float amax = 0.f;
  for (int64_t c = c0; c < c1; ++c) amax = fmaxf(amax, fabsf(load_f32(x, xdt, base + c)));
  int shared = 0;
  if (amax > 0.f) {
    int e;
    frexpf(amax, &e);  // amax = m * 2^e, m in [0.5, 1)
    shared = (e - 1) - emax_elem(fmt);
    shared = shared < -127 ? -127 : (shared > 127 ? 127 : shared);
  }
  scales[id] = (uint8_t)(shared + 127);
  // ascending magnitudes of the positive payloads and their midpoints
  const int npos = 1 << (f.bits - 1);
  float mids[31];
  float prev = decode_float(0, f);
  for (int j = 1; j < npos; ++j) {
    const float cur = decode_float((uint32_t)j, f);
    mids[j - 1] = 0.5f * (prev + cur);
    prev = cur;
  }
  uint64_t acc = 0;
  int nbits = 0;
  int64_t out = (base + c0) * f.bits / 8;
  for (int64_t c = c0; c < c1; ++c) {
    const float v = ldexpf(load_f32(x, xdt, base + c), -shared);
    const float a = fabsf(v);
    uint32_t idx = 0;
    for (int j = 0; j < npos - 1; ++j)
      if (a > mids[j] || (a == mids[j] && (j & 1))) idx = (uint32_t)j + 1;
    const uint32_t sign = (v < 0.f && idx > 0) ? 1u : 0u;
    const uint32_t code = (sign << (f.bits - 1)) | idx;
    acc |= (uint64_t)code << nbits;
    nbits += f.bits;
    while (nbits >= 8) {
      data[out++] = (uint8_t)(acc & 0xFF);
      acc >>= 8;
      nbits -= 8;
    }
  }
  if (nbits > 0) data[out] = (uint8_t)(acc & 0xFF);
}

// Eight codes per thread: 4 bytes (4-bit) or 6 bytes (6-bit) at byte offset t*bits.
__global__ void __launch_bounds__(256) pack_codes_kernel(const uint8_t* __restrict__ codes, int64_t count, int bits,
                                                         uint8_t* __restrict__ out) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t first = t * 8;
  if (first >= count) return;
  uint64_t acc = 0;
  const uint32_t mask = (1u << bits) - 1u;
  for (int j = 0; j < 8; ++j) {
    const int64_t i = first + j;
    const uint64_t c = i < count ? (uint64_t)(codes[i] & mask) : 0ull;
    acc |= c << (j * bits);
  }
  const int64_t nbytes_total = (count * bits + 7) / 8;
  const int64_t o = t * bits;
  for (int b = 0; b < bits; ++b)
    if (o + b < nbytes_total) out[o + b] = (uint8_t)((acc >> (8 * b)) & 0xFF);
}

}  // namespace tgm

using namespace tgm;

extern "C" int tgm_quantize_mx(const void* x, int x_dtype, int64_t rows, int64_t k, int fmt, int64_t block_size,
                               void* data, void* scales, void* stream) {
  clear_error();
  TGM_CHECK_ARG(fmt == TGM_FMT_FP4_E2M1 || fmt == TGM_FMT_FP6_E2M3 || fmt == TGM_FMT_FP6_E3M2,
                "MX quantisation needs an FP4/FP6 format");
  TGM_CHECK_ARG(x_dtype == TGM_BF16 || x_dtype == TGM_F16 || x_dtype == TGM_F32, "quantiser input must be bf16/f16/f32");
  TGM_CHECK_ARG(rows >= 0 && k >= 1 && block_size >= 1, "invalid quantiser sizes");
  const int bits = format_info(fmt).bits;
  TGM_CHECK_ARG((k * bits) % 8 == 0 && (block_size * bits) % 8 == 0,
                "rows and blocks must start on byte boundaries (K*bits and block*bits multiples of 8)");
  if (rows == 0) return TGM_OK;
  const int64_t nblk = (k + block_size - 1) / block_size;
  const int64_t total = rows * nblk;
  hipLaunchKernelGGL(quantize_mx_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream, x,
                     x_dtype, rows, k, fmt, block_size, nblk, (uint8_t*)data, (uint8_t*)scales);
  return launch_status("tgm_quantize_mx");
}

extern "C" int tgm_pack_codes(const void* codes, int64_t count, int bits, void* out, void* stream) {
  clear_error();
  TGM_CHECK_ARG(bits == 4 || bits == 6, "pack width must be 4 or 6 bits");
  TGM_CHECK_ARG(count >= 0, "invalid code count");
  if (count == 0) return TGM_OK;
  const int64_t threads = (count + 7) / 8;
  hipLaunchKernelGGL(pack_codes_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint8_t*)codes, count, bits, (uint8_t*)out);
  return launch_status("tgm_pack_codes");
}
