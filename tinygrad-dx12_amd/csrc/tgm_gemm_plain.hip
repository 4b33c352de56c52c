// Exact-width GEMM for operand combinations outside the MFMA families.
//
// This is the device analogue of the reference's ordinary-matmul fallback
// (alexandreteles/tinygrad-dx12 src/tinygrad_dx12/codegen/linalg.py:169-174 and
// :219-223).  Products are formed at the accumulator width, as the reference's DX12
// device does for narrow integers (test/backend/test_linalg.py:221-230), so int8/uint8
// products never wrap and fp64/int64 operands keep their precision
// (test_linalg.py:173-183, :202-218).
//
// 16x16 output tile per workgroup; each thread owns one output element and walks K.
// Operands are read through element strides, so transposed views need no copy.
#include "tgm_common.h"

namespace tgm {

template <typename Acc>
__device__ __forceinline__ Acc load_acc(const void* p, int dt, int64_t i);

template <>
__device__ __forceinline__ float load_acc<float>(const void* p, int dt, int64_t i) { return load_f32(p, dt, i); }
template <>
__device__ __forceinline__ double load_acc<double>(const void* p, int dt, int64_t i) { return load_f64(p, dt, i); }
template <>
__device__ __forceinline__ uint64_t load_acc<uint64_t>(const void* p, int dt, int64_t i) {
  return (uint64_t)load_i64(p, dt, i);
}

template <typename Acc>
__device__ __forceinline__ void store_acc(void* p, int dt, int64_t i, Acc v);
template <>
__device__ __forceinline__ void store_acc<float>(void* p, int dt, int64_t i, float v) { store_from_f32(p, dt, i, v); }
template <>
__device__ __forceinline__ void store_acc<double>(void* p, int dt, int64_t i, double v) { store_from_f64(p, dt, i, v); }
template <>
__device__ __forceinline__ void store_acc<uint64_t>(void* p, int dt, int64_t i, uint64_t v) {
  if (dt == TGM_U64) ((uint64_t*)p)[i] = v;
  else if (is_float_dtype(dt)) store_from_f64(p, dt, i, (double)(int64_t)v);
  else store_from_i64(p, dt, i, (int64_t)v);
}

template <typename Acc>
__global__ void __launch_bounds__(256) gemm_plain_kernel(const void* __restrict__ a, int adt, int64_t sa0, int64_t sa1,
                                                         const void* __restrict__ b, int bdt, int64_t sb0, int64_t sb1,
                                                         void* __restrict__ c, int cdt, int64_t sc0, int64_t sc1,
                                                         int64_t M, int64_t N, int64_t K) {
  const int64_t i = (int64_t)blockIdx.y * 16 + (threadIdx.x >> 4);
  const int64_t j = (int64_t)blockIdx.x * 16 + (threadIdx.x & 15);
  if (i >= M || j >= N) return;
  Acc acc = (Acc)0;
  for (int64_t kk = 0; kk < K; ++kk)
    acc += load_acc<Acc>(a, adt, i * sa0 + kk * sa1) * load_acc<Acc>(b, bdt, kk * sb0 + j * sb1);
  store_acc<Acc>(c, cdt, i * sc0 + j * sc1, acc);
}

}  // namespace tgm

using namespace tgm;

extern "C" int tgm_gemm_plain(const void* a, int a_dtype, int64_t sa0, int64_t sa1, const void* b, int b_dtype,
                              int64_t sb0, int64_t sb1, void* c, int c_dtype, int64_t sc0, int64_t sc1, int64_t m,
                              int64_t n, int64_t k, int acc_dtype, void* stream) {
  clear_error();
  TGM_CHECK_ARG(m >= 0 && n >= 0 && k >= 0, "invalid gemm sizes");
  TGM_CHECK_ARG(dtype_size(a_dtype) > 0 && dtype_size(b_dtype) > 0 && dtype_size(c_dtype) > 0, "invalid gemm dtype");
  if (m == 0 || n == 0) return TGM_OK;
  hipStream_t s = (hipStream_t)stream;
  dim3 grid((unsigned)((n + 15) / 16), (unsigned)((m + 15) / 16));
  TGM_CHECK_ARG(grid.y <= 65535u, "M too large for the plain gemm grid");
  switch (acc_dtype) {
    case TGM_F32:
      hipLaunchKernelGGL(gemm_plain_kernel<float>, grid, dim3(256), 0, s, a, a_dtype, sa0, sa1, b, b_dtype, sb0, sb1, c,
                         c_dtype, sc0, sc1, m, n, k);
      break;
    case TGM_F64:
      hipLaunchKernelGGL(gemm_plain_kernel<double>, grid, dim3(256), 0, s, a, a_dtype, sa0, sa1, b, b_dtype, sb0, sb1, c,
                         c_dtype, sc0, sc1, m, n, k);
      break;
    case TGM_I32: case TGM_U32: case TGM_I64: case TGM_U64:
      hipLaunchKernelGGL(gemm_plain_kernel<uint64_t>, grid, dim3(256), 0, s, a, a_dtype, sa0, sa1, b, b_dtype, sb0, sb1,
                         c, c_dtype, sc0, sc1, m, n, k);
      break;
    default:
      TGM_CHECK_ARG(false, "accumulator dtype %d is not supported", acc_dtype);
  }
  return launch_status("tgm_gemm_plain");
}
