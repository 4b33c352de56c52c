// Vendor comparison for the FP4 x FP4 block-scaled GEMM: the MXFP4 GEMM instances that
// ROCm's Composable Kernel ships prebuilt (libdevice_gemm_operations.a,
// add_device_gemm_mx_xdl_f4_f4_f16_mk_nk_mn_default_instances: A [M, K] and B [N, K]
// K-contiguous FP4 E2M1, E8M0 scales per 32, fp16 out), timed on the same operands as
// this library's tgm_gemm_mx in one process.  The hipBLASLt of this ROCm image ships no
// FP4 kernels for gfx950, so Composable Kernel is the vendor bar here.
//
// Every E8M0 byte is 127 (2^0): Composable Kernel reads its scales in its own shuffled
// order, and with one value everywhere that order cannot change the product.  The FP4 codes
// are random bytes.  Both libraries' outputs are checked against an exact host sum at 64
// sampled outputs (relative to the largest |C| sampled), so neither figure is of a wrong
// product.
//
// Usage: ck_mx_gemm_bar M N K [timed_launches [libtgm_mi355x.so [tgm-only]]] -- one line per
// step on stdout (unbuffered), then one JSON line: {"ck_best_us": .., "tgm_us": .., ...}.  With
// "tgm-only" the Composable Kernel instances are not run (their fields read -1).
#include <hip/hip_runtime.h>
#include <dlfcn.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "ck/ck.hpp"
#include "ck/library/tensor_operation_instance/gpu/gemm_mx.hpp"
#include "ck/tensor_operation/gpu/element/element_wise_operation.hpp"

namespace {

using PassThrough = ck::tensor_operation::element_wise::PassThrough;
using Row = ck::tensor_layout::gemm::RowMajor;
using Col = ck::tensor_layout::gemm::ColumnMajor;
using Mfma = ck::tensor_layout::gemm::MFMA;
using DeviceOp = ck::tensor_operation::device::DeviceGemmMX<Row, Col, Row, ck::f4x2_pk_t, int32_t, ck::f4x2_pk_t,
                                                            int32_t, ck::half_t, 32, PassThrough, PassThrough,
                                                            PassThrough>;
using DeviceOpPre = ck::tensor_operation::device::DeviceGemmMX<Row, Mfma, Row, ck::f4x2_pk_t, int32_t, ck::f4x2_pk_t,
                                                               int32_t, ck::half_t, 32, PassThrough, PassThrough,
                                                               PassThrough>;

#define CK_HIP(x)                                                                         \
  do {                                                                                    \
    hipError_t e_ = (x);                                                                  \
    if (e_ != hipSuccess) {                                                               \
      printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);                \
      exit(2);                                                                            \
    }                                                                                     \
  } while (0)

const float kFp4[16] = {0.f, .5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f, -0.f, -.5f, -1.f, -1.5f, -2.f, -3.f, -4.f, -6.f};

float half_to_float(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
float bf16_to_float(uint16_t h) { return __builtin_bit_cast(float, (unsigned)h << 16); }

// Median of ``n`` launches, each bracketed by events, after at least 60 ms of untimed launches
// (the clocks rise over the first tens of milliseconds of MFMA load).
template <typename F>
double median_us(hipStream_t s, F&& launch, int n) {
  hipEvent_t e0, e1;
  CK_HIP(hipEventCreate(&e0));
  CK_HIP(hipEventCreate(&e1));
  double spent = 0;
  int done = 0;
  while (spent < 60.0 || done < 10) {
    CK_HIP(hipEventRecord(e0, s));
    for (int i = 0; i < 5; ++i) launch();
    CK_HIP(hipEventRecord(e1, s));
    CK_HIP(hipEventSynchronize(e1));
    float ms;
    CK_HIP(hipEventElapsedTime(&ms, e0, e1));
    spent += ms;
    done += 5;
    if (done > 2000) break;
  }
  std::vector<hipEvent_t> ev(2 * n);
  for (auto& e : ev) CK_HIP(hipEventCreate(&e));
  for (int i = 0; i < n; ++i) {
    CK_HIP(hipEventRecord(ev[2 * i], s));
    launch();
    CK_HIP(hipEventRecord(ev[2 * i + 1], s));
  }
  CK_HIP(hipStreamSynchronize(s));
  std::vector<double> t(n);
  for (int i = 0; i < n; ++i) {
    float ms;
    CK_HIP(hipEventElapsedTime(&ms, ev[2 * i], ev[2 * i + 1]));
    t[i] = ms * 1e3;
  }
  for (auto& e : ev) CK_HIP(hipEventDestroy(e));
  CK_HIP(hipEventDestroy(e0));
  CK_HIP(hipEventDestroy(e1));
  std::sort(t.begin(), t.end());
  return t[n / 2];
}

}  // namespace

int main(int argc, char** argv) {
  setvbuf(stdout, nullptr, _IONBF, 0);
  if (argc < 4) {
    printf("usage: %s M N K [timed_launches]\n", argv[0]);
    return 2;
  }
  const int M = atoi(argv[1]), N = atoi(argv[2]), K = atoi(argv[3]);
  const int timed = argc > 4 ? atoi(argv[4]) : 20;
  if (M <= 0 || N <= 0 || K <= 0 || K % 256 || M % 256 || N % 256 || timed < 1) {
    printf("sizes must be positive multiples of 256\n");
    return 2;
  }
  const double flops = 2.0 * M * N * K;
  printf("step: operands M=%d N=%d K=%d\n", M, N, K);
  const size_t abytes = (size_t)M * K / 2, bbytes = (size_t)N * K / 2;
  const size_t sabytes = (size_t)M * K / 32, sbbytes = (size_t)N * K / 32;
  std::vector<unsigned char> ha(abytes), hb(bbytes);
  unsigned long long st = 0x243F6A8885A308D3ull;
  auto next = [&]() {
    st = st * 6364136223846793005ull + 1442695040888963407ull;
    return (unsigned char)(st >> 56);
  };
  for (auto& v : ha) v = next();
  for (auto& v : hb) v = next();
  void *a, *b, *sa, *sb, *c16, *c32;
  CK_HIP(hipMalloc(&a, abytes));
  CK_HIP(hipMalloc(&b, bbytes));
  CK_HIP(hipMalloc(&sa, sabytes));
  CK_HIP(hipMalloc(&sb, sbbytes));
  CK_HIP(hipMalloc(&c16, (size_t)M * N * 2));
  CK_HIP(hipMalloc(&c32, (size_t)M * N * 2));
  CK_HIP(hipMemcpy(a, ha.data(), abytes, hipMemcpyHostToDevice));
  CK_HIP(hipMemcpy(b, hb.data(), bbytes, hipMemcpyHostToDevice));
  CK_HIP(hipMemset(sa, 127, sabytes));
  CK_HIP(hipMemset(sb, 127, sbbytes));
  hipStream_t s;
  CK_HIP(hipStreamCreate(&s));

  // exact host sums at 64 sampled outputs
  std::vector<int> sm(64), sn(64);
  std::vector<double> want(64);
  double wmax = 0;
  for (int i = 0; i < 64; ++i) {
    sm[i] = (int)((i * 2654435761u) % (unsigned)M);
    sn[i] = (int)((i * 40503u + 7919u) % (unsigned)N);
    double acc = 0;
    for (int k = 0; k < K; ++k) {
      const unsigned char ba = ha[((size_t)sm[i] * K + k) / 2], bb = hb[((size_t)sn[i] * K + k) / 2];
      const int ca = k & 1 ? ba >> 4 : ba & 15, cb = k & 1 ? bb >> 4 : bb & 15;
      acc += (double)kFp4[ca] * kFp4[cb];
    }
    want[i] = acc;
    wmax = std::max(wmax, std::fabs(acc));
  }
  auto check = [&](void* c, bool bf16) {
    std::vector<uint16_t> row(1);
    double err = 0;
    for (int i = 0; i < 64; ++i) {
      CK_HIP(hipMemcpy(row.data(), (uint16_t*)c + (size_t)sm[i] * N + sn[i], 2, hipMemcpyDeviceToHost));
      const double got = bf16 ? bf16_to_float(row[0]) : half_to_float(row[0]);
      err = std::max(err, std::fabs(got - want[i]) / std::max(wmax, 1e-30));
    }
    return err;
  };

  // this library's kernel on the same operands
  double tgm_us = -1, tgm_err = -1;
  if (argc > 5) {
    printf("step: load %s\n", argv[5]);
    void* lib = dlopen(argv[5], RTLD_NOW | RTLD_LOCAL);
    if (!lib) {
      printf("dlopen failed: %s\n", dlerror());
      return 2;
    }
    typedef int (*gemm_fn)(const void*, int, const void*, int64_t, const void*, int, const void*, int64_t, int64_t,
                           void*, int, int64_t, void*);
    auto fn = (gemm_fn)dlsym(lib, "tgm_gemm_mx");
    if (!fn) {
      printf("tgm_gemm_mx not exported\n");
      return 2;
    }
    const int fp4 = 2, bf16 = 12;
    auto run = [&]() {
      const int rc = fn(a, fp4, sa, M, b, fp4, sb, N, K, c32, bf16, N, s);
      if (rc != 0) {
        printf("tgm_gemm_mx returned %d\n", rc);
        exit(2);
      }
    };
    printf("step: tgm_gemm_mx\n");
    tgm_us = median_us(s, run, timed);
    tgm_err = check(c32, true);
    printf("tgm_gemm_mx: %.1f us  %.1f TFLOP/s  max rel err %.2e\n", tgm_us, flops / tgm_us * 1e-6, tgm_err);
  }

  const bool tgm_only = argc > 6 && std::string(argv[6]) == "tgm-only";
  std::vector<std::unique_ptr<DeviceOp>> ops;
  std::vector<std::unique_ptr<DeviceOpPre>> pre;
  if (!tgm_only) {
    printf("step: list Composable Kernel MXFP4 instances\n");
    ck::tensor_operation::device::instance::add_device_gemm_mx_xdl_f4_f4_f16_mk_nk_mn_default_instances(ops);
    ck::tensor_operation::device::instance::add_device_gemm_mx_xdl_f4_f4_f16_mk_mfma_mn_default_instances(pre);
  }
  printf("%zu instances\n", ops.size());
  double best = 1e30, best_err = -1;
  std::string best_name;
  int supported = 0;
  for (size_t i = 0; i < ops.size(); ++i) {
    auto& op = ops[i];
    auto arg = op->MakeArgumentPointer(a, sa, b, sb, c16, M, N, K, K, K / 32, K, K / 32, N, 1, PassThrough{},
                                       PassThrough{}, PassThrough{});
    const std::string name = op->GetTypeString();
    if (!op->IsSupportedArgument(arg.get())) {
      printf("instance %zu unsupported: %s\n", i, name.c_str());
      continue;
    }
    ++supported;
    auto inv = op->MakeInvokerPointer();
    printf("step: instance %zu %s\n", i, name.c_str());
    auto run = [&]() { inv->Run(arg.get(), StreamConfig{s, false}); };
    CK_HIP(hipMemsetAsync(c16, 0, (size_t)M * N * 2, s));
    run();
    CK_HIP(hipStreamSynchronize(s));
    const double err = check(c16, false);
    const double us = median_us(s, run, timed);
    printf("instance %zu: %.1f us  %.1f TFLOP/s  max rel err %.2e\n", i, us, flops / us * 1e-6, err);
    if (err <= 1e-2 && us < best) {
      best = us;
      best_name = name;
      best_err = err;
    }
  }
  // B pre-shuffled into Composable Kernel's MFMA operand order (the layout its fastest
  // kernels read straight into registers): timed on the same random bytes, which in that
  // order are a different (equally random) B, so its output is not checked.
  printf("%zu instances with pre-shuffled B\n", pre.size());
  double best_pre = 1e30;
  std::string best_pre_name;
  for (size_t i = 0; i < pre.size(); ++i) {
    auto& op = pre[i];
    auto arg = op->MakeArgumentPointer(a, sa, b, sb, c16, M, N, K, K, K / 32, K, K / 32, N, 1, PassThrough{},
                                       PassThrough{}, PassThrough{});
    const std::string name = op->GetTypeString();
    if (!op->IsSupportedArgument(arg.get())) {
      printf("pre-shuffled instance %zu unsupported: %s\n", i, name.c_str());
      continue;
    }
    auto inv = op->MakeInvokerPointer();
    printf("step: pre-shuffled instance %zu %s\n", i, name.c_str());
    auto run = [&]() { inv->Run(arg.get(), StreamConfig{s, false}); };
    const double us = median_us(s, run, timed);
    printf("pre-shuffled instance %zu: %.1f us  %.1f TFLOP/s\n", i, us, flops / us * 1e-6);
    if (us < best_pre) {
      best_pre = us;
      best_pre_name = name;
    }
  }
  printf("{\"M\": %d, \"N\": %d, \"K\": %d, \"ck_instances\": %zu, \"ck_supported\": %d, \"ck_best_us\": %.3f, "
         "\"ck_best_tflops\": %.1f, \"ck_best_err\": %.3g, \"ck_best_instance\": \"%s\", \"tgm_us\": %.3f, "
         "\"tgm_tflops\": %.1f, \"tgm_err\": %.3g, \"ck_preshuffled_best_us\": %.3f, \"ck_preshuffled_best_instance\": \"%s\"}\n",
         M, N, K, ops.size(), supported, best < 1e29 ? best : -1.0, best < 1e29 ? flops / best * 1e-6 : -1.0,
         best_err, best_name.c_str(), tgm_us, tgm_us > 0 ? flops / tgm_us * 1e-6 : -1.0, tgm_err, best_pre < 1e29 ? best_pre : -1.0,
         best_pre_name.c_str());
  return 0;
}
