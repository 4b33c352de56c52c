// Measurement probes: the ceilings the packed kernels are judged against on this machine.
//
// No reference counterpart (the reference has no kernels of its own to measure).  bench.py
// times them like the kernels they bound:
//
//  * tgm_probe_read streams ``nbytes`` from device memory with the decode GEMV's access shape
//    (each wave reads a contiguous run, 16 bytes per lane per instruction, all of a wave's loads
//    in flight, non-temporal) and discards the data: the fastest a single launch can read the
//    bytes a GEMV of that size must read.
//  * tgm_probe_mfma_fp4 issues v_mfma_scale_f32_32x32x64_f8f6f4 on FP4 operands from registers
//    only, with operand bits changing every instruction as a GEMM's do (the chip's power draw,
//    and with it the clock it sustains, depends on operand toggling): the FP4 MFMA throughput
//    the FP4 GEMM could reach with no data movement at all, on the GEMM's grid (1024
//    workgroups of 8 waves at 8192^3).
//  * tgm_probe_launch is an empty kernel: the fixed cost of one launch of a grid, which a
//    memory-bound kernel of a few microseconds pays in full on top of its transfer time.
//  * tgm_probe_bf16_rounding checks the hardware fp32 -> bf16 conversion every bf16 epilogue
//    uses (v_cvt_pk_bf16_f32 via bf16x2_bits) against the integer round-to-nearest-even formula,
//    in both halves of the packed pair, over any range of fp32 bit patterns (all 2^32 in one
//    launch), and can write the converted bits out for comparison on the host.
#include "tgm_mfma_common.h"

namespace tgm {

typedef unsigned u32x4p __attribute__((ext_vector_type(4)));

constexpr int kProbeRun = 8;  // 1 KB loads per wave: 8 KB contiguous per wave

__global__ void __launch_bounds__(256) probe_read(const unsigned char* __restrict__ p, int64_t nbytes,
                                                  unsigned* __restrict__ sink) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t base = wave * kProbeRun * 1024;
  u32x4p v[kProbeRun];
#pragma unroll
  for (int i = 0; i < kProbeRun; ++i) {
    int64_t off = base + (int64_t)i * 1024 + 16 * lane;
    off = off + 16 <= nbytes ? off : nbytes - 16;  // clamped inside the buffer
    v[i] = __builtin_nontemporal_load((const u32x4p*)(p + off));
  }
  unsigned x = 0;
#pragma unroll
  for (int i = 0; i < kProbeRun; ++i) x ^= v[i][0] ^ v[i][1] ^ v[i][2] ^ v[i][3];
  if (x == 0x9E3779B9u) sink[0] = x;  // keeps the loads; practically never stores
}

__global__ void __launch_bounds__(512) probe_mfma_fp4(int iters, unsigned seed, float* __restrict__ sink) {
  const int lane = threadIdx.x & 63;
  unsigned h = (blockIdx.x * 512u + threadIdx.x) * 2654435761u ^ seed;
  // four operand tuples held in place (no per-instruction register copies); consecutive MFMAs
  // alternate between them and one dword of each changes every round
  i32x8 ta[2], tb[2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      h = h * 1664525u + 1013904223u;
      ta[t][i] = (int)h;
      h = h * 1664525u + 1013904223u;
      tb[t][i] = (int)h;
      ta[t][4 + i] = 0;
      tb[t][4 + i] = 0;
    }
  const int sa = 124 + lane % 6, sb = 125 + lane % 5;  // E8M0 scales 2^-3 .. 2^2
  f32x16 acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = f32x16{};
  for (int it = 0; it < iters; it += 4) {  // iters is a multiple of 4 (host)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        acc[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(ta[j & 1], tb[(j >> 1) & 1], acc[j], 4, 4, 0, sa, 0, sb);
#pragma unroll
      for (int t = 0; t < 2; ++t) {  // new operand bits for the next round
        ta[t][r] ^= (int)(0x9E3779B9u * (unsigned)(it + r + 1));
        tb[t][(r + 1) & 3] += (int)(0x85EBCA6Bu * (unsigned)(it + r + 2));
      }
    }
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) s += acc[j][0] + acc[j][15];
  if (s == 1234.5f) sink[0] = s;  // keeps the MFMAs; practically never stores
}

// An empty kernel: what one launch of a given grid costs with no work at all -- dispatch, the
// workgroups' start and end, and the launch's completion -- timed like the kernels it bounds.
__global__ void __launch_bounds__(1024) probe_launch(unsigned* __restrict__ sink, int never) {
  if ((int)threadIdx.x == never) sink[0] = 1;  // the host passes a thread index past the block
}

// Inputs first + i for i < count (count even, at most 2^32); each thread takes 64 consecutive
// patterns as 32 pairs and converts each pair in both orders.  bad[0] counts mismatches, bad[1]
// receives the smallest mismatching pattern (the host starts them at 0 and 0xFFFFFFFF).
constexpr int kRoundRun = 64;

__global__ void __launch_bounds__(256) probe_bf16_rounding(uint32_t first, int64_t count,
                                                           uint16_t* __restrict__ bits, unsigned* __restrict__ bad) {
  const int64_t base = ((int64_t)blockIdx.x * 256 + threadIdx.x) * kRoundRun;
  unsigned n = 0, low = 0xFFFFFFFFu;
  for (int i = 0; i < kRoundRun && base + i < count; i += 2) {
    const uint32_t u0 = first + (uint32_t)(base + i), u1 = u0 + 1u;
    const float x0 = bits_f32(u0), x1 = bits_f32(u1);
    const uint32_t w0 = f32_to_bf16_int(x0), w1 = f32_to_bf16_int(x1);
    const uint32_t ab = bf16x2_bits(x0, x1), ba = bf16x2_bits(x1, x0);
    const bool bad0 = (ab & 0xFFFFu) != w0 || (ba >> 16) != w0;
    const bool bad1 = (ab >> 16) != w1 || (ba & 0xFFFFu) != w1;
    n += bad0 + bad1;
    if (bad0) low = min(low, u0);
    if (bad1) low = min(low, u1);
    if (bits) {
      bits[base + i] = (uint16_t)(ab & 0xFFFFu);
      bits[base + i + 1] = (uint16_t)(ab >> 16);
    }
  }
  if (n) {
    atomicAdd(&bad[0], n);
    atomicMin(&bad[1], low);
  }
}

}  // namespace tgm

using namespace tgm;

extern "C" int tgm_probe_bf16_rounding(uint32_t first, int64_t count, void* bits, void* bad, void* stream) {
  clear_error();
  TGM_CHECK_ARG(bad, "null operand");
  TGM_CHECK_ARG(count > 0 && count % 2 == 0 && count <= (1ll << 32) && first % 2 == 0 &&
                    (int64_t)first + count <= (1ll << 32),
                "invalid range (first and count even, first + count <= 2^32)");
  const int64_t per_block = 256 * kRoundRun;
  const int64_t grid = (count + per_block - 1) / per_block;
  hipLaunchKernelGGL(probe_bf16_rounding, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, first, count,
                     (uint16_t*)bits, (unsigned*)bad);
  return launch_status("tgm_probe_bf16_rounding");
}

extern "C" int tgm_probe_launch(int64_t groups, int64_t threads, void* sink, void* stream) {
  clear_error();
  TGM_CHECK_ARG(sink, "null operand");
  TGM_CHECK_ARG(groups > 0 && groups < (1ll << 31) && threads > 0 && threads <= 1024, "invalid launch shape");
  hipLaunchKernelGGL(probe_launch, dim3((unsigned)groups), dim3((unsigned)threads), 0, (hipStream_t)stream,
                     (unsigned*)sink, (int)threads);
  return launch_status("tgm_probe_launch");
}

extern "C" int tgm_probe_read(const void* p, int64_t nbytes, void* sink, void* stream) {
  clear_error();
  TGM_CHECK_ARG(p && sink, "null operand");
  TGM_CHECK_ARG(nbytes >= 16 && nbytes % 16 == 0, "nbytes must be a positive multiple of 16");
  const int64_t per_block = 4 * kProbeRun * 1024;
  const int64_t grid = (nbytes + per_block - 1) / per_block;
  TGM_CHECK_ARG(grid < (1ll << 31), "too many bytes");
  hipLaunchKernelGGL(probe_read, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, (const unsigned char*)p,
                     nbytes, (unsigned*)sink);
  return launch_status("tgm_probe_read");
}

extern "C" int tgm_probe_mfma_fp4(int64_t blocks, int64_t iters, void* sink, void* stream) {
  clear_error();
  TGM_CHECK_ARG(sink, "null operand");
  TGM_CHECK_ARG(blocks > 0 && blocks < (1ll << 31) && iters > 0 && iters < (1ll << 31) && iters % 4 == 0,
                "invalid sizes (iters a positive multiple of 4)");
  hipLaunchKernelGGL(probe_mfma_fp4, dim3((unsigned)blocks), dim3(512), 0, (hipStream_t)stream, (int)iters, 0x5EEDu,
                     (float*)sink);
  return launch_status("tgm_probe_mfma_fp4");
}
