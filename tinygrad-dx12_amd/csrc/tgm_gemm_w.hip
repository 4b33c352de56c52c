// Kernel family 2, dequant path: packed FP4 / FP6 weights x bf16 activations on bf16 MFMA.
//
// Replaces the reference's collective LinAlg GEMM (alexandreteles/tinygrad-dx12
// src/tinygrad_dx12/renderer/linalg.py:38-124) when one operand is packed: the reference
// decodes the weight to the fp32 intermediate in memory (codegen/decomp/dx12.py:49-106,
// 115-138) and multiplies that.  Here the packed codes are decoded in registers:
// v_cvt_scalef32_pk32_bf16_fp6 / _bf6 / _pk_bf16_fp4 turn 32 codes and their E8M0 scale into
// bf16 values.  An FP4/FP6 code times a power-of-two scale is exact in bf16, so the MFMA
// multiplies exactly the values the reference does; only the fp32 summation order differs.
//
//   C[m, n] = sum_k A[m, k] * deq(W)[n, k]      A bf16 [M, K] (row stride lda)
//                                               W packed [N, K], E8M0 scales [N, K/32]
//
// v_mfma_f32_32x32x16_bf16: lane l supplies row (l % 32) of A (column of B) and 8 K values.
// The K order inside a 128-element step is a free choice as long as A and B agree: lane
// half h = l / 32 owns K [64 h, 64 h + 64) of the step, and MFMA j (0..7) takes its values
// [64 h + 8 j, + 8).  So a lane's B data for a step is 64 consecutive codes of one weight
// row -- two MX blocks, two scale bytes -- decoded with two 32-wide conversions (FP6).
// D layout: lane l holds column l % 32, rows 8 (v / 4) + 4 (l / 32) + v % 4.
//
// Workgroup: 128 (M) x 256 (N) output tile, eight waves in 2 x 4, each 64 x 64 = 2 x 2 MFMA
// tiles.  K steps of 128: the A panel (128 rows x 256 B, XOR-swizzled 16-byte columns), the
// packed W panel (256 rows x 96 B for FP6, 64 B for FP4) and the step's scale dwords are
// loaded straight into a double-buffered LDS stage (buffer_load ... lds, zero-filled past
// M and N); the loads of step s + 2 run while step s + 1 computes.
#include "tgm_mfma_common.h"

namespace tgm {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
typedef __attribute__((__vector_size__(32 * sizeof(__bf16)))) __bf16 bf16x32;
typedef __attribute__((__vector_size__(6 * sizeof(int)))) int i32x6;

constexpr int kWM = 128, kWN = 256, kWK = 128;  // output tile and K step
constexpr int kAPanel = kWM * kWK * 2;           // 32 KB of bf16 A per stage
constexpr int kWPanelMax = kWN * 96;             // 24 KB of packed W (FP6) per stage
constexpr int kWScales = kWN * 4;                // one E8M0 dword (4 blocks) per W row per stage
constexpr int kWStage = kAPanel + kWPanelMax + kWScales;
constexpr int kWGroupM = 8;

template <int FMT>
struct GemmWTraits {
  static constexpr int kRow = FMT == TGM_FMT_FP4_E2M1 ? 64 : 96;  // packed bytes per W row per step
  static constexpr int kPanelLoads = kWN * kRow / 1024;             // 16-byte-per-lane load instructions
};

// Decode the 64 codes a lane owns in one step to 8 MFMA operands (K order 8 j .. 8 j + 7).
template <int FMT>
__device__ __forceinline__ void decode64(const u32x4* raw, unsigned sbits, bf16x8 out[8]) {
  const float s0 = __builtin_bit_cast(float, (sbits & 0xFFu) << 23);
  const float s1 = __builtin_bit_cast(float, ((sbits >> 8) & 0xFFu) << 23);
  if constexpr (FMT == TGM_FMT_FP4_E2M1) {
    // 32 bytes = 8 dwords; dword d holds codes 8 d .. 8 d + 7 (low nibble first)
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      const unsigned v = raw[d >> 2][d & 3];
      const float s = d < 4 ? s0 : s1;
      const bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, s, 0);
      const bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, s, 1);
      const bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, s, 2);
      const bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, s, 3);
      out[d] = bf16x8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
    }
  } else {
    // 48 bytes = 12 dwords: two 32-code blocks of 6 dwords
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      i32x6 v;
#pragma unroll
      for (int q = 0; q < 6; ++q) v[q] = (int)raw[(6 * blk + q) >> 2][(6 * blk + q) & 3];
      bf16x32 d;
      if constexpr (FMT == TGM_FMT_FP6_E2M3) d = __builtin_amdgcn_cvt_scalef32_pk32_bf16_fp6(v, blk ? s1 : s0);
      else d = __builtin_amdgcn_cvt_scalef32_pk32_bf16_bf6(v, blk ? s1 : s0);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        out[4 * blk + j] = bf16x8{d[8 * j], d[8 * j + 1], d[8 * j + 2], d[8 * j + 3],
                                  d[8 * j + 4], d[8 * j + 5], d[8 * j + 6], d[8 * j + 7]};
    }
  }
}

template <int FMT, bool SCALED>
__global__ void __launch_bounds__(512) gemm_w_mx(const uint8_t* __restrict__ a, unsigned lda_bytes,
                                                 const uint8_t* __restrict__ w, const uint8_t* __restrict__ sw,
                                                 int M, int N, int K, void* __restrict__ c, int cdt, int64_t ldc) {
  using T = GemmWTraits<FMT>;
  constexpr int FA = 2, FB = 2;
  __shared__ __attribute__((aligned(16))) unsigned char lds[2 * kWStage];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  const int tiles_m = (M + kWM - 1) / kWM, tiles_n = (N + kWN - 1) / kWN;
  int tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, kWGroupM, tm, tn);
  const int m0 = tm * kWM, n0 = tn * kWN;
  const int nsteps = K / kWK;
  const unsigned kbw = (unsigned)K / 8u * (FMT == TGM_FMT_FP4_E2M1 ? 4u : 6u);  // packed bytes per W row
  const unsigned kblk = (unsigned)K / 32u;
  const i32x4v ra = buffer_rsrc(a, (unsigned)(M - 1) * lda_bytes + (unsigned)K * 2u);
  const i32x4v rw = buffer_rsrc(w, (unsigned)N * kbw);
  const i32x4v rs = buffer_rsrc(sw, SCALED ? (unsigned)N * kblk : 0u);
  const unsigned lds_base = (unsigned)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)lds;

  // ---- global -> LDS load offsets (per lane, per instruction; the step adds a uniform part)
  // A: instruction i = 4 wave + q covers rows 4 i .. 4 i + 3; lane l fills slot l % 16 of row
  // 4 i + l / 16, which holds logical 16-byte column (l % 16) ^ (row % 16).
  unsigned voa[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int row = 4 * (4 * wave + q) + (lane >> 4);
    const unsigned col = (unsigned)((lane & 15) ^ (row & 15));
    voa[q] = (unsigned)(m0 + row) * lda_bytes + col * 16u;
  }
  // W: FP6 rows are 96 bytes, stored densely (flat byte f = row * 96 + b); FP4 rows are 64
  // bytes with 16-byte chunks swizzled by (row / 4) % 4.
  constexpr int NWL = (T::kPanelLoads + 7) / 8;  // W load instructions per wave
  unsigned vow[NWL];
#pragma unroll
  for (int q = 0; q < NWL; ++q) {
    const int i = NWL * wave + q;
    if constexpr (FMT == TGM_FMT_FP4_E2M1) {
      const int row = 16 * i + (lane >> 2);
      const unsigned chunk = (unsigned)((lane & 3) ^ ((row >> 2) & 3));
      vow[q] = (unsigned)(n0 + row) * kbw + chunk * 16u;
    } else {
      const int f = 1024 * i + 16 * lane;
      vow[q] = (unsigned)(n0 + f / 96) * kbw + (unsigned)(f % 96);
    }
  }
  const unsigned vos = (unsigned)(n0 + 64 * (wave & 3) + lane) * kblk;  // scale dword of row, waves 0..3

  auto dma_step = [&](int s, int buf) __attribute__((always_inline)) {
    const unsigned st = lds_base + (unsigned)(buf * kWStage);
#pragma unroll
    for (int q = 0; q < 4; ++q) lds_dma16(ra, st + (unsigned)(4 * wave + q) * 1024u, voa[q] + (unsigned)s * 256u);
#pragma unroll
    for (int q = 0; q < NWL; ++q)
      if (NWL * wave + q < T::kPanelLoads)
        lds_dma16(rw, st + kAPanel + (unsigned)(NWL * wave + q) * 1024u, vow[q] + (unsigned)s * (unsigned)T::kRow);
    if (SCALED && wave < 4) lds_dma4(rs, st + kAPanel + kWPanelMax + (unsigned)wave * 256u, vos + (unsigned)s * 4u);
  };

  // ---- fragment reads
  const int half = lane >> 5;
  const int a_row = wm * 64 + (lane & 31);  // + 32 t
  const int b_row = wn * 64 + (lane & 31);  // + 32 t
  auto read_a = [&](int buf, int j, bf16x8 out[FA]) __attribute__((always_inline)) {
    const unsigned char* pa = lds + buf * kWStage;
#pragma unroll
    for (int t = 0; t < FA; ++t) {
      const int row = a_row + 32 * t;
      const int col = (8 * half + j) ^ (row & 15);
      out[t] = *(const bf16x8*)(pa + row * 256 + col * 16);
    }
  };
  bf16x8 bfr[FB][8];
  auto read_decode_b = [&](int buf) __attribute__((always_inline)) {
    const unsigned char* pw = lds + buf * kWStage + kAPanel;
    const unsigned* ps = (const unsigned*)(lds + buf * kWStage + kAPanel + kWPanelMax);
#pragma unroll
    for (int t = 0; t < FB; ++t) {
      const int row = b_row + 32 * t;
      u32x4 raw[3];
      if constexpr (FMT == TGM_FMT_FP4_E2M1) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const int chunk = (2 * half + q) ^ ((row >> 2) & 3);
          raw[q] = *(const u32x4*)(pw + row * 64 + chunk * 16);
        }
      } else {
#pragma unroll
        for (int q = 0; q < 3; ++q) raw[q] = *(const u32x4*)(pw + row * 96 + 48 * half + 16 * q);
      }
      const unsigned sbits = SCALED ? ps[row] >> (16 * half) : 0x7F7Fu;  // blocks 2 h, 2 h + 1
      decode64<FMT>(raw, sbits, bfr[t]);
    }
  };

  f32x16 acc[FA][FB];
#pragma unroll
  for (int i = 0; i < FA; ++i)
#pragma unroll
    for (int j = 0; j < FB; ++j) acc[i][j] = f32x16{};

  const int s1 = nsteps > 1 ? 1 : 0;
  dma_step(0, 0);
  dma_step(s1, 1);
  wait_lds_dma();
  __syncthreads();
  for (int s = 0; s < nsteps; ++s) {
    const int cur = s & 1;
    const int s2 = s + 2 < nsteps ? s + 2 : nsteps - 1;
    read_decode_b(cur);
    bf16x8 af[2][FA];
    read_a(cur, 0, af[0]);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (j < 7) read_a(cur, j + 1, af[(j + 1) & 1]);
#pragma unroll
      for (int ta = 0; ta < FA; ++ta)
#pragma unroll
        for (int tb = 0; tb < FB; ++tb)
          acc[ta][tb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[j & 1][ta], bfr[tb][j], acc[ta][tb], 0, 0, 0);
    }
    wait_lds_dma();  // this wave's loads of step s + 1
    __syncthreads();  // every wave is done with this buffer; step s + 1 is complete in the other
    dma_step(s2, cur);
  }
  wait_lds_dma();
  __syncthreads();  // the epilogue reuses the LDS

  // Epilogue: each 32 x 32 tile through a per-wave LDS block (rows padded to 36 floats), then
  // 16-element row segments per lane, rounded once.
  float* ep = (float*)lds + wave * 32 * 36;
  const int er = lane >> 1, ec = (lane & 1) * 16;
  auto out_tile = [&](const f32x16 t, int i, int j) __attribute__((always_inline)) {
#pragma unroll
    for (int v = 0; v < 16; ++v) ep[(8 * (v >> 2) + 4 * half + (v & 3)) * 36 + (lane & 31)] = t[v];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float vals[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const f32x4 f = *(const f32x4*)(ep + er * 36 + ec + 4 * q);
      vals[4 * q] = f[0]; vals[4 * q + 1] = f[1]; vals[4 * q + 2] = f[2]; vals[4 * q + 3] = f[3];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int row = m0 + wm * 64 + i * 32 + er;
    const int col = n0 + wn * 64 + j * 32 + ec;
    if (row < M) {
      const int64_t o = (int64_t)row * ldc + col;
      if (col + 15 < N && (o & 7) == 0 && cdt != TGM_F32) {
        unsigned pk[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          if (cdt == TGM_BF16)
            pk[q] = f32_to_bf16(vals[2 * q]) | ((unsigned)f32_to_bf16(vals[2 * q + 1]) << 16);
          else
            pk[q] = __builtin_bit_cast(unsigned short, (_Float16)vals[2 * q]) |
                    ((unsigned)__builtin_bit_cast(unsigned short, (_Float16)vals[2 * q + 1]) << 16);
        }
        *(u32x4*)((uint16_t*)c + o) = u32x4{pk[0], pk[1], pk[2], pk[3]};
        *(u32x4*)((uint16_t*)c + o + 8) = u32x4{pk[4], pk[5], pk[6], pk[7]};
      } else if (col + 15 < N && (o & 3) == 0 && cdt == TGM_F32) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *(f32x4*)((float*)c + o + 4 * q) = f32x4{vals[4 * q], vals[4 * q + 1], vals[4 * q + 2], vals[4 * q + 3]};
      } else {
#pragma unroll
        for (int q = 0; q < 16; ++q)
          if (col + q < N) store_c(c, cdt, o + q, vals[q]);
      }
    }
  };
  out_tile(acc[0][0], 0, 0);
  out_tile(acc[0][1], 0, 1);
  out_tile(acc[1][0], 1, 0);
  out_tile(acc[1][1], 1, 1);
}

template <int FMT, bool SCALED>
int launch_gemm_w(const void* a, int64_t lda, const void* w, const void* scales, int64_t m, int64_t n, int64_t k,
                  void* c, int cdt, int64_t ldc, hipStream_t stream) {
  const int64_t tiles = ((m + kWM - 1) / kWM) * ((n + kWN - 1) / kWN);
  hipLaunchKernelGGL((gemm_w_mx<FMT, SCALED>), dim3((unsigned)tiles), dim3(512), 0, stream, (const uint8_t*)a,
                     (unsigned)(lda * 2), (const uint8_t*)w, (const uint8_t*)scales, (int)m, (int)n, (int)k, c, cdt,
                     ldc);
  return launch_status("tgm_gemm_w");
}

}  // namespace tgm

using namespace tgm;

extern "C" int tgm_gemm_w(const void* a, int a_dtype, int64_t m, int64_t lda, const void* w, int fmt, int64_t n,
                          int64_t k, const void* scales, int scale_dtype, int64_t block_size, void* c, int c_dtype,
                          int64_t ldc, void* stream) {
  clear_error();
  TGM_CHECK_ARG(a && w && c, "null operand");
  TGM_CHECK_ARG(valid_format(fmt), "unknown packed format %d", fmt);
  TGM_CHECK_ARG(m >= 0 && n >= 0 && k >= 0, "invalid gemm sizes");
  TGM_CHECK_ARG(m <= 1 || lda >= k, "lda smaller than K");
  TGM_CHECK_ARG(c_dtype == TGM_BF16 || c_dtype == TGM_F16 || c_dtype == TGM_F32, "output must be bf16, f16 or f32");
  TGM_CHECK_ARG(m <= 1 || ldc >= n, "ldc smaller than N");
  if (m == 0 || n == 0) return TGM_OK;
  if (a_dtype != TGM_BF16) TGM_UNSUPPORTED("tgm_gemm_w: activations must be bf16");
  if (fmt != TGM_FMT_FP4_E2M1 && fmt != TGM_FMT_FP6_E2M3 && fmt != TGM_FMT_FP6_E3M2)
    TGM_UNSUPPORTED("tgm_gemm_w: only FP4 / FP6 weights have a bf16-MFMA kernel");
  const bool scaled = scales != nullptr;
  if (scaled && (scale_dtype != TGM_E8M0 || block_size != 32))
    TGM_UNSUPPORTED("tgm_gemm_w: scales must be E8M0 per 32 K-elements");
  if (k == 0 || k % kWK != 0) TGM_UNSUPPORTED("tgm_gemm_w: K must be a positive multiple of %d", kWK);
  if (m > 1 && (lda * 2) % 16 != 0) TGM_UNSUPPORTED("tgm_gemm_w: activation rows must be 16-byte aligned");
  const int64_t kbw = k / 8 * (fmt == TGM_FMT_FP4_E2M1 ? 4 : 6);
  if (m >= (1ll << 31) || n >= (1ll << 31) || (m - 1) * lda * 2 + k * 2 >= (1ll << 32) || n * kbw >= (1ll << 32))
    TGM_UNSUPPORTED("tgm_gemm_w: operands must be under 4 GiB (32-bit offsets)");
  if ((uintptr_t)a % 16 || (uintptr_t)w % 16 || (scaled && (uintptr_t)scales % 4))
    TGM_UNSUPPORTED("tgm_gemm_w: operands must be 16-byte and scales 4-byte aligned");
  const hipStream_t st = (hipStream_t)stream;
  const int64_t lda_eff = m > 1 ? lda : k;
  switch (fmt * 2 + (scaled ? 1 : 0)) {
    case TGM_FMT_FP4_E2M1 * 2 + 1: return launch_gemm_w<TGM_FMT_FP4_E2M1, true>(a, lda_eff, w, scales, m, n, k, c, c_dtype, ldc, st);
    case TGM_FMT_FP4_E2M1 * 2: return launch_gemm_w<TGM_FMT_FP4_E2M1, false>(a, lda_eff, w, scales, m, n, k, c, c_dtype, ldc, st);
    case TGM_FMT_FP6_E2M3 * 2 + 1: return launch_gemm_w<TGM_FMT_FP6_E2M3, true>(a, lda_eff, w, scales, m, n, k, c, c_dtype, ldc, st);
    case TGM_FMT_FP6_E2M3 * 2: return launch_gemm_w<TGM_FMT_FP6_E2M3, false>(a, lda_eff, w, scales, m, n, k, c, c_dtype, ldc, st);
    case TGM_FMT_FP6_E3M2 * 2 + 1: return launch_gemm_w<TGM_FMT_FP6_E3M2, true>(a, lda_eff, w, scales, m, n, k, c, c_dtype, ldc, st);
    default: return launch_gemm_w<TGM_FMT_FP6_E3M2, false>(a, lda_eff, w, scales, m, n, k, c, c_dtype, ldc, st);
  }
}
