// Kernel family 2, scaled-MFMA path for FP4 / FP6 operand pairs: v_mfma_scale_f32_32x32x64_f8f6f4
// with FP6 (E2M3, E3M2) or FP4 (E2M1) codes on either side, each with E8M0 scales per 32
// K-elements or unscaled (scale byte 127 = 1.0).  tgm_gemm_mx sends FP4 x FP4 with scales on
// both sides to its own kernel (tgm_gemm_mx.hip) and every other FP4 / FP6 pair here.
//
// Replaces the reference's collective LinAlg GEMM (alexandreteles/tinygrad-dx12
// src/tinygrad_dx12/renderer/linalg.py:38-124) for two packed operands.  The reference decodes
// them to their common intermediate -- FP8 when both are unscaled and share an exact FP8 type,
// fp32 when either is scaled (codegen/decomp/dx12.py:115-138) -- and multiplies those with fp32
// accumulation (renderer/linalg.py:33-35).  Every FP4 / FP6 code times a power-of-two scale,
// and every product of two such values, is exact in fp32, and the MFMA sums them exactly for
// every pair but one: measured on gfx950 with random codes, E3M2 x E3M2 (BF6 x BF6) sums lose
// up to ~1e-4 of sum |products| (and the FP8 modes ~2e-4), while every other FP4 / FP6 pair
// matches the exact fp64 sum to fp32 rounding.  E3M2 x E3M2 is therefore not taken here
// (TGM_E_UNSUPPORTED); the caller decodes one side to bf16 and uses the weight GEMM.
//
//   C[m, n] = sum_k deq(A)[m, k] * deq(B)[n, k]      A [M, K], B [N, K], K contiguous
//
// MFMA operand layout (32x32x64): lane l supplies row l % 32 and the 32 K-elements
// [32 (l / 32), +32) of the 64-element substep, i.e. one MX block: 16 bytes of FP4 or 24 of FP6
// in the low 4 or 6 registers of the operand, and that block's E8M0 byte.
//
// Workgroup: 256 (M) x 128 (N) output tile, eight waves in 4 x 2, each 64 x 64 = 2 x 2 MFMA
// tiles.  K advances in steps of 128 elements: 64 (FP4) or 96 (FP6) bytes per row and operand,
// loaded straight into a double-buffered LDS stage (buffer_load ... lds, rows past M or N read
// zeros).  Rows are stored densely; the 16-byte columns of row r are permuted so that the 32 rows
// one fragment read touches fall in different banks (XOR with (r >> 2) & 3 for 4 columns,
// rotation by (r >> 3) & 1 for 6).  E8M0 scales arrive four steps at a time (16 bytes per row)
// into their own double buffer.
#include "tgm_mfma_common.h"

namespace tgm {

// v_mfma_scale_f32_32x32x64_f8f6f4 operand type codes (cbsz / blgp) of the FP6 / FP4 formats
constexpr int kOpE2M3 = 2, kOpE3M2 = 3, kOpE2M1 = 4;

template <int T>
struct F8F6F4 {
  static constexpr int bits = T <= kOpE3M2 ? 6 : 4;
  static constexpr int RB = 128 * bits / 8;  // bytes per row and 128-element step
  static constexpr int C = RB / 16;          // 16-byte columns per row and step
  static constexpr int L = 4 * bits;         // bytes of one lane's 32 values
};

template <int C>
__device__ __forceinline__ int col_phys(int r, int c) {
  if constexpr (C == 4) return c ^ ((r >> 2) & 3);
  else return (c + ((r >> 3) & 1)) % 6;
}
template <int C>
__device__ __forceinline__ int col_logical(int r, int pc) {
  if constexpr (C == 4) return pc ^ ((r >> 2) & 3);
  else return (pc + 6 - ((r >> 3) & 1)) % 6;
}

constexpr int kGM = 256, kGN = 128, kGK = 128;  // output tile and K step
constexpr int kGBatchSteps = 4;                 // steps per batch of E8M0 scales
constexpr int kGBatchRow = kGBatchSteps * kGK / 32;  // scale bytes of one row per batch (16)
constexpr int kGBatch = (kGM + kGN) * kGBatchRow;    // A and B scales of one batch (6 KB)

// One lane's 32 values of row r (panel at ``panel``) for block kb (0..3) of a step.
template <int T>
__device__ __forceinline__ i32x8 read_block(const unsigned char* panel, int r, int kb) {
  using O = F8F6F4<T>;
  const unsigned char* row = panel + r * O::RB;
  i32x8 v = {0, 0, 0, 0, 0, 0, 0, 0};
  if constexpr (O::bits == 4) {
    const u32x4 q = *(const u32x4*)(row + 16 * col_phys<O::C>(r, kb));
    v[0] = (int)q[0]; v[1] = (int)q[1]; v[2] = (int)q[2]; v[3] = (int)q[3];
  } else {  // 24 bytes at 24 kb: three 8-byte pieces, each inside one 16-byte column
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const int b = 24 * kb + 8 * i;
      const u32x2 q = *(const u32x2*)(row + 16 * col_phys<O::C>(r, b >> 4) + (b & 15));
      v[2 * i] = (int)q[0];
      v[2 * i + 1] = (int)q[1];
    }
  }
  return v;
}

// sa / sb may be null (unscaled operand).  lda / ldb: bytes between rows.
template <int TA, int TB>
__global__ void __launch_bounds__(512) gemm_f8f6f4(const uint8_t* __restrict__ a, unsigned lda,
                                                  const uint8_t* __restrict__ sa, const uint8_t* __restrict__ b,
                                                  unsigned ldb, const uint8_t* __restrict__ sb, int M, int N, int K,
                                                  void* __restrict__ c, int cdt, int64_t ldc) {
  using OA = F8F6F4<TA>;
  using OB = F8F6F4<TB>;
  constexpr int PA = kGM * OA::RB, PB = kGN * OB::RB;  // panel bytes of one stage
  constexpr int STAGE = PA + PB;
  constexpr int NIA = PA / 1024, NIB = PB / 1024;      // 1 KB load instructions per stage
  constexpr int QA = (NIA + 7) / 8, QB = (NIB + 7) / 8;
  __shared__ __attribute__((aligned(16))) unsigned char lds[2 * STAGE + 2 * kGBatch];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int tiles_m = (M + kGM - 1) / kGM, tiles_n = (N + kGN - 1) / kGN;
  int tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, 8, tm, tn);
  const int m0 = tm * kGM, n0 = tn * kGN;
  const int nsteps = K / kGK;
  const unsigned kblk = (unsigned)(K / 32);
  const i32x4v ra = buffer_rsrc(a, (unsigned)(M - 1) * lda + (unsigned)K * OA::bits / 8);
  const i32x4v rb = buffer_rsrc(b, (unsigned)(N - 1) * ldb + (unsigned)K * OB::bits / 8);
  const i32x4v rsa = buffer_rsrc(sa, sa ? (unsigned)M * kblk : 0u);
  const i32x4v rsb = buffer_rsrc(sb, sb ? (unsigned)N * kblk : 0u);
  const unsigned lds_base = (unsigned)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)lds;

  // Load instruction g of a panel fills LDS bytes [1024 g, +1024): lane l writes slot
  // s = 64 g + l, i.e. row s / C, physical column s % C, which holds logical column
  // col_logical(row, s % C) of that row's step chunk.  Instruction g is issued by wave g % 8.
  unsigned voa[QA], vob[QB];
#pragma unroll
  for (int q = 0; q < QA; ++q) {
    const int s = 64 * (8 * q + wave) + lane, r = s / OA::C;
    voa[q] = (unsigned)(m0 + r) * lda + 16u * (unsigned)col_logical<OA::C>(r, s % OA::C);
  }
#pragma unroll
  for (int q = 0; q < QB; ++q) {
    const int s = 64 * (8 * q + wave) + lane, r = s / OB::C;
    vob[q] = (unsigned)(n0 + r) * ldb + 16u * (unsigned)col_logical<OB::C>(r, s % OB::C);
  }
  auto dma_step = [&](int s, int buf) __attribute__((always_inline)) {
    const unsigned st = lds_base + (unsigned)(buf * STAGE);
#pragma unroll
    for (int q = 0; q < QA; ++q)
      if (8 * q + wave < NIA) lds_dma16(ra, st + (unsigned)(8 * q + wave) * 1024u, voa[q] + (unsigned)(s * OA::RB));
#pragma unroll
    for (int q = 0; q < QB; ++q)
      if (8 * q + wave < NIB)
        lds_dma16(rb, st + (unsigned)(PA + (8 * q + wave) * 1024), vob[q] + (unsigned)(s * OB::RB));
  };
  // Scale batch b (steps 4b .. 4b + 3): the 16 E8M0 bytes of tile row r land at byte 16 r of
  // buffer b & 1 (A rows 0..255, then B rows), one lane per row: waves 0-3 load A, 4-5 load B.
  // Bytes past a row's end (the last batch when K is not a multiple of 512) belong to steps that
  // do not exist.
  auto issue_batch = [&](int bt) __attribute__((always_inline)) {
    const unsigned dst = lds_base + (unsigned)(2 * STAGE + (bt & 1) * kGBatch + wave * 1024);
    const unsigned boff = (unsigned)bt * (unsigned)kGBatchRow;
    if (wave < 4 && sa) lds_dma16(rsa, dst, (unsigned)(m0 + 64 * wave + lane) * kblk + boff);
    else if (wave >= 4 && wave < 6 && sb) lds_dma16(rsb, dst, (unsigned)(n0 + 64 * (wave - 4) + lane) * kblk + boff);
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

  const int half = lane >> 5;
  const int ar = wm * 64 + (lane & 31), br = wn * 64 + (lane & 31);  // + 32 t
  const int s1 = nsteps > 1 ? 1 : 0;
  issue_batch(0);
  dma_step(0, 0);
  dma_step(s1, 1);
  wait_lds_dma();
  __syncthreads();
  for (int s = 0; s < nsteps; ++s) {
    const int cur = s & 1;
    const unsigned char* pa = lds + cur * STAGE;
    const unsigned char* pb = pa + PA;
    const unsigned* bat = (const unsigned*)(lds + 2 * STAGE + ((s / kGBatchSteps) & 1) * kGBatch) + (s % kGBatchSteps);
    unsigned sca[2], scb[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      sca[t] = sa ? bat[4 * (ar + 32 * t)] : 0x7F7F7F7Fu;
      scb[t] = sb ? bat[4 * (kGM + br + 32 * t)] : 0x7F7F7F7Fu;
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int kb = 2 * u + half;  // this lane's block of the step
      i32x8 fa[2], fb[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        fa[t] = read_block<TA>(pa, ar + 32 * t, kb);
        fb[t] = read_block<TB>(pb, br + 32 * t, kb);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
              fa[i], fb[j], acc[i][j], TA, TB, 0, (int)(sca[i] >> (8 * kb)), 0, (int)(scb[j] >> (8 * kb)));
    }
    wait_lds_dma();   // this wave's loads of step s + 1 (and of a scale batch issued at step s - 1)
    __syncthreads();  // every wave is done with buffer cur; step s + 1 is complete in the other
    dma_step(s + 2 < nsteps ? s + 2 : nsteps - 1, cur);
    // batch b + 1 replaces batch b - 1, whose last reads (step 4b - 1) are behind this barrier
    if (s % kGBatchSteps == 0) issue_batch(s / kGBatchSteps + 1);
  }
  wait_lds_dma();
  __syncthreads();  // the epilogue reuses the LDS
  float* ep = (float*)lds + wave * 32 * 36;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
      store_tile32(acc[i][j], ep, lane, m0 + wm * 64 + i * 32, n0 + wn * 64 + j * 32, M, N, c, cdt, ldc);
}

// Operand type code of a packed format; -1 when the MFMA has none.
int f8f6f4_code_of_format(int fmt) {
  switch (fmt) {
    case TGM_FMT_FP4_E2M1: return kOpE2M1;
    case TGM_FMT_FP6_E2M3: return kOpE2M3;
    case TGM_FMT_FP6_E3M2: return kOpE3M2;
    default: return -1;
  }
}

template <int TA, int TB>
static void launch_f8f6f4_t(hipStream_t s, const void* a, unsigned lda, const void* sa, const void* b, unsigned ldb,
                            const void* sb, int m, int n, int k, void* c, int cdt, int64_t ldc) {
  const int64_t tiles = ((int64_t)(m + kGM - 1) / kGM) * ((n + kGN - 1) / kGN);
  hipLaunchKernelGGL((gemm_f8f6f4<TA, TB>), dim3((unsigned)tiles), dim3(512), 0, s, (const uint8_t*)a, lda,
                     (const uint8_t*)sa, (const uint8_t*)b, ldb, (const uint8_t*)sb, m, n, k, c, cdt, ldc);
}

// Checks, then the launch.  ta / tb are operand type codes.
int launch_f8f6f4(hipStream_t s, int ta, const void* a, int64_t lda, const void* sa, int64_t m, int tb,
                  const void* b, int64_t ldb, const void* sb, int64_t n, int64_t k, void* c, int cdt, int64_t ldc,
                  const char* who) {
  if (ta == kOpE3M2 && tb == kOpE3M2)
    TGM_UNSUPPORTED("%s: the scaled MFMA does not sum E3M2 x E3M2 products exactly; decode one operand", who);
  if (k == 0 || k % kGK != 0) TGM_UNSUPPORTED("%s: K must be a positive multiple of %d", who, kGK);
  if (m >= (1ll << 31) || n >= (1ll << 31) || (m - 1) * lda + k >= (1ll << 32) || (n - 1) * ldb + k >= (1ll << 32))
    TGM_UNSUPPORTED("%s: operands must be under 4 GiB (32-bit offsets)", who);
  if ((uintptr_t)a % 16 || (uintptr_t)b % 16 || lda % 16 || ldb % 16)
    TGM_UNSUPPORTED("%s: operand rows must be 16-byte aligned", who);
  if ((sa && (uintptr_t)sa % 4) || (sb && (uintptr_t)sb % 4)) TGM_UNSUPPORTED("%s: scales must be 4-byte aligned", who);
  const unsigned ua = (unsigned)lda, ub = (unsigned)ldb;
  const int im = (int)m, in = (int)n, ik = (int)k;
#define TGM_F8F6F4(A, B)                                                              \
  if (ta == A && tb == B) {                                                           \
    launch_f8f6f4_t<A, B>(s, a, ua, sa, b, ub, sb, im, in, ik, c, cdt, ldc);          \
    return launch_status(who);                                                        \
  }
  TGM_F8F6F4(kOpE2M1, kOpE2M1) TGM_F8F6F4(kOpE2M1, kOpE2M3) TGM_F8F6F4(kOpE2M1, kOpE3M2)
  TGM_F8F6F4(kOpE2M3, kOpE2M1) TGM_F8F6F4(kOpE2M3, kOpE2M3) TGM_F8F6F4(kOpE2M3, kOpE3M2)
  TGM_F8F6F4(kOpE3M2, kOpE2M1) TGM_F8F6F4(kOpE3M2, kOpE2M3)
#undef TGM_F8F6F4
  TGM_UNSUPPORTED("%s: no scaled-MFMA kernel for operand types %d x %d", who, ta, tb);
}

}  // namespace tgm
