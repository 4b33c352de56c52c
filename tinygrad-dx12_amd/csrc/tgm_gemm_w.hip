// Kernel family 2, dequant path: packed FP4 / FP6 weights x bf16 activations on bf16 MFMA,
// and INT4 / UINT4 weights with per-group scales x f16 activations on f16 MFMA (gemm_w_i4).
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
#include <mutex>

#include "tgm_mfma_common.h"

namespace tgm {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
typedef __attribute__((__vector_size__(32 * sizeof(__bf16)))) __bf16 bf16x32;
typedef __attribute__((__vector_size__(6 * sizeof(int)))) int i32x6;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8;
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

constexpr int kWM = 128, kWN = 256, kWK = 128;  // output tile and K step
constexpr int kAPanel = kWM * kWK * 2;           // 32 KB of bf16 A per stage
constexpr int kWPanelMax = kWN * 96;             // 24 KB of packed W (FP6) per stage
constexpr int kWStage = kAPanel + kWPanelMax;
constexpr int kWBatchSteps = 4;                  // steps per batch of E8M0 scales
constexpr int kWBatch = kWN * 4 * kWBatchSteps;  // one E8M0 dword per W row and step (4 KB)
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

template <int FMT, bool SCALED, bool SWIGLU = false>
__global__ void __launch_bounds__(512) gemm_w_mx(const uint8_t* __restrict__ a, unsigned lda_bytes,
                                                 const uint8_t* __restrict__ w, const uint8_t* __restrict__ sw,
                                                 int M, int N, int K, void* __restrict__ c, int cdt, int64_t ldc,
                                                 int kps, float* __restrict__ part) {
  using T = GemmWTraits<FMT>;
  constexpr int FA = 2, FB = 2;
  __shared__ __attribute__((aligned(16))) unsigned char lds[2 * kWStage + 2 * kWBatch];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  const int tiles_m = (M + kWM - 1) / kWM, tiles_n = (N + kWN - 1) / kWN;
  int tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, kWGroupM, tm, tn);
  const int m0 = tm * kWM, n0 = tn * kWN;
  // split K: blockIdx.y takes steps [s_begin, s_begin + kps) and then writes an fp32 partial tile
  const int s_begin = (int)blockIdx.y * kps;
  const int nsteps = min(kps, K / kWK - s_begin);
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
  // E8M0 scales arrive four steps at a time: batch b (local steps 4b .. 4b + 3) puts the 16 scale
  // bytes of W row r at byte 16 r of scale buffer b & 1, one 16-byte lane per row, waves 0..3
  // loading 64 rows each.  A row's scale bytes of one step are one dword: fetching them step by
  // step costs a cache-line access per row and step, as many as the A panel's.  Bytes past a
  // row's end (the last batch of a K range) belong to steps that do not exist.
  const unsigned vos = (unsigned)(n0 + 64 * (wave & 3) + lane) * kblk + (unsigned)s_begin * 4u;
  auto issue_batch = [&](int b) __attribute__((always_inline)) {
    if (SCALED && wave < 4)
      lds_dma16(rs, lds_base + (unsigned)(2 * kWStage + (b & 1) * kWBatch + wave * 1024), vos + (unsigned)b * 16u);
  };

  auto dma_step = [&](int s, int buf) __attribute__((always_inline)) {
    const unsigned st = lds_base + (unsigned)(buf * kWStage);
    const unsigned sk = (unsigned)(s_begin + s);
#pragma unroll
    for (int q = 0; q < 4; ++q) lds_dma16(ra, st + (unsigned)(4 * wave + q) * 1024u, voa[q] + sk * 256u);
#pragma unroll
    for (int q = 0; q < NWL; ++q)
      if (NWL * wave + q < T::kPanelLoads)
        lds_dma16(rw, st + kAPanel + (unsigned)(NWL * wave + q) * 1024u, vow[q] + sk * (unsigned)T::kRow);
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
  auto read_decode_b = [&](int buf, int s) __attribute__((always_inline)) {
    const unsigned char* pw = lds + buf * kWStage + kAPanel;
    const unsigned* ps = (const unsigned*)(lds + 2 * kWStage + ((s / kWBatchSteps) & 1) * kWBatch) + (s % kWBatchSteps);
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
      const unsigned sbits = SCALED ? ps[4 * row] >> (16 * half) : 0x7F7Fu;  // blocks 2 h, 2 h + 1
      decode64<FMT>(raw, sbits, bfr[t]);
    }
  };

  f32x16 acc[FA][FB];
#pragma unroll
  for (int i = 0; i < FA; ++i)
#pragma unroll
    for (int j = 0; j < FB; ++j) acc[i][j] = f32x16{};

  const int s1 = nsteps > 1 ? 1 : 0;
  issue_batch(0);
  dma_step(0, 0);
  dma_step(s1, 1);
  wait_lds_dma();
  __syncthreads();
  for (int s = 0; s < nsteps; ++s) {
    const int cur = s & 1;
    const int s2 = s + 2 < nsteps ? s + 2 : nsteps - 1;
    read_decode_b(cur, s);
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
    wait_lds_dma();  // this wave's loads of step s + 1 (and a scale batch issued at step s - 1)
    __syncthreads();  // every wave is done with this buffer; step s + 1 is complete in the other
    dma_step(s2, cur);
    // batch b + 1 replaces batch b - 1, last read at step 4b - 1; complete after the next wait
    if (s % kWBatchSteps == 0) issue_batch(s / kWBatchSteps + 1);
  }
  wait_lds_dma();
  __syncthreads();  // the epilogue reuses the LDS

  // Epilogue: each 32 x 32 tile through the wave's LDS block (store_tile32).
  float* ep = (float*)lds + wave * 32 * 36;
#pragma unroll
  for (int i = 0; i < FA; ++i)
#pragma unroll
    for (int j = 0; j < FB; ++j)
      if (part)
        store_tile32(acc[i][j], ep, lane, m0 + wm * 64 + i * 32, n0 + wn * 64 + j * 32, M, N,
                     part + (int64_t)blockIdx.y * M * N, TGM_F32, N);
      else if constexpr (SWIGLU)
        store_tile32_swiglu(acc[i][j], ep, lane, m0 + wm * 64 + i * 32, n0 + wn * 64 + j * 32, M, N, c, cdt, ldc);
      else
        store_tile32(acc[i][j], ep, lane, m0 + wm * 64 + i * 32, n0 + wn * 64 + j * 32, M, N, c, cdt, ldc);
}

// ---------------------------------------------------------------------------------------------
// Persistent form for K a multiple of 512 and at least one round of 128 x 256 tiles
// (gemm_w_stream): the same tile, waves, panels, K order and decode as gemm_w_mx, on the step
// pipeline of the persistent FP4 GEMM (tgm_gemm_mx.hip) --
//
//  * one workgroup per CU (G, a multiple of 8) walks tiles blockIdx.x, blockIdx.x + G, ... as one
//    stream of K steps; the loads of the next tile's first steps are issued during the current
//    tile's last, so no tile waits for its operands and no workgroup is launched per tile;
//  * a step is eight substeps of 16 K (MFMA j takes K [64 h + 8 j, + 8) for lane half h); after
//    each MFMA the wave issues an even share of the work placed on its substep, fenced by
//    scheduling barriers: the next substep's A fragments, the panel loads (the rest of step
//    s + 1's in substeps 0 and 1, the first of step s + 2's in substep 7) and the weight decode;
//  * the step barrier sits before substep 7: there the next step's A fragments, packed weights
//    and E8M0 words are read from the other buffer, and the first of the two MX blocks each lane
//    owns per weight fragment is decoded; the second block is decoded under the next step's
//    first substep.  So no step begins with an LDS round trip and a full decode;
//  * at a tile's end each wave rounds its 32 x 32 tiles to 16 bits through its own 2 KB LDS slice
//    and writes 16-byte row segments with non-temporal stores.
// Measured in one process against gemm_w_mx: config 3 (2048 x 11008 x 4096, FP6 E3M2) 156.5 against
// 171.0 us; with FP4 weights the batch-8 decoder prefill (its down projections 4096 x 4096 x 14336 on
// this kernel) came out even (15.96 against 15.81 ms).  The SwiGLU form keeps gemm_w_mx.
constexpr int kVEpi = 8 * 2048;                                    // one 2 KB epilogue slice per wave
constexpr int kVLds = 2 * kWStage + 2 * kWBatch + kVEpi;           // 136 KB
constexpr int kVKMultiple = kWK * kWBatchSteps;                     // K = 512: whole scale batches per tile

// MX block ``blk`` (0 or 1) of the 64 codes a lane owns in one step (raw: 12 dwords FP6 / 8
// dwords FP4, block 1 from dword 6 / 4) to the operands of MFMAs 4 blk .. 4 blk + 3; its E8M0
// byte is byte ``sbyte`` of ``sword`` (the shift happens here, at the decode, not where the word
// is read from LDS).
template <int FMT>
__device__ __forceinline__ void decode_block(const unsigned* raw, int blk, unsigned sword, int sbyte, bf16x8 out[4]) {
  const float s = __builtin_bit_cast(float, ((sword >> (8 * sbyte)) & 0xFFu) << 23);
  if constexpr (FMT == TGM_FMT_FP4_E2M1) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const unsigned v = raw[4 * blk + d];
      const bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, s, 0);
      const bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, s, 1);
      const bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, s, 2);
      const bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, s, 3);
      out[d] = bf16x8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
    }
  } else {
    i32x6 v;
#pragma unroll
    for (int q = 0; q < 6; ++q) v[q] = (int)raw[6 * blk + q];
    bf16x32 d;
    if constexpr (FMT == TGM_FMT_FP6_E2M3) d = __builtin_amdgcn_cvt_scalef32_pk32_bf16_fp6(v, s);
    else d = __builtin_amdgcn_cvt_scalef32_pk32_bf16_bf6(v, s);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      out[j] = bf16x8{d[8 * j], d[8 * j + 1], d[8 * j + 2], d[8 * j + 3], d[8 * j + 4], d[8 * j + 5], d[8 * j + 6],
                      d[8 * j + 7]};
  }
}

template <int FMT, bool SCALED>
__global__ void __launch_bounds__(512) gemm_w_stream(const uint8_t* __restrict__ a, unsigned lda_bytes,
                                                     const uint8_t* __restrict__ w, const uint8_t* __restrict__ sw,
                                                     int M, int N, int K, void* __restrict__ c, int cdt, int64_t ldc) {
  using T = GemmWTraits<FMT>;
  constexpr bool FP4 = FMT == TGM_FMT_FP4_E2M1;
  constexpr int R = T::kRow;            // packed weight bytes per row and step
  constexpr int FA = 2, FB = 2;
  constexpr int NPA = 4;                // A panel: 32 instructions of 4 rows, 4 per wave
  constexpr int NPW = T::kPanelLoads / 8;  // W panel: 16 (FP4) or 24 (FP6) instructions, 2 or 3 per wave
  constexpr int NP = NPA + NPW;         // load pieces per wave and step
  constexpr int NP0 = NP / 2;           // pieces of step s + 2 issued in step s's last substep
  constexpr int NRB = FP4 ? 1 : 2;      // LDS reads of one MX block of a weight fragment
  __shared__ __attribute__((aligned(16))) unsigned char lds[kVLds];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  const int tiles_m = (M + kWM - 1) / kWM, tiles_n = (N + kWN - 1) / kWN;
  const int ntiles = tiles_m * tiles_n;
  const int G = gridDim.x;
  const int my_tiles = (ntiles - (int)blockIdx.x + G - 1) / G;  // >= 1 (the host launches G <= ntiles)
  const int nsteps = K / kWK;                                    // a multiple of kWBatchSteps
  const int total = my_tiles * nsteps;
  const unsigned kbw = (unsigned)K / 8u * (FP4 ? 4u : 6u);       // packed bytes per weight row
  const unsigned kblk = (unsigned)K / 32u;
  const i32x4v ra = buffer_rsrc(a, (unsigned)(M - 1) * lda_bytes + (unsigned)K * 2u);
  const i32x4v rw = buffer_rsrc(w, (unsigned)N * kbw);
  const i32x4v rs = buffer_rsrc(sw, SCALED ? (unsigned)N * kblk : 0u);
  const unsigned lds_base = (unsigned)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)lds;

  // Per-lane load offsets within a tile's step (the uniform tile and step parts come from step_off).
  // A: instruction 4 wave + q covers rows 16 wave + 4 q .. + 3; lane l fills slot l % 16 of row
  // 16 wave + 4 q + l / 16, which holds logical 16-byte column (l % 16) ^ (row % 16).
  unsigned voa[NPA];
#pragma unroll
  for (int q = 0; q < NPA; ++q) {
    const int row = 16 * wave + 4 * q + (lane >> 4);
    voa[q] = (unsigned)row * lda_bytes + (unsigned)(((lane & 15) ^ (row & 15)) * 16);
  }
  // W: instruction wave + 8 q fills bytes [1024 i, + 1024) of the panel: FP6 rows are 96 bytes
  // stored densely; FP4 rows are 64 bytes with 16-byte chunks swizzled by (row / 4) % 4.
  unsigned vow[NPW];
#pragma unroll
  for (int q = 0; q < NPW; ++q) {
    const int i = wave + 8 * q;
    if constexpr (FP4) {
      const int row = 16 * i + (lane >> 2);
      vow[q] = (unsigned)row * kbw + (unsigned)(((lane & 3) ^ ((row >> 2) & 3)) * 16);
    } else {
      const int f = 1024 * i + 16 * lane;
      vow[q] = (unsigned)(f / 96) * kbw + (unsigned)(f % 96);
    }
  }
  struct Tiles {
    int base, mc, nc, mn, nn;  // first stream step of the tile; origins of this tile and the next
  } tl;
  auto tile_origin = [&](int t, int& m0, int& n0) __attribute__((always_inline)) {
    int tm, tn;
    tile_of((int)blockIdx.x + t * G, tiles_m, tiles_n, kWGroupM, tm, tn);
    m0 = tm * kWM;
    n0 = tn * kWN;
  };
  auto set_tile = [&](int t) __attribute__((always_inline)) {
    tl.base = t * nsteps;
    tile_origin(t, tl.mc, tl.nc);
    tile_origin(t + 1 < my_tiles ? t + 1 : t, tl.mn, tl.nn);
    tl.mc = __builtin_amdgcn_readfirstlane(tl.mc);
    tl.nc = __builtin_amdgcn_readfirstlane(tl.nc);
    tl.mn = __builtin_amdgcn_readfirstlane(tl.mn);
    tl.nn = __builtin_amdgcn_readfirstlane(tl.nn);
  };
  struct StepAt {
    int m0, n0, st;
  };
  // (tile origins, step within the tile) of stream step gs, clamped to the stream; gs lies in the
  // current tile or the next
  auto step_at = [&](int gs) __attribute__((always_inline)) {
    gs = gs < total ? gs : total - 1;
    const int local = gs - tl.base;
    return local < nsteps ? StepAt{tl.mc, tl.nc, local} : StepAt{tl.mn, tl.nn, local - nsteps};
  };
  struct StepOff {
    unsigned a, w;
  };
  auto step_off = [&](int gs) __attribute__((always_inline)) {
    const StepAt at = step_at(gs);
    return StepOff{
        (unsigned)__builtin_amdgcn_readfirstlane((int)((unsigned)at.m0 * lda_bytes + (unsigned)(at.st * kWK * 2))),
        (unsigned)__builtin_amdgcn_readfirstlane((int)((unsigned)at.n0 * kbw + (unsigned)(at.st * R)))};
  };
  auto dma_piece = [&](const StepOff& o, int buf, int p) __attribute__((always_inline)) {
    const unsigned st = lds_base + (unsigned)(buf * kWStage);
    if (p < NPA) lds_dma16(ra, st + (unsigned)(4 * wave + p) * 1024u, voa[p < NPA ? p : 0] + o.a);
    else {
      const int q = p - NPA;
      lds_dma16(rw, st + (unsigned)kAPanel + (unsigned)(wave + 8 * q) * 1024u, vow[q < NPW ? q : 0] + o.w);
    }
  };
  auto dma_pieces = [&](int gs, int buf, int p0, int p1) __attribute__((always_inline)) {
    const StepOff o = step_off(gs);
#pragma unroll
    for (int p = 0; p < NP; ++p)
      if (p >= p0 && p < p1) dma_piece(o, buf, p);
  };
  // E8M0 scales arrive four steps at a time: batch gb of the stream (steps 4 gb .. 4 gb + 3, one
  // tile) puts the 16 bytes of W row r at byte 16 r of scale buffer gb & 1; waves 0..3 load 64
  // rows each.
  auto issue_batch = [&](int gb) __attribute__((always_inline)) {
    if (SCALED && wave < 4) {
      const int gs = gb * kWBatchSteps < total ? gb * kWBatchSteps : total - kWBatchSteps;
      const StepAt at = step_at(gs);
      lds_dma16(rs, lds_base + (unsigned)(2 * kWStage + (gb & 1) * kWBatch + wave * 1024),
                (unsigned)(at.n0 + 64 * wave + lane) * kblk + (unsigned)at.st * 4u);
    }
  };

  f32x16 acc[FA][FB];
#pragma unroll
  for (int i = 0; i < FA; ++i)
#pragma unroll
    for (int j = 0; j < FB; ++j) acc[i][j] = f32x16{};

  const int half = lane >> 5;
  const int a_row = (wm * 64 + (lane & 31)) * 256;  // + 32 t rows
  const int w_row = wn * 64 + (lane & 31);          // + 32 t
  bf16x8 fa[2][FA];                                 // A fragments of substeps j (slot j & 1)
  bf16x8 wd[FB][8];                                 // decoded weights of the step (MFMA j: wd[t][j])
  unsigned raw[FB][FP4 ? 8 : 12];                  // packed codes of the step's weight fragments
  unsigned sword[FB];                               // E8M0 word of the step (blocks 2 h, 2 h + 1: bytes 2 h, 2 h + 1)
  auto read_a = [&](int buf, int j, int t) __attribute__((always_inline)) {
    const int col = (8 * half + j) ^ (lane & 15);
    fa[j & 1][t] = *(const bf16x8*)(lds + buf * kWStage + a_row + t * 32 * 256 + col * 16);
  };
  // read q (< NRB) of MX block blk of weight fragment t: FP4 one 16-byte chunk; FP6 the block's 24
  // bytes as 16 + 8 (block 0) or 8 + 16 (block 1) at 8-byte aligned offsets of the lane's 48
  auto read_raw = [&](int buf, int t, int blk, int q) __attribute__((always_inline)) {
    const unsigned char* pw = lds + buf * kWStage + kAPanel;
    const int row = w_row + 32 * t;
    if constexpr (FP4) {
      const u32x4 v = *(const u32x4*)(pw + row * 64 + ((2 * half + blk) ^ ((row >> 2) & 3)) * 16);
#pragma unroll
      for (int e = 0; e < 4; ++e) raw[t][4 * blk + e] = v[e];
    } else {
      const unsigned char* p = pw + row * 96 + 48 * half + 24 * blk;
      if ((blk == 0) == (q == 0)) {  // the 16-byte piece: block 0 at +0, block 1 at +8
        const u32x4 v = *(const u32x4*)(p + (blk ? 8 : 0));
#pragma unroll
        for (int e = 0; e < 4; ++e) raw[t][6 * blk + (blk ? 2 : 0) + e] = v[e];
      } else {                       // the 8-byte piece: block 0 at +16, block 1 at +0
        const u32x2 v = *(const u32x2*)(p + (blk ? 0 : 16));
#pragma unroll
        for (int e = 0; e < 2; ++e) raw[t][6 * blk + (blk ? 0 : 4) + e] = v[e];
      }
    }
  };
  auto read_scale = [&](int gs, int t) __attribute__((always_inline)) {  // scales of stream step gs
    if constexpr (SCALED) {
      const unsigned* ps = (const unsigned*)(lds + 2 * kWStage + ((gs / kWBatchSteps) & 1) * kWBatch);
      sword[t] = ps[4 * (w_row + 32 * t) + gs % kWBatchSteps];
    } else {
      sword[t] = 0x7F7F7F7Fu;  // 2^0
    }
  };
  auto decode = [&](int t, int blk) __attribute__((always_inline)) {
    decode_block<FMT>(raw[t], blk, sword[t], 2 * half + blk, &wd[t][4 * blk]);
  };
  auto mfmas = [&](int j, auto&& hook) __attribute__((always_inline)) {
#pragma unroll
    for (int ta = 0; ta < FA; ++ta)
#pragma unroll
      for (int tb = 0; tb < FB; ++tb) {
        acc[ta][tb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[j & 1][ta], wd[tb][j], acc[ta][tb], 0, 0, 0);
        hook(ta * FB + tb);
      }
  };
  // Items of a substep, spread over its FA * FB MFMAs in order: it < n_items.
  constexpr int kMaxItems = FA + 2 * FB + FB * NRB + NP;
  auto run_items = [&](int j, int n_items, auto&& item) __attribute__((always_inline)) {
    mfmas(j, [&](int idx) __attribute__((always_inline)) {
#pragma unroll
      for (int it = 0; it < kMaxItems; ++it) {
        if (it < n_items && it * FA * FB / n_items == idx) {
          __builtin_amdgcn_sched_barrier(0);
          item(it);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    });
  };
  // Step gs from buffer cur (fa[0] and wd[.][0..3] hold substep 0's operands on entry, raw and sword
  // the step's block-0 codes and E8M0 words):
  //   j = 0: A of j = 1; block 1 of the packed weights; pieces [NP0, NP1) of step gs + 1
  //   j = 1: A of j = 2; the remaining pieces of step gs + 1
  //   j = 2: A of j = 3; decode block 1 (MFMAs 4 .. 7)
  //   j = 3: A of j = 4; the E8M0 words of step gs + 1.  Their batch is complete (a batch is issued
  //          four steps ahead of its first step and waited for by the step after that), and the batch
  //          that overwrites a buffer is issued only after the barrier of the step whose words it
  //          last held were read two steps before, so the reads need no barrier of their own
  //   j = 4 .. 6: A of j + 1
  //   wait for this wave's loads of step gs + 1, barrier
  //   j = 7: A of step gs + 1's j = 0 and block 0 of its packed weights (other buffer); pieces
  //          [0, NP0) of step gs + 2 (into this buffer); decode block 0
  constexpr int NP1 = NP0 + (NP - NP0 + 1) / 2;
  auto step = [&](int gs, int cur, bool batch) __attribute__((always_inline)) {
    const StepOff o1 = step_off(gs + 1), o2 = step_off(gs + 2);
    run_items(0, FA + FB * NRB + (NP1 - NP0), [&](int it) __attribute__((always_inline)) {
      if (it < FA) read_a(cur, 1, it);
      else if (it < FA + FB * NRB) read_raw(cur, (it - FA) / NRB, 1, (it - FA) % NRB);
      else dma_piece(o1, cur ^ 1, NP0 + it - FA - FB * NRB);
    });
    run_items(1, FA + (NP - NP1), [&](int it) __attribute__((always_inline)) {
      if (it < FA) read_a(cur, 2, it);
      else dma_piece(o1, cur ^ 1, NP1 + it - FA);
    });
    run_items(2, FA + FB, [&](int it) __attribute__((always_inline)) {
      if (it < FA) read_a(cur, 3, it);
      else decode(it - FA, 1);
    });
    run_items(3, FA + FB, [&](int it) __attribute__((always_inline)) {
      if (it < FA) read_a(cur, 4, it);
      else read_scale(gs + 1, it - FA);  // its batch is complete (see below): no barrier needed
    });
#pragma unroll
    for (int j = 4; j < 7; ++j)
      run_items(j, FA, [&](int it) __attribute__((always_inline)) { read_a(cur, j + 1, it); });
    __builtin_amdgcn_sched_barrier(0);
    wait_lds_dma();  // this wave's loads of step gs + 1 (and of a scale batch issued at step gs - 3)
    __syncthreads();
    run_items(7, FA + FB * NRB + NP0 + FB, [&](int it) __attribute__((always_inline)) {
      if (it < FA) read_a(cur ^ 1, 0, it);
      else if (it < FA + FB * NRB) read_raw(cur ^ 1, (it - FA) / NRB, 0, (it - FA) % NRB);
      else if (it < FA + FB * NRB + NP0) dma_piece(o2, cur, it - FA - FB * NRB);
      else decode(it - FA - FB * NRB - NP0, 0);
    });
    __builtin_amdgcn_sched_barrier(0);
    // Batch b + 1 goes to the buffer batch b - 1 used; its last reads (step 4 b - 1's words, in
    // step 4 b - 2) are behind this step's barrier; it is complete after step 4 b + 3's wait.
    if (batch) issue_batch(gs / kWBatchSteps + 1);
    __builtin_amdgcn_sched_barrier(0);
  };

  set_tile(0);
  issue_batch(0);
  dma_pieces(0, 0, 0, NP);
  dma_pieces(1, 1, 0, NP0);
  wait_lds_dma();
  __syncthreads();
#pragma unroll
  for (int t = 0; t < FB; ++t) {
    read_scale(0, t);
#pragma unroll
    for (int q = 0; q < NRB; ++q) read_raw(0, t, 0, q);
  }
#pragma unroll
  for (int t = 0; t < FA; ++t) read_a(0, 0, t);
#pragma unroll
  for (int t = 0; t < FB; ++t) decode(t, 0);
  __builtin_amdgcn_sched_barrier(0);

  unsigned char* ep = lds + 2 * kWStage + 2 * kWBatch + wave * 2048;  // this wave's epilogue slice
  static_assert(kWBatchSteps == 4, "the step loop is unrolled by four");
  int gs = 0;
  for (int t = 0; t < my_tiles; ++t) {
    set_tile(t);
    for (int s = 0; s < nsteps; s += kWBatchSteps, gs += kWBatchSteps) {
      step(gs, 0, true);
      step(gs + 1, 1, false);
      step(gs + 2, 0, false);
      step(gs + 3, 1, false);
    }
    // Tile t is complete (MFMA D layout: lane l holds column l % 32 and rows 8 (v / 4) + 4 (l / 32)
    // + v % 4 of each 32 x 32 tile: columns are weight rows, rows are activation rows).
    const int row0 = tl.mc + wm * 64;
    const int col0 = tl.nc + wn * 64;
#pragma unroll
    for (int i = 0; i < FA; ++i)
#pragma unroll
      for (int j = 0; j < FB; ++j) {
        if (cdt == TGM_F32) {
          const int col = col0 + 32 * j + (lane & 31);
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int row = row0 + 32 * i + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
            if (row < M && col < N) ((float*)c)[(int64_t)row * ldc + col] = acc[i][j][v];
          }
        } else {
          unsigned short* e16 = (unsigned short*)ep;  // 32 rows x 32 columns
#pragma unroll
          for (int v = 0; v < 16; v += 2) {
            const float x0 = acc[i][j][v], x1 = acc[i][j][v + 1];
            const unsigned h = cdt == TGM_BF16 ? bf16x2_bits(x0, x1)
                                               : __builtin_bit_cast(unsigned short, (_Float16)x0) |
                                                     ((unsigned)__builtin_bit_cast(unsigned short, (_Float16)x1) << 16);
            const int r = 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
            e16[r * 32 + (lane & 31)] = (unsigned short)h;
            e16[(r + 1) * 32 + (lane & 31)] = (unsigned short)(h >> 16);
          }
          __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
          __builtin_amdgcn_wave_barrier();
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
          for (int q = 0; q < 2; ++q) {  // lane l: row l / 4 + 16 q, columns 8 (l % 4) .. + 8
            const int r = (lane >> 2) + 16 * q, cc = 8 * (lane & 3);
            const int row = row0 + 32 * i + r, col = col0 + 32 * j + cc;
            uint16_t* out = (uint16_t*)c + (int64_t)row * ldc + col;
            if (row < M) {
              if (col + 7 < N && ((uintptr_t)out & 15) == 0) {
                __builtin_nontemporal_store(*(const u32x4*)(e16 + r * 32 + cc), (u32x4*)out);
              } else {
#pragma unroll 1
                for (int e = 0; e < 8 && col + e < N; ++e) out[e] = e16[r * 32 + cc + e];
              }
            }
          }
          __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
          __builtin_amdgcn_wave_barrier();
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
        acc[i][j] = f32x16{};
      }
  }
  wait_lds_dma();
}

// Sum of the split-K partial products [splits][M][N] (fp32) in split order, rounded once to
// C; 4 consecutive elements of a row per thread and pass (N % 4 == 0).
__global__ void __launch_bounds__(256) gemm_split_reduce(const float* __restrict__ part, int splits, int64_t M,
                                                         int64_t N, void* __restrict__ c, int cdt, int64_t ldc) {
  const int64_t total = M * N;
  for (int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4; i < total; i += (int64_t)gridDim.x * 256 * 4) {
    f32x4 acc = *(const f32x4*)(part + i);
    for (int z = 1; z < splits; ++z) {
      const f32x4 v = *(const f32x4*)(part + (int64_t)z * total + i);
      acc[0] += v[0];
      acc[1] += v[1];
      acc[2] += v[2];
      acc[3] += v[3];
    }
    const int64_t r = i / N, col = i - r * N;
#pragma unroll
    for (int e = 0; e < 4; ++e) store_c(c, cdt, r * ldc + col + e, acc[e]);
  }
}

// ---- INT4 / UINT4 weights x f16 activations, per-group scales (f16, bf16 or f32).
//
// The reference decodes int4 as (p ^ 8) - 8 and uint4 as p (dx12.py:93-94), multiplies each
// value by its group's scale in fp32 (dx12.py:101-106) and multiplies the fp32 intermediate.
// Here the codes become exact f16 values in registers (nibble n -- n ^ 8 for int4 -- goes
// under the f16 byte 0x64, i.e. 1024 + n, and a packed f16 subtraction removes 1024 or 1032),
// f16 MFMA sums code * activation products of one scale group in fp32, and the group's sum
// is multiplied by the fp32 scale of its weight row and added to the accumulator.  The
// products are the reference's; the summation order differs.
//
// Same tile, waves, A panel and W panel (64-byte rows per 128-element step, the FP4 layout)
// as gemm_w_mx, but MFMA j of a step takes K [16 j + 8 h, + 8) for lane half h (the natural
// order), so that one MFMA never spans two scale groups of 32 or 64.  A lane's codes for
// MFMA j are dword 2 j + h of its weight row: two ds_read2_b32 per 16-byte chunk.  Scales
// are read per step straight from global memory (2 rows x 128 / G values per lane), issued
// one step ahead.
template <bool SIGNED>
__device__ __forceinline__ f16x8 decode_i4x8(unsigned v) {
  if (SIGNED) v ^= 0x88888888u;
  const unsigned lo = v & 0x0F0F0F0Fu, hi = (v >> 4) & 0x0F0F0F0Fu;
  const unsigned x01 = __builtin_amdgcn_perm(hi, lo, 0x05010400u);  // n0 n1 n2 n3 (one per byte)
  const unsigned x23 = __builtin_amdgcn_perm(hi, lo, 0x07030602u);  // n4 n5 n6 n7
  const half2v bias = SIGNED ? half2v{(_Float16)1032.0f, (_Float16)1032.0f} : half2v{(_Float16)1024.0f, (_Float16)1024.0f};
  const half2v p0 = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, x01, 0x04010400u)) - bias;
  const half2v p1 = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, x01, 0x04030402u)) - bias;
  const half2v p2 = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, x23, 0x04010400u)) - bias;
  const half2v p3 = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, x23, 0x04030402u)) - bias;
  return f16x8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

template <int SDT>
__device__ __forceinline__ float scale_value(const void* p, int64_t i) {
  if constexpr (SDT == TGM_F16) return (float)((const _Float16*)p)[i];
  else if constexpr (SDT == TGM_BF16) return __builtin_bit_cast(float, (unsigned)((const uint16_t*)p)[i] << 16);
  else return ((const float*)p)[i];
}

// G: scale group (32, 64 or 128 K-elements; 0 = unscaled), SDT: scale dtype.
template <int G, int SDT, bool SIGNED>
__global__ void __launch_bounds__(512) gemm_w_i4(const uint8_t* __restrict__ a, unsigned lda_bytes,
                                                 const uint8_t* __restrict__ w, const void* __restrict__ sw,
                                                 int M, int N, int K, void* __restrict__ c, int cdt, int64_t ldc,
                                                 int kps, float* __restrict__ part) {
  constexpr int FA = 2, FB = 2, kRow = 64, kPanelLoads = kWN * kRow / 1024, NWL = kPanelLoads / 8;
  constexpr int GS = G ? kWK / G : 1;  // scale groups per step
  __shared__ __attribute__((aligned(16))) unsigned char lds[2 * (kAPanel + kWN * kRow)];
  constexpr int kStage = kAPanel + kWN * kRow;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  const int tiles_m = (M + kWM - 1) / kWM, tiles_n = (N + kWN - 1) / kWN;
  int tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, kWGroupM, tm, tn);
  const int m0 = tm * kWM, n0 = tn * kWN;
  const int s_begin = (int)blockIdx.y * kps;  // split K, as in gemm_w_mx
  const int nsteps = min(kps, K / kWK - s_begin);
  const unsigned kbw = (unsigned)K / 2u;
  const i32x4v ra = buffer_rsrc(a, (unsigned)(M - 1) * lda_bytes + (unsigned)K * 2u);
  const i32x4v rw = buffer_rsrc(w, (unsigned)N * kbw);
  const unsigned lds_base = (unsigned)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)lds;
  // A: as gemm_w_mx (row 4 i + l / 16, logical 16-byte column (l % 16) ^ (row % 16)).
  unsigned voa[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int row = 4 * (4 * wave + q) + (lane >> 4);
    voa[q] = (unsigned)(m0 + row) * lda_bytes + (unsigned)((lane & 15) ^ (row & 15)) * 16u;
  }
  // W: 64-byte rows, 16-byte chunk (l % 4) ^ ((row / 4) % 4).
  unsigned vow[NWL];
#pragma unroll
  for (int q = 0; q < NWL; ++q) {
    const int row = 16 * (NWL * wave + q) + (lane >> 2);
    vow[q] = (unsigned)(n0 + row) * kbw + (unsigned)((lane & 3) ^ ((row >> 2) & 3)) * 16u;
  }
  auto dma_step = [&](int s, int buf) __attribute__((always_inline)) {
    const unsigned st = lds_base + (unsigned)(buf * kStage);
    const unsigned sk = (unsigned)(s_begin + s);
#pragma unroll
    for (int q = 0; q < 4; ++q) lds_dma16(ra, st + (unsigned)(4 * wave + q) * 1024u, voa[q] + sk * 256u);
#pragma unroll
    for (int q = 0; q < NWL; ++q)
      lds_dma16(rw, st + kAPanel + (unsigned)(NWL * wave + q) * 1024u, vow[q] + sk * (unsigned)kRow);
  };
  const int half = lane >> 5;
  const int a_row = wm * 64 + (lane & 31);
  const int b_row = wn * 64 + (lane & 31);
  // Scales of this lane's two weight rows (clamped below N; those columns are not stored).
  const int64_t ngroups = G ? K / G : 0;
  int64_t srow[FB];
#pragma unroll
  for (int t = 0; t < FB; ++t) {
    const int n = n0 + b_row + 32 * t;
    srow[t] = (int64_t)(n < N ? n : N - 1) * ngroups;
  }
  float sc[FB][GS], sn[FB][GS];
  auto load_scales = [&](int s, float (&dst)[FB][GS]) __attribute__((always_inline)) {
    if constexpr (G != 0) {
#pragma unroll
      for (int t = 0; t < FB; ++t)
#pragma unroll
        for (int g = 0; g < GS; ++g) dst[t][g] = scale_value<SDT>(sw, srow[t] + (int64_t)(s_begin + s) * GS + g);
    }
  };
  f32x16 acc[FA][FB];
#pragma unroll
  for (int i = 0; i < FA; ++i)
#pragma unroll
    for (int j = 0; j < FB; ++j) acc[i][j] = f32x16{};

  const int s1 = nsteps > 1 ? 1 : 0;
  load_scales(0, sc);
  dma_step(0, 0);
  dma_step(s1, 1);
  wait_lds_dma();
  __syncthreads();
  for (int s = 0; s < nsteps; ++s) {
    const int cur = s & 1;
    const int s2 = s + 2 < nsteps ? s + 2 : nsteps - 1;
    load_scales(s + 1 < nsteps ? s + 1 : s, sn);
    const unsigned char* pa = lds + cur * kStage;
    const unsigned char* pw = pa + kAPanel;
    // codes: dwords 2 j + h of both weight rows (chunk j / 2, dword 2 (j % 2) + h)
    unsigned cw[FB][8];
#pragma unroll
    for (int t = 0; t < FB; ++t) {
      const int row = b_row + 32 * t;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const unsigned* p = (const unsigned*)(pw + row * kRow + ((q ^ ((row >> 2) & 3)) * 16) + 4 * half);
        cw[t][2 * q] = p[0];
        cw[t][2 * q + 1] = p[2];
      }
    }
    f32x16 part[FA][FB];
    f16x8 af[2][FA];
    auto read_a = [&](int j, f16x8 (&dst)[FA]) __attribute__((always_inline)) {
#pragma unroll
      for (int t = 0; t < FA; ++t) {
        const int row = a_row + 32 * t;
        dst[t] = *(const f16x8*)(pa + row * 256 + (((2 * j + half) ^ (row & 15)) * 16));
      }
    };
    read_a(0, af[0]);
    f16x8 bf[2][FB];
#pragma unroll
    for (int t = 0; t < FB; ++t) bf[0][t] = decode_i4x8<SIGNED>(cw[t][0]);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      // one MFMA group at a time: A of group j + 1 is read, and its codes decoded, while the
      // MFMAs of group j run
      __builtin_amdgcn_sched_barrier(0);
      if (j < 7) read_a(j + 1, af[(j + 1) & 1]);
      constexpr int JPG = G ? G / 16 : 8;  // MFMAs per scale group
#pragma unroll
      for (int ta = 0; ta < FA; ++ta)
#pragma unroll
        for (int tb = 0; tb < FB; ++tb) {
          if constexpr (G == 0) {
            acc[ta][tb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[j & 1][ta], bf[j & 1][tb], acc[ta][tb], 0, 0, 0);
          } else {
            part[ta][tb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[j & 1][ta], bf[j & 1][tb],
                                                                   j % JPG ? part[ta][tb] : f32x16{}, 0, 0, 0);
            if (j % JPG == JPG - 1) {
              const float sv = sc[tb][j / JPG];
#pragma unroll
              for (int v = 0; v < 16; ++v) acc[ta][tb][v] += part[ta][tb][v] * sv;
            }
          }
        }
      if (j < 7)
#pragma unroll
        for (int t = 0; t < FB; ++t) bf[(j + 1) & 1][t] = decode_i4x8<SIGNED>(cw[t][j + 1]);
    }
    wait_lds_dma();  // this wave's loads of step s + 1 (and its scale loads)
    if constexpr (G != 0) {
      // the scale loads are complete; make the compiler's wait for them happen here, before
      // the next step's loads are issued
#pragma unroll
      for (int t = 0; t < FB; ++t)
#pragma unroll
        for (int g = 0; g < GS; ++g) asm volatile("" : "+v"(sn[t][g]));
    }
    __syncthreads();
    dma_step(s2, cur);
#pragma unroll
    for (int t = 0; t < FB; ++t)
#pragma unroll
      for (int g = 0; g < GS; ++g) sc[t][g] = sn[t][g];
  }
  wait_lds_dma();
  __syncthreads();
  float* ep = (float*)lds + wave * 32 * 36;
#pragma unroll
  for (int i = 0; i < FA; ++i)
#pragma unroll
    for (int j = 0; j < FB; ++j)
      if (part)
        store_tile32(acc[i][j], ep, lane, m0 + wm * 64 + i * 32, n0 + wn * 64 + j * 32, M, N,
                     part + (int64_t)blockIdx.y * M * N, TGM_F32, N);
      else
        store_tile32(acc[i][j], ep, lane, m0 + wm * 64 + i * 32, n0 + wn * 64 + j * 32, M, N, c, cdt, ldc);
}

template <int G, int SDT, bool SIGNED>
int launch_gemm_w_i4(const void* a, int64_t lda, const void* w, const void* scales, int64_t m, int64_t n, int64_t k,
                     void* c, int cdt, int64_t ldc, hipStream_t stream, int splits = 1, float* part = nullptr) {
  const int64_t tiles = ((m + kWM - 1) / kWM) * ((n + kWN - 1) / kWN);
  const int kps = (int)((k / kWK + splits - 1) / splits);
  hipLaunchKernelGGL((gemm_w_i4<G, SDT, SIGNED>), dim3((unsigned)tiles, (unsigned)splits), dim3(512), 0, stream,
                     (const uint8_t*)a, (unsigned)(lda * 2), (const uint8_t*)w, scales, (int)m, (int)n, (int)k, c, cdt,
                     ldc, kps, part);
  return launch_status("tgm_gemm_w");
}

template <bool SIGNED>
int dispatch_gemm_w_i4(const void* a, int64_t lda, const void* w, const void* scales, int sdt, int64_t bs, int64_t m,
                       int64_t n, int64_t k, void* c, int cdt, int64_t ldc, hipStream_t st, int splits, float* part) {
  if (!scales) return launch_gemm_w_i4<0, TGM_F32, SIGNED>(a, lda, w, scales, m, n, k, c, cdt, ldc, st, splits, part);
#define TGM_I4_CASE(G, SDT) \
  if (bs == G && sdt == SDT)  \
    return launch_gemm_w_i4<G, SDT, SIGNED>(a, lda, w, scales, m, n, k, c, cdt, ldc, st, splits, part);
  TGM_I4_CASE(32, TGM_F16) TGM_I4_CASE(64, TGM_F16) TGM_I4_CASE(128, TGM_F16)
  TGM_I4_CASE(32, TGM_BF16) TGM_I4_CASE(64, TGM_BF16) TGM_I4_CASE(128, TGM_BF16)
  TGM_I4_CASE(32, TGM_F32) TGM_I4_CASE(64, TGM_F32) TGM_I4_CASE(128, TGM_F32)
#undef TGM_I4_CASE
  TGM_UNSUPPORTED("tgm_gemm_w: int4 scales must be f16, bf16 or f32 per 32, 64 or 128 K-elements");
}

template <int FMT, bool SCALED, bool SWIGLU = false>
int launch_gemm_w(const void* a, int64_t lda, const void* w, const void* scales, int64_t m, int64_t n, int64_t k,
                  void* c, int cdt, int64_t ldc, hipStream_t stream, int splits = 1, float* part = nullptr) {
  const int64_t tiles = ((m + kWM - 1) / kWM) * ((n + kWN - 1) / kWN);
  const int cus = stream_cu_count(stream);
  if (!SWIGLU && splits == 1 && !part && k % kVKMultiple == 0 && cus >= 8 && tiles >= cus) {
    // at least one round of tiles: persistent, one workgroup per CU (a multiple of 8 of them)
    hipLaunchKernelGGL((gemm_w_stream<FMT, SCALED>), dim3((unsigned)(cus / 8 * 8)), dim3(512), 0, stream,
                       (const uint8_t*)a, (unsigned)(lda * 2), (const uint8_t*)w, (const uint8_t*)scales, (int)m,
                       (int)n, (int)k, c, cdt, ldc);
    return launch_status(SWIGLU ? "tgm_gemm_w_swiglu" : "tgm_gemm_w");
  }
  const int kps = (int)((k / kWK + splits - 1) / splits);
  hipLaunchKernelGGL((gemm_w_mx<FMT, SCALED, SWIGLU>), dim3((unsigned)tiles, (unsigned)splits), dim3(512), 0, stream,
                     (const uint8_t*)a, (unsigned)(lda * 2), (const uint8_t*)w, (const uint8_t*)scales, (int)m, (int)n,
                     (int)k, c, cdt, ldc, kps, part);
  return launch_status(SWIGLU ? "tgm_gemm_w_swiglu" : "tgm_gemm_w");
}

}  // namespace tgm

using namespace tgm;

// tgm_gemm_w with K split over `splits` rows of workgroups (fp32 partials in `part`, summed by
// gemm_split_reduce); splits == 1 with part == nullptr is the plain product.
static int gemm_w_impl(const void* a, int a_dtype, int64_t m, int64_t lda, const void* w, int fmt, int64_t n, int64_t k,
                       const void* scales, int scale_dtype, int64_t block_size, void* c, int c_dtype, int64_t ldc,
                       int splits, float* part, void* stream) {
  TGM_CHECK_ARG(a && w && c, "null operand");
  TGM_CHECK_ARG(valid_format(fmt), "unknown packed format %d", fmt);
  TGM_CHECK_ARG(m >= 0 && n >= 0 && k >= 0, "invalid gemm sizes");
  TGM_CHECK_ARG(m <= 1 || lda >= k, "lda smaller than K");
  TGM_CHECK_ARG(c_dtype == TGM_BF16 || c_dtype == TGM_F16 || c_dtype == TGM_F32, "output must be bf16, f16 or f32");
  TGM_CHECK_ARG(m <= 1 || ldc >= n, "ldc smaller than N");
  if (m == 0 || n == 0) return TGM_OK;
  const bool int4 = fmt == TGM_FMT_INT4 || fmt == TGM_FMT_UINT4;
  if (int4 && a_dtype != TGM_F16) TGM_UNSUPPORTED("tgm_gemm_w: int4 / uint4 weights take f16 activations");
  if (!int4 && a_dtype != TGM_BF16) TGM_UNSUPPORTED("tgm_gemm_w: FP4 / FP6 weights take bf16 activations");
  const bool scaled = scales != nullptr;
  if (!int4 && scaled && (scale_dtype != TGM_E8M0 || block_size != 32))
    TGM_UNSUPPORTED("tgm_gemm_w: FP4 / FP6 scales must be E8M0 per 32 K-elements");
  if (k == 0 || k % kWK != 0) TGM_UNSUPPORTED("tgm_gemm_w: K must be a positive multiple of %d", kWK);
  if (m > 1 && (lda * 2) % 16 != 0) TGM_UNSUPPORTED("tgm_gemm_w: activation rows must be 16-byte aligned");
  const int64_t kbw = k / 8 * (fmt == TGM_FMT_FP6_E2M3 || fmt == TGM_FMT_FP6_E3M2 ? 6 : 4);
  if (m >= (1ll << 31) || n >= (1ll << 31) || (m - 1) * lda * 2 + k * 2 >= (1ll << 32) || n * kbw >= (1ll << 32))
    TGM_UNSUPPORTED("tgm_gemm_w: operands must be under 4 GiB (32-bit offsets)");
  if ((uintptr_t)a % 16 || (uintptr_t)w % 16 || (scaled && (uintptr_t)scales % 4))
    TGM_UNSUPPORTED("tgm_gemm_w: operands must be 16-byte and scales 4-byte aligned");
  const hipStream_t st = (hipStream_t)stream;
  const int64_t lda_eff = m > 1 ? lda : k;
  if (int4)
    return fmt == TGM_FMT_INT4
               ? dispatch_gemm_w_i4<true>(a, lda_eff, w, scales, scale_dtype, block_size, m, n, k, c, c_dtype, ldc, st,
                                          splits, part)
               : dispatch_gemm_w_i4<false>(a, lda_eff, w, scales, scale_dtype, block_size, m, n, k, c, c_dtype, ldc, st,
                                           splits, part);
  switch (fmt * 2 + (scaled ? 1 : 0)) {
    case TGM_FMT_FP4_E2M1 * 2 + 1: return launch_gemm_w<TGM_FMT_FP4_E2M1, true>(a, lda_eff, w, scales, m, n, k, c, c_dtype, ldc, st, splits, part);
    case TGM_FMT_FP4_E2M1 * 2: return launch_gemm_w<TGM_FMT_FP4_E2M1, false>(a, lda_eff, w, scales, m, n, k, c, c_dtype, ldc, st, splits, part);
    case TGM_FMT_FP6_E2M3 * 2 + 1: return launch_gemm_w<TGM_FMT_FP6_E2M3, true>(a, lda_eff, w, scales, m, n, k, c, c_dtype, ldc, st, splits, part);
    case TGM_FMT_FP6_E2M3 * 2: return launch_gemm_w<TGM_FMT_FP6_E2M3, false>(a, lda_eff, w, scales, m, n, k, c, c_dtype, ldc, st, splits, part);
    case TGM_FMT_FP6_E3M2 * 2 + 1: return launch_gemm_w<TGM_FMT_FP6_E3M2, true>(a, lda_eff, w, scales, m, n, k, c, c_dtype, ldc, st, splits, part);
    default: return launch_gemm_w<TGM_FMT_FP6_E3M2, false>(a, lda_eff, w, scales, m, n, k, c, c_dtype, ldc, st, splits, part);
  }
}

extern "C" int tgm_gemm_w(const void* a, int a_dtype, int64_t m, int64_t lda, const void* w, int fmt, int64_t n,
                          int64_t k, const void* scales, int scale_dtype, int64_t block_size, void* c, int c_dtype,
                          int64_t ldc, void* stream) {
  clear_error();
  return gemm_w_impl(a, a_dtype, m, lda, w, fmt, n, k, scales, scale_dtype, block_size, c, c_dtype, ldc, 1, nullptr,
                     stream);
}

extern "C" int64_t tgm_gemm_w_split_workspace(int64_t m, int64_t n, int64_t splits) {
  return splits > 1 && m > 0 && n > 0 ? splits * m * n * (int64_t)sizeof(float) : 0;
}

// Number of K groups a split-K call runs: every group holds at least one kWK step; 1 means
// the single-pass product (also when N % 4 != 0, which the reduction does not take).
static int64_t effective_splits(int64_t m, int64_t n, int64_t k, int64_t splits) {
  const int64_t steps = k > 0 && k % kWK == 0 ? k / kWK : 1;
  const int64_t kps = (steps + splits - 1) / (splits < steps ? splits : steps);
  const int64_t eff = (steps + kps - 1) / kps;
  return eff <= 1 || n % 4 != 0 || m == 0 || n == 0 ? 1 : eff;
}

// Split-K product into the fp32 partial buffer `part` ([eff][M][N]), then the ordered reduction.
static int gemm_w_split_run(const void* a, int a_dtype, int64_t m, int64_t lda, const void* w, int fmt, int64_t n,
                            int64_t k, const void* scales, int scale_dtype, int64_t block_size, void* c, int c_dtype,
                            int64_t ldc, int64_t eff, float* part, void* stream, const char* what) {
  const int st = gemm_w_impl(a, a_dtype, m, lda, w, fmt, n, k, scales, scale_dtype, block_size, c, c_dtype, ldc,
                             (int)eff, part, stream);
  if (st != TGM_OK) return st;
  const int64_t quads = m * n / 4;
  const unsigned grid = (unsigned)((quads + 255) / 256 < 8192 ? (quads + 255) / 256 : 8192);
  hipLaunchKernelGGL(gemm_split_reduce, dim3(grid), dim3(256), 0, (hipStream_t)stream, (const float*)part, (int)eff, m,
                     n, c, c_dtype, ldc);
  return launch_status(what);
}

extern "C" int tgm_gemm_w_split(const void* a, int a_dtype, int64_t m, int64_t lda, const void* w, int fmt, int64_t n,
                                int64_t k, const void* scales, int scale_dtype, int64_t block_size, void* c,
                                int c_dtype, int64_t ldc, int64_t splits, void* workspace, int64_t workspace_bytes,
                                void* stream) {
  clear_error();
  TGM_CHECK_ARG(splits >= 1 && splits <= 64, "splits must be in [1, 64]");
  const int64_t eff = effective_splits(m, n, k, splits);
  if (eff == 1)
    return gemm_w_impl(a, a_dtype, m, lda, w, fmt, n, k, scales, scale_dtype, block_size, c, c_dtype, ldc, 1, nullptr,
                       stream);
  TGM_CHECK_ARG(workspace && workspace_bytes >= tgm_gemm_w_split_workspace(m, n, eff) &&
                    (uintptr_t)workspace % 16 == 0,
                "split-K needs a 16-byte aligned workspace of tgm_gemm_w_split_workspace() bytes");
  return gemm_w_split_run(a, a_dtype, m, lda, w, fmt, n, k, scales, scale_dtype, block_size, c, c_dtype, ldc, eff,
                          (float*)workspace, stream, "tgm_gemm_w_split");
}

// ---- tgm_gemm_w_split without a caller workspace (for callers that cannot allocate).
//
// The fp32 partials go to `scratch`, a fixed array in device memory that every GPU the library
// runs on holds once, from the code object's load until the process ends.  Its device address
// differs per GPU and is only known to the runtime: host code never passes `scratch` itself (in
// host code that name is a stand-in, not a device address) but the address hipGetSymbolAddress
// returns for the current device, looked up on the first call on each device and kept.  Each
// call overwrites every partial it later reads (every split writes its whole [M][N] slab), so
// nothing is cleared between calls.  All calls on one GPU share its array: calls that overlap in
// time on one GPU (two streams, two threads) race on it and must be ordered by the caller.
static constexpr int64_t kScratchBytes = int64_t(32) << 20;  // 32 MiB
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

static constexpr int kMaxDevices = 64;
static std::mutex scratch_lock;
static float* scratch_ptr[kMaxDevices];

// The address of `scratch` on the device `stream` launches on, which must be the calling
// thread's current device: hipGetSymbolAddress answers for the current device, so a stream of
// another device is rejected (TGM_E_INVALID) rather than handed that device's array.  The null
// stream and the legacy / per-thread default streams launch on the current device.  Returns a
// TGM_* status; *out is set on success.
static int scratch_address(hipStream_t stream, float** out) {
  int device = -1;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices) {
    set_error("tgm_gemm_w_split_noalloc: no usable current HIP device (%d)", device);
    return TGM_E_INVALID;
  }
  if (stream != nullptr && stream != hipStreamLegacy && stream != hipStreamPerThread) {
    hipDevice_t stream_device = -1;
    const hipError_t err = hipStreamGetDevice(stream, &stream_device);
    if (err != hipSuccess) {
      set_error("tgm_gemm_w_split_noalloc: hipStreamGetDevice failed: %s (%d)", hipGetErrorString(err), (int)err);
      return TGM_E_INVALID;
    }
    if ((int)stream_device != device) {
      set_error("tgm_gemm_w_split_noalloc: the stream belongs to device %d but device %d is current; make the "
                "stream's device current before the call", (int)stream_device, device);
      return TGM_E_INVALID;
    }
  }
  std::lock_guard<std::mutex> guard(scratch_lock);
  if (!scratch_ptr[device]) {
    void* ptr = nullptr;
    const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !ptr) {
      set_error("tgm_gemm_w_split_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s (%d)", device,
                hipGetErrorString(err), (int)err);
      return (int)(err != hipSuccess ? err : hipErrorInvalidSymbol);
    }
    scratch_ptr[device] = (float*)ptr;
  }
  *out = scratch_ptr[device];
  return TGM_OK;
}

extern "C" int64_t tgm_gemm_w_split_noalloc_capacity(void) { return kScratchBytes; }

extern "C" int tgm_gemm_w_split_noalloc(const void* a, int a_dtype, int64_t m, int64_t lda, const void* w, int fmt,
                                        int64_t n, int64_t k, const void* scales, int scale_dtype, int64_t block_size,
                                        void* c, int c_dtype, int64_t ldc, int64_t splits, void* stream) {
  clear_error();
  TGM_CHECK_ARG(splits >= 1 && splits <= 64, "splits must be in [1, 64]");
  const int64_t eff = effective_splits(m, n, k, splits);
  if (eff == 1)
    return gemm_w_impl(a, a_dtype, m, lda, w, fmt, n, k, scales, scale_dtype, block_size, c, c_dtype, ldc, 1, nullptr,
                       stream);
  const int64_t need = tgm_gemm_w_split_workspace(m, n, eff);
  TGM_CHECK_ARG(need <= kScratchBytes,
                "tgm_gemm_w_split_noalloc: %lld split(s) of %lld x %lld fp32 partials need %lld bytes, more than the "
                "%lld-byte static scratch; use fewer splits or tgm_gemm_w_split with a workspace",
                (long long)eff, (long long)m, (long long)n, (long long)need, (long long)kScratchBytes);
  float* part = nullptr;
  const int rc = scratch_address((hipStream_t)stream, &part);
  if (rc != TGM_OK) return rc;
  return gemm_w_split_run(a, a_dtype, m, lda, w, fmt, n, k, scales, scale_dtype, block_size, c, c_dtype, ldc, eff,
                          part, stream, "tgm_gemm_w_split_noalloc");
}

extern "C" int tgm_gemm_w_swiglu(const void* a, int a_dtype, int64_t m, int64_t lda, const void* w, int fmt, int64_t n,
                                 int64_t k, const void* scales, int scale_dtype, int64_t block_size, void* c,
                                 int c_dtype, int64_t ldc, void* stream) {
  clear_error();
  TGM_CHECK_ARG(a && w && c, "null operand");
  TGM_CHECK_ARG(valid_format(fmt), "unknown packed format %d", fmt);
  TGM_CHECK_ARG(m >= 0 && n >= 0 && k >= 0 && n % 2 == 0, "invalid gemm sizes (N must be even)");
  TGM_CHECK_ARG(m <= 1 || lda >= k, "lda smaller than K");
  TGM_CHECK_ARG(c_dtype == TGM_BF16 || c_dtype == TGM_F16 || c_dtype == TGM_F32, "output must be bf16, f16 or f32");
  TGM_CHECK_ARG(m <= 1 || ldc >= n / 2, "ldc smaller than N / 2");
  if (m == 0 || n == 0) return TGM_OK;
  if (fmt != TGM_FMT_FP4_E2M1 || a_dtype != TGM_BF16)
    TGM_UNSUPPORTED("tgm_gemm_w_swiglu: FP4 weights with bf16 activations only");
  const bool scaled = scales != nullptr;
  if (scaled && (scale_dtype != TGM_E8M0 || block_size != 32))
    TGM_UNSUPPORTED("tgm_gemm_w_swiglu: scales must be E8M0 per 32 K-elements");
  if (k == 0 || k % kWK != 0) TGM_UNSUPPORTED("tgm_gemm_w_swiglu: K must be a positive multiple of %d", kWK);
  if (m > 1 && (lda * 2) % 16 != 0) TGM_UNSUPPORTED("tgm_gemm_w_swiglu: activation rows must be 16-byte aligned");
  if (m >= (1ll << 31) || n >= (1ll << 31) || (m - 1) * lda * 2 + k * 2 >= (1ll << 32) || n * (k / 2) >= (1ll << 32))
    TGM_UNSUPPORTED("tgm_gemm_w_swiglu: operands must be under 4 GiB (32-bit offsets)");
  if ((uintptr_t)a % 16 || (uintptr_t)w % 16 || (scaled && (uintptr_t)scales % 4))
    TGM_UNSUPPORTED("tgm_gemm_w_swiglu: operands must be 16-byte and scales 4-byte aligned");
  const int64_t lda_eff = m > 1 ? lda : k;
  return scaled ? launch_gemm_w<TGM_FMT_FP4_E2M1, true, true>(a, lda_eff, w, scales, m, n, k, c, c_dtype, ldc,
                                                              (hipStream_t)stream)
                : launch_gemm_w<TGM_FMT_FP4_E2M1, false, true>(a, lda_eff, w, scales, m, n, k, c, c_dtype, ldc,
                                                               (hipStream_t)stream);
}
