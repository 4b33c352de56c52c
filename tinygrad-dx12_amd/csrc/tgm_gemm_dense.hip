// Kernel family 2, ordinary operands: bf16 x bf16 or f16 x f16 GEMM on 32x32x16 MFMA, and FP8 x
// FP8 (E4M3 / E5M2) decoded to bf16 in registers on the same MFMA (tgm_gemm_fp8).
//
// The reference lowers an ordinary scheduled matrix product to its collective LinAlg GEMM
// (alexandreteles/tinygrad-dx12 src/tinygrad_dx12/codegen/matmul.py:156-246, source from
// renderer/linalg.py:38-124).  This is that product on gfx950:
//
//   C[m, n] = sum_k A[m, k] * B[n, k]      A [M, K] (row stride lda), B [N, K] (row stride ldb)
//
// i.e. A @ B^T with both operands K-contiguous (batched over blockIdx.y with per-operand
// strides; consecutive batches may share B); a row-major B [K, N] is first transposed by
// tgm_transpose16 (the caller's staging copy, as the reference stages operands it cannot
// bind directly, matmul.py:218-226).  Products of two bf16 or two f16 values are exact in
// fp32; accumulation is fp32 and the output is rounded once.
//
// Workgroup: 128 (M) x 256 (N) output tile, eight waves in 2 x 4 (64 x 64 each, 2 x 2 MFMA
// tiles).  K advances 64 elements per step: the A panel (128 rows x 128 B) and B panel (256 rows
// x 128 B) go straight from global memory into a double-buffered LDS stage (buffer_load ... lds,
// zero-filled past M and N), 16-byte columns XOR-swizzled by (row / 2) % 8 so that the 32 rows a
// fragment read touches fall in distinct banks.  MFMA j of a step takes K [16 j + 8 h, + 8) for
// lane half h.  Loads of step s + 2 run while step s + 1 computes.
#include <type_traits>

#include "tgm_mfma_common.h"

namespace tgm {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 dn_bf16x8;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 dn_f16x8;

constexpr int kDM = 128, kDN = 256, kDK = 64;        // tile and K step
constexpr int kDRow = kDK * 2;                        // bytes per panel row and step
constexpr int kDStage = (kDM + kDN) * kDRow;          // 48 KB
constexpr int kDGroupM = 8;

// FP8 operands (E4M3 / E5M2) decoded to bf16 in registers: every FP8 value is exact in bf16, so
// the bf16 MFMA multiplies exactly the FP8 values.  (The gfx950 FP8 MFMA sums its 64-element
// products at reduced precision, measured ~2e-4 of sum |products|; the bf16 MFMA keeps fp32.)
template <bool E5M2>
__device__ __forceinline__ dn_bf16x8 fp8x8_to_bf16(u32x2 q) {
  typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 b2;
  b2 p[4];
  if constexpr (E5M2) {
    p[0] = __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(q[0], 1.0f, false);
    p[1] = __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(q[0], 1.0f, true);
    p[2] = __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(q[1], 1.0f, false);
    p[3] = __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(q[1], 1.0f, true);
  } else {
    p[0] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q[0], 1.0f, false);
    p[1] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q[0], 1.0f, true);
    p[2] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q[1], 1.0f, false);
    p[3] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q[1], 1.0f, true);
  }
  return dn_bf16x8{p[0][0], p[0][1], p[1][0], p[1][1], p[2][0], p[2][1], p[3][0], p[3][1]};
}

// Batched: blockIdx.y = z selects A + z * sa, B + (z / b_group) * sb and
// C + (z / c_group) * scg + (z % c_group) * sc (elements).  TA / TB: operand dtypes (TGM_BF16 /
// TGM_F16 on both sides, or TGM_FP8E4M3 / TGM_FP8E5M2 on each side).  A step is 128 bytes of
// each row: 64 16-bit or 128 FP8 elements.  alpha_a / alpha_b: optional fp32 device factors on
// the sums before the output rounding.
template <int TA, int TB>
__global__ void __launch_bounds__(512) gemm_dense(const uint8_t* __restrict__ a, unsigned lda_bytes,
                                                  const uint8_t* __restrict__ b, unsigned ldb_bytes, int M, int N,
                                                  int K, void* __restrict__ c, int cdt, int64_t ldc, int64_t sa,
                                                  int64_t sb, int64_t sc, int b_group, int c_group, int64_t scg,
                                                  const float* __restrict__ alpha_a, const float* __restrict__ alpha_b) {
  constexpr bool FP8 = TA == TGM_FP8E4M3 || TA == TGM_FP8E5M2;
  constexpr int ES = FP8 ? 1 : 2;   // bytes per element
  constexpr int KS = kDRow / ES;    // elements per step
  constexpr int FA = 2, FB = 2;
  const int z = blockIdx.y;
  a += z * sa * ES;
  b += (z / b_group) * sb * ES;
  c = (uint8_t*)c + ((int64_t)(z / c_group) * scg + (int64_t)(z % c_group) * sc) * dtype_size(cdt);
  __shared__ __attribute__((aligned(16))) unsigned char lds[2 * kDStage];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  const int tiles_m = (M + kDM - 1) / kDM, tiles_n = (N + kDN - 1) / kDN;
  int tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, kDGroupM, tm, tn);
  const int m0 = tm * kDM, n0 = tn * kDN;
  const int nsteps = K / KS;
  const i32x4v ra = buffer_rsrc(a, (unsigned)(M - 1) * lda_bytes + (unsigned)K * ES);
  const i32x4v rb = buffer_rsrc(b, (unsigned)(N - 1) * ldb_bytes + (unsigned)K * ES);
  const unsigned lds_base = (unsigned)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)lds;
  // Load instruction i fills rows 8 i .. 8 i + 7 of a panel: lane l writes slot l % 8 of row
  // 8 i + l / 8, which holds logical column (l % 8) ^ ((row / 2) % 8).  A: instructions
  // 2 wave, 2 wave + 1; B: 4 wave .. 4 wave + 3.
  unsigned voa[2], vob[4];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int row = 8 * (2 * wave + q) + (lane >> 3);
    voa[q] = (unsigned)(m0 + row) * lda_bytes + (unsigned)((lane & 7) ^ ((row >> 1) & 7)) * 16u;
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int row = 8 * (4 * wave + q) + (lane >> 3);
    vob[q] = (unsigned)(n0 + row) * ldb_bytes + (unsigned)((lane & 7) ^ ((row >> 1) & 7)) * 16u;
  }
  auto dma_step = [&](int s, int buf) __attribute__((always_inline)) {
    const unsigned st = lds_base + (unsigned)(buf * kDStage);
#pragma unroll
    for (int q = 0; q < 2; ++q) lds_dma16(ra, st + (unsigned)(2 * wave + q) * 1024u, voa[q] + (unsigned)s * kDRow);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      lds_dma16(rb, st + (unsigned)(kDM * kDRow) + (unsigned)(4 * wave + q) * 1024u, vob[q] + (unsigned)s * kDRow);
  };
  const int half = lane >> 5;
  const int a_row = wm * 64 + (lane & 31), b_row = wn * 64 + (lane & 31);
  using V = typename std::conditional<TA == TGM_F16, dn_f16x8, dn_bf16x8>::type;  // the MFMA operand type
  // MFMA j of a step takes K [16 j + 8 h, + 8) for lane half h: 16 bytes at logical column
  // 2 j + h (16-bit), or 8 bytes at byte 8 h of column j (FP8, decoded to bf16)
  auto frag = [&](const unsigned char* panel, int row, int j, auto tag) __attribute__((always_inline)) {
    if constexpr (FP8) {
      const u32x2 q = *(const u32x2*)(panel + row * kDRow + ((j ^ ((row >> 1) & 7)) * 16) + 8 * half);
      return fp8x8_to_bf16<decltype(tag)::value == TGM_FP8E5M2>(q);
    } else {
      return *(const V*)(panel + row * kDRow + (((2 * j + half) ^ ((row >> 1) & 7)) * 16));
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
    const unsigned char* pa = lds + cur * kDStage;
    const unsigned char* pb = pa + kDM * kDRow;
#pragma unroll
    for (int j = 0; j < KS / 16; ++j) {
      V fa[FA], fb[FB];
#pragma unroll
      for (int t = 0; t < FA; ++t) fa[t] = frag(pa, a_row + 32 * t, j, std::integral_constant<int, TA>{});
#pragma unroll
      for (int t = 0; t < FB; ++t) fb[t] = frag(pb, b_row + 32 * t, j, std::integral_constant<int, TB>{});
#pragma unroll
      for (int ta = 0; ta < FA; ++ta)
#pragma unroll
        for (int tb = 0; tb < FB; ++tb) {
          if constexpr (TA == TGM_F16)
            acc[ta][tb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[ta], fb[tb], acc[ta][tb], 0, 0, 0);
          else
            acc[ta][tb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[ta], fb[tb], acc[ta][tb], 0, 0, 0);
        }
    }
    wait_lds_dma();   // this wave's loads of step s + 1
    __syncthreads();  // every wave is done with this buffer; step s + 1 is complete in the other
    dma_step(s2, cur);
  }
  wait_lds_dma();
  __syncthreads();  // the epilogue reuses the LDS
  if (alpha_a || alpha_b) {
    const float alpha = (alpha_a ? *alpha_a : 1.0f) * (alpha_b ? *alpha_b : 1.0f);
#pragma unroll
    for (int i = 0; i < FA; ++i)
#pragma unroll
      for (int j = 0; j < FB; ++j) acc[i][j] *= alpha;
  }
  float* ep = (float*)lds + wave * 32 * 36;
#pragma unroll
  for (int i = 0; i < FA; ++i)
#pragma unroll
    for (int j = 0; j < FB; ++j)
      store_tile32(acc[i][j], ep, lane, m0 + wm * 64 + i * 32, n0 + wn * 64 + j * 32, M, N, c, cdt, ldc);
}

// ---------------------------------------------------------------------------------------------
// Persistent form for one large bf16 / f16 product (K a multiple of 128, at least one round of
// 256 x 256 tiles): the FP4 GEMM's persistent schedule (tgm_gemm_mx.hip, gemm_mx_fp4_stream) on
// the 16-bit MFMA.  A K step of 64 elements is 128 bytes of a row -- the FP4 kernel's step width
// -- so panels, swizzle, load pieces and fragment reads are laid out exactly as there:
//
//  * one workgroup per CU (G, a multiple of 8, so a workgroup keeps to its XCD's tile range)
//    walks tiles blockIdx.x, blockIdx.x + G, ... of 256 x 256 as one stream of K steps;
//  * eight waves in 4 x 2, each 64 x 128 = 2 x 4 MFMA tiles of v_mfma_f32_32x32x16_{bf16,f16}
//    (128 fp32 accumulators per lane, two waves per SIMD): 0.75 KB of LDS fragment reads per
//    MFMA, against 1 KB for gemm_dense's 64 x 64 wave tiles;
//  * a step's A and B panels (256 rows x 128 B each) go straight from global memory into one of
//    two 64 KB LDS buffers (buffer_load ... lds), 16-byte columns XOR-swizzled by (row / 2) % 8;
//    the loads of step s + 2 are issued during step s + 1's MFMAs, half in its first substep and
//    half in its last, across tile boundaries (the next tile's first steps load during the
//    current tile's last);
//  * substep u of a step takes K [16 u + 8 h, + 8) for lane half h (16-byte column 2 u + h); after
//    every MFMA the wave issues an even share of the next substep's fragment reads and of the
//    panel loads, fenced by scheduling barriers;
//  * at a tile's end each wave rounds its 32 x 32 tiles to 16 bits through its own 2 KB LDS slice
//    and writes 16-byte row segments with non-temporal stores (fp32 output goes out per element).
constexpr int kSB = 256;                 // output tile edge
constexpr int kSRow = 128;               // bytes per panel row and step
constexpr int kSPanel = kSB * kSRow;     // 32 KB
constexpr int kSBuffer = 2 * kSPanel;    // A and B panels of one step
constexpr int kSEpi = 8 * 2048;          // one 2 KB epilogue slice per wave
constexpr int kSLds = 2 * kSBuffer + kSEpi;

template <int T>
__global__ void __launch_bounds__(512) gemm_dense_stream(const uint8_t* __restrict__ a, unsigned lda_bytes,
                                                         const uint8_t* __restrict__ b, unsigned ldb_bytes, int M,
                                                         int N, int K, void* __restrict__ c, int cdt, int64_t ldc) {
  using V = typename std::conditional<T == TGM_F16, dn_f16x8, dn_bf16x8>::type;
  __shared__ __attribute__((aligned(16))) unsigned char lds[kSLds];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  constexpr int WN = 2, FA = 2, FB = 4;  // 4 x 2 waves of 64 x 128
  constexpr int NI = 4, NP = 2 * NI;     // panel loads per wave, operand and step; pieces per step
  const int wm = wave / WN, wn = wave % WN;
  const int tiles_m = (M + kSB - 1) / kSB, tiles_n = (N + kSB - 1) / kSB;
  const int ntiles = tiles_m * tiles_n;
  const int G = gridDim.x;
  const int my_tiles = (ntiles - (int)blockIdx.x + G - 1) / G;  // >= 1 (the host launches G <= ntiles)
  const int nsteps = K / 64;                                     // even (K % 128 == 0)
  const int total = my_tiles * nsteps;

  const i32x4v ra = buffer_rsrc(a, (unsigned)(M - 1) * lda_bytes + (unsigned)K * 2u);
  const i32x4v rb = buffer_rsrc(b, (unsigned)(N - 1) * ldb_bytes + (unsigned)K * 2u);
  // Load instruction i of a wave fills rows 32 wave + 8 i .. + 7 of a panel: lane l writes slot
  // l % 8 of row 32 wave + 8 i + l / 8, which holds logical column (l % 8) ^ ((row >> 1) & 7) =
  // (l % 8) ^ (l >> 4), flipped by 4 for odd i.  Rows past M or N read zeros (buffer bounds).
  const int lrow = wave * 32 + (lane >> 3);
  const unsigned lcol = (unsigned)(((lane & 7) ^ (lane >> 4)) * 16);
  const unsigned la0 = (unsigned)lrow * lda_bytes, lb0 = (unsigned)lrow * ldb_bytes;
  const unsigned lds_base = (unsigned)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)lds;
  struct Tiles {
    int base, mc, nc, mn, nn;  // first stream step of the tile; origins of this tile and the next
  } tl;
  auto tile_origin = [&](int t, int& m0, int& n0) __attribute__((always_inline)) {
    int tm, tn;
    tile_of((int)blockIdx.x + t * G, tiles_m, tiles_n, kDGroupM, tm, tn);
    m0 = tm * kSB;
    n0 = tn * kSB;
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
  struct StepOff {
    unsigned a, b;  // uniform byte offsets of a stream step in A and B
  };
  // stream step gs (clamped to the stream) lies in the current tile or the next
  auto step_off = [&](int gs) __attribute__((always_inline)) {
    gs = gs < total ? gs : total - 1;
    const int local = gs - tl.base;
    const bool cur = local < nsteps;
    const int m0 = cur ? tl.mc : tl.mn, n0 = cur ? tl.nc : tl.nn, st = cur ? local : local - nsteps;
    return StepOff{(unsigned)__builtin_amdgcn_readfirstlane((int)((unsigned)m0 * lda_bytes + (unsigned)(st * kSRow))),
                   (unsigned)__builtin_amdgcn_readfirstlane((int)((unsigned)n0 * ldb_bytes + (unsigned)(st * kSRow)))};
  };
  auto dma_piece = [&](const StepOff& o, int buf, int p) __attribute__((always_inline)) {
    const int i = p >> 1;
    const unsigned col = lcol ^ (unsigned)((i & 1) * 64);
    const unsigned la = lds_base + (unsigned)(buf * kSBuffer + (p & 1) * kSPanel + wave * 4096 + i * 1024);
    if (p & 1) lds_dma16(rb, la, lb0 + (unsigned)(8 * i) * ldb_bytes + col + o.b);
    else lds_dma16(ra, la, la0 + (unsigned)(8 * i) * lda_bytes + col + o.a);
  };
  auto dma_pieces = [&](int gs, int buf, int p0, int p1) __attribute__((always_inline)) {
    const StepOff o = step_off(gs);
#pragma unroll
    for (int p = 0; p < NP; ++p)
      if (p >= p0 && p < p1) dma_piece(o, buf, p);
  };
  f32x16 acc[FA][FB];
#pragma unroll
  for (int i = 0; i < FA; ++i)
#pragma unroll
    for (int j = 0; j < FB; ++j) acc[i][j] = f32x16{};

  const int half = lane >> 5;
  const int sw = (lane >> 1) & 7;  // (row >> 1) & 7 of every row this lane reads
  const int fa_row = (wm * FA * 32 + (lane & 31)) * kSRow;
  const int fb_row = (wn * FB * 32 + (lane & 31)) * kSRow;
  struct Frags {
    u32x4 a[FA], b[FB];
  };
  // fragment t (A 0..FA-1, then B) of substep u from buffer buf
  auto read_item = [&](Frags& f, int buf, int u, int t) __attribute__((always_inline)) {
    const unsigned char* la = lds + buf * kSBuffer;
    const int col = ((2 * u + half) ^ sw) * 16;
    if (t < FA) f.a[t < FA ? t : 0] = *(const u32x4*)(la + fa_row + col + t * 32 * kSRow);
    else f.b[t < FA ? 0 : t - FA] = *(const u32x4*)(la + kSPanel + fb_row + col + (t - FA) * 32 * kSRow);
  };
  auto mfmas = [&](const Frags& f, auto&& hook) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < FA; ++i)
#pragma unroll
      for (int j = 0; j < FB; ++j) {
        const V va = __builtin_bit_cast(V, f.a[i]), vb = __builtin_bit_cast(V, f.b[j]);
        if constexpr (T == TGM_F16) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, vb, acc[i][j], 0, 0, 0);
        else acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, vb, acc[i][j], 0, 0, 0);
        hook(i * FB + j);
      }
  };
  // One substep: the MFMAs of fragments fc, with the reads of fn (substep ru of buffer rbuf) and
  // load pieces [p0, p1) of offsets lo into buffer dbuf spread over them, one item after each
  // MFMA share (reads first).
  constexpr int kMaxItems = (FA + FB) + NP;
  auto substep = [&](const Frags& fc, Frags& fn, int rbuf, int ru, const StepOff* lo, int dbuf, int p0,
                     int p1) __attribute__((always_inline)) {
    constexpr int nr = FA + FB;
    const int ni = nr + (p1 - p0);
    mfmas(fc, [&](int idx) __attribute__((always_inline)) {
#pragma unroll
      for (int it = 0; it < kMaxItems; ++it) {
        if (it < ni && it * FA * FB / ni == idx) {
          __builtin_amdgcn_sched_barrier(0);
          if (it >= nr) dma_piece(*lo, dbuf, p0 + it - nr);
          else read_item(fn, rbuf, ru, it);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    });
  };
  set_tile(0);
  dma_pieces(0, 0, 0, NP);
  dma_pieces(1, 1, 0, NP / 2);
  wait_lds_dma();
  __syncthreads();
  Frags f0, f1;
#pragma unroll
  for (int t = 0; t < FA + FB; ++t) {
    __builtin_amdgcn_sched_barrier(0);
    read_item(f0, 0, 0, t);
  }
  __builtin_amdgcn_sched_barrier(0);
  // Step gs from buffer cur:
  //   u0 (f0): read f1 <- u1; second half of step gs + 1's loads (into the other buffer)
  //   u1 (f1): read f0 <- u2
  //   u2 (f0): read f1 <- u3
  //   wait for this wave's loads of step gs + 1, barrier: step gs + 1 is complete in the other
  //       buffer and every read of this buffer has been issued and completed
  //   u3 (f1): read f0 <- u0 of step gs + 1; first half of step gs + 2's loads (into this buffer)
  auto step = [&](int gs, int cur) __attribute__((always_inline)) {
    const StepOff o1 = step_off(gs + 1), o2 = step_off(gs + 2);
    substep(f0, f1, cur, 1, &o1, cur ^ 1, NP / 2, NP);
    substep(f1, f0, cur, 2, &o1, 0, 0, 0);
    substep(f0, f1, cur, 3, &o1, 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    wait_lds_dma();
    __syncthreads();
    substep(f1, f0, cur ^ 1, 0, &o2, cur, 0, NP / 2);
    __builtin_amdgcn_sched_barrier(0);
  };
  uint16_t* ep = (uint16_t*)(lds + 2 * kSBuffer) + wave * 1024;
  int gs = 0;
  for (int t = 0; t < my_tiles; ++t) {
    set_tile(t);
    for (int s = 0; s < nsteps; s += 2, gs += 2) {
      step(gs, 0);
      step(gs + 1, 1);
    }
    // Tile t is complete (MFMA D layout: lane l holds column l % 32 and rows 8 (v / 4) + 4 (l / 32)
    // + v % 4 of each 32 x 32 tile); the wave's epilogue slice is its own.
    const int col0 = tl.nc + wn * FB * 32;
    const int row0 = tl.mc + wm * FA * 32;
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
#pragma unroll
          for (int v = 0; v < 16; v += 2) {  // rows v and v + 1 of the lane's column, one rounding instruction
            const float x0 = acc[i][j][v], x1 = acc[i][j][v + 1];
            const unsigned h = cdt == TGM_BF16 ? bf16x2_bits(x0, x1)
                                               : __builtin_bit_cast(unsigned short, (_Float16)x0) |
                                                     ((unsigned)__builtin_bit_cast(unsigned short, (_Float16)x1) << 16);
            const int r = 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
            ep[r * 32 + (lane & 31)] = (unsigned short)h;
            ep[(r + 1) * 32 + (lane & 31)] = (unsigned short)(h >> 16);
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
                __builtin_nontemporal_store(*(const u32x4*)(ep + r * 32 + cc), (u32x4*)out);
              } else {  // the ragged edge, element by element from LDS
#pragma unroll 1
                for (int e = 0; e < 8 && col + e < N; ++e) out[e] = ep[r * 32 + cc + e];
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

// out[j, i] = in[i, j] through padded 64 x 64 LDS tiles; T = uint16_t (bf16 / f16) or uint8_t (fp8).
template <typename T>
__global__ void __launch_bounds__(256) transpose_t(const T* __restrict__ in, int rows, int cols, int64_t ld_in,
                                                   T* __restrict__ out, int64_t ld_out) {
  __shared__ T t[64][65];
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int i = ty; i < 64; i += 4) {
    const int r = r0 + i, cc = c0 + tx;
    if (r < rows && cc < cols) t[i][tx] = in[(int64_t)r * ld_in + cc];
  }
  __syncthreads();
  for (int i = ty; i < 64; i += 4) {
    const int cc = c0 + i, r = r0 + tx;
    if (cc < cols && r < rows) out[(int64_t)cc * ld_out + r] = t[tx][i];
  }
}

}  // namespace tgm

using namespace tgm;

extern "C" int tgm_gemm_dense_batched(const void* a, int a_dtype, int64_t m, int64_t lda, int64_t stride_a,
                                      const void* b, int b_dtype, int64_t n, int64_t ldb, int64_t stride_b,
                                      int64_t b_group, int64_t k, void* c, int c_dtype, int64_t ldc, int64_t stride_c,
                                      int64_t c_group, int64_t stride_c_group,
                                      int64_t batch, void* stream) {
  clear_error();
  TGM_CHECK_ARG(a && b && c, "null operand");
  TGM_CHECK_ARG(m >= 0 && n >= 0 && k >= 0 && batch >= 0 && b_group >= 1 && c_group >= 1 && b_group < (1ll << 31) &&
                    c_group < (1ll << 31),
                "invalid gemm sizes");
  TGM_CHECK_ARG(m <= 1 || lda >= k, "lda smaller than K");
  TGM_CHECK_ARG(n <= 1 || ldb >= k, "ldb smaller than K");
  TGM_CHECK_ARG(m <= 1 || ldc >= n, "ldc smaller than N");
  TGM_CHECK_ARG(stride_a >= 0 && stride_b >= 0 && stride_c >= 0 && stride_c_group >= 0, "negative batch stride");
  TGM_CHECK_ARG(c_dtype == TGM_BF16 || c_dtype == TGM_F16 || c_dtype == TGM_F32, "output must be bf16, f16 or f32");
  if (m == 0 || n == 0 || batch == 0) return TGM_OK;
  if (a_dtype != b_dtype || (a_dtype != TGM_BF16 && a_dtype != TGM_F16))
    TGM_UNSUPPORTED("tgm_gemm_dense: operands must both be bf16 or both f16");
  if (k == 0 || k % kDK != 0) TGM_UNSUPPORTED("tgm_gemm_dense: K must be a positive multiple of %d", kDK);
  const int64_t lda_eff = m > 1 ? lda : k, ldb_eff = n > 1 ? ldb : k;
  if ((lda_eff * 2) % 16 || (ldb_eff * 2) % 16 || (uintptr_t)a % 16 || (uintptr_t)b % 16 ||
      (batch > 1 && ((stride_a * 2) % 16 || (stride_b * 2) % 16)))
    TGM_UNSUPPORTED("tgm_gemm_dense: operands and their rows must be 16-byte aligned");
  if (m >= (1ll << 31) || n >= (1ll << 31) || (m - 1) * lda_eff * 2 + k * 2 >= (1ll << 32) ||
      (n - 1) * ldb_eff * 2 + k * 2 >= (1ll << 32) || batch > 65535)
    TGM_UNSUPPORTED("tgm_gemm_dense: operands must be under 4 GiB (32-bit offsets), at most 65535 batches");
  const hipStream_t st = (hipStream_t)stream;
  const int64_t tiles_s = ((m + kSB - 1) / kSB) * ((n + kSB - 1) / kSB);
  const int cus = stream_cu_count(st);
  if (batch == 1 && k % 128 == 0 && cus >= 8 && tiles_s >= cus) {
    // one large product: persistent, one workgroup per CU (a multiple of 8 of them)
    const dim3 g((unsigned)(cus / 8 * 8));
    if (a_dtype == TGM_BF16)
      hipLaunchKernelGGL((gemm_dense_stream<TGM_BF16>), g, dim3(512), 0, st, (const uint8_t*)a, (unsigned)(lda_eff * 2),
                         (const uint8_t*)b, (unsigned)(ldb_eff * 2), (int)m, (int)n, (int)k, c, c_dtype, ldc);
    else
      hipLaunchKernelGGL((gemm_dense_stream<TGM_F16>), g, dim3(512), 0, st, (const uint8_t*)a, (unsigned)(lda_eff * 2),
                         (const uint8_t*)b, (unsigned)(ldb_eff * 2), (int)m, (int)n, (int)k, c, c_dtype, ldc);
    return launch_status("tgm_gemm_dense");
  }
  const int64_t tiles = ((m + kDM - 1) / kDM) * ((n + kDN - 1) / kDN);
  const dim3 grid((unsigned)tiles, (unsigned)batch);
  if (a_dtype == TGM_BF16)
    hipLaunchKernelGGL((gemm_dense<TGM_BF16, TGM_BF16>), grid, dim3(512), 0, st, (const uint8_t*)a,
                       (unsigned)(lda_eff * 2), (const uint8_t*)b, (unsigned)(ldb_eff * 2), (int)m, (int)n, (int)k, c,
                       c_dtype, ldc, stride_a, stride_b, stride_c, (int)b_group, (int)c_group, stride_c_group,
                       (const float*)nullptr, (const float*)nullptr);
  else
    hipLaunchKernelGGL((gemm_dense<TGM_F16, TGM_F16>), grid, dim3(512), 0, st, (const uint8_t*)a,
                       (unsigned)(lda_eff * 2), (const uint8_t*)b, (unsigned)(ldb_eff * 2), (int)m, (int)n, (int)k, c,
                       c_dtype, ldc, stride_a, stride_b, stride_c, (int)b_group, (int)c_group, stride_c_group,
                       (const float*)nullptr, (const float*)nullptr);
  return launch_status("tgm_gemm_dense");
}

extern "C" int tgm_gemm_fp8(const void* a, int a_dtype, int64_t lda, int64_t m, const void* b, int b_dtype,
                            int64_t ldb, int64_t n, int64_t k, const float* scale_a, const float* scale_b, void* c,
                            int c_dtype, int64_t ldc, void* stream) {
  clear_error();
  TGM_CHECK_ARG(a && b && c, "null operand");
  TGM_CHECK_ARG(m >= 0 && n >= 0 && k >= 0, "invalid gemm sizes");
  TGM_CHECK_ARG(m <= 1 || lda >= k, "lda smaller than K");
  TGM_CHECK_ARG(n <= 1 || ldb >= k, "ldb smaller than K");
  TGM_CHECK_ARG(m <= 1 || ldc >= n, "ldc smaller than N");
  TGM_CHECK_ARG(c_dtype == TGM_BF16 || c_dtype == TGM_F16 || c_dtype == TGM_F32, "output must be bf16, f16 or f32");
  const bool fa = a_dtype == TGM_FP8E4M3 || a_dtype == TGM_FP8E5M2, fb = b_dtype == TGM_FP8E4M3 || b_dtype == TGM_FP8E5M2;
  TGM_CHECK_ARG(fa && fb, "tgm_gemm_fp8 takes FP8 E4M3 / E5M2 operands");
  if (m == 0 || n == 0) return TGM_OK;
  if (k == 0 || k % kDRow != 0) TGM_UNSUPPORTED("tgm_gemm_fp8: K must be a positive multiple of %d", kDRow);
  const int64_t lda_eff = m > 1 ? lda : k, ldb_eff = n > 1 ? ldb : k;
  if (lda_eff % 16 || ldb_eff % 16 || (uintptr_t)a % 16 || (uintptr_t)b % 16)
    TGM_UNSUPPORTED("tgm_gemm_fp8: operands and their rows must be 16-byte aligned");
  if (m >= (1ll << 31) || n >= (1ll << 31) || k >= (1ll << 31) || (m - 1) * lda_eff + k >= (1ll << 32) ||
      (n - 1) * ldb_eff + k >= (1ll << 32))
    TGM_UNSUPPORTED("tgm_gemm_fp8: operands must be under 4 GiB (32-bit offsets)");
  const int64_t tiles = ((m + kDM - 1) / kDM) * ((n + kDN - 1) / kDN);
  const hipStream_t st = (hipStream_t)stream;
#define TGM_FP8_PAIR(A, B)                                                                                       \
  if (a_dtype == A && b_dtype == B) {                                                                            \
    hipLaunchKernelGGL((gemm_dense<A, B>), dim3((unsigned)tiles), dim3(512), 0, st, (const uint8_t*)a,           \
                       (unsigned)lda_eff, (const uint8_t*)b, (unsigned)ldb_eff, (int)m, (int)n, (int)k, c, c_dtype, \
                       ldc, (int64_t)0, (int64_t)0, (int64_t)0, 1, 1, (int64_t)0, scale_a, scale_b);           \
    return launch_status("tgm_gemm_fp8");                                                                        \
  }
  TGM_FP8_PAIR(TGM_FP8E4M3, TGM_FP8E4M3) TGM_FP8_PAIR(TGM_FP8E4M3, TGM_FP8E5M2)
  TGM_FP8_PAIR(TGM_FP8E5M2, TGM_FP8E4M3) TGM_FP8_PAIR(TGM_FP8E5M2, TGM_FP8E5M2)
#undef TGM_FP8_PAIR
  return TGM_E_UNSUPPORTED;
}

extern "C" int tgm_gemm_dense(const void* a, int a_dtype, int64_t m, int64_t lda, const void* b, int b_dtype, int64_t n,
                              int64_t ldb, int64_t k, void* c, int c_dtype, int64_t ldc, void* stream) {
  return tgm_gemm_dense_batched(a, a_dtype, m, lda, 0, b, b_dtype, n, ldb, 0, 1, k, c, c_dtype, ldc, 0, 1, 0, 1, stream);
}

extern "C" int tgm_transpose16(const void* in, int64_t rows, int64_t cols, int64_t ld_in, void* out, int64_t ld_out,
                               void* stream) {
  clear_error();
  TGM_CHECK_ARG(in && out, "null operand");
  TGM_CHECK_ARG(rows >= 0 && cols >= 0 && rows < (1ll << 31) && cols < (1ll << 31), "invalid sizes");
  TGM_CHECK_ARG(rows <= 1 || ld_in >= cols, "ld_in smaller than cols");
  TGM_CHECK_ARG(cols <= 1 || ld_out >= rows, "ld_out smaller than rows");
  if (rows == 0 || cols == 0) return TGM_OK;
  const dim3 grid((unsigned)((cols + 63) / 64), (unsigned)((rows + 63) / 64));
  if (grid.y > 65535) TGM_UNSUPPORTED("tgm_transpose16: too many rows");
  hipLaunchKernelGGL(transpose_t<uint16_t>, grid, dim3(256), 0, (hipStream_t)stream, (const uint16_t*)in, (int)rows,
                     (int)cols, ld_in, (uint16_t*)out, ld_out);
  return launch_status("tgm_transpose16");
}

extern "C" int tgm_transpose8(const void* in, int64_t rows, int64_t cols, int64_t ld_in, void* out, int64_t ld_out,
                              void* stream) {
  clear_error();
  TGM_CHECK_ARG(in && out, "null operand");
  TGM_CHECK_ARG(rows >= 0 && cols >= 0 && rows < (1ll << 31) && cols < (1ll << 31), "invalid sizes");
  TGM_CHECK_ARG(rows <= 1 || ld_in >= cols, "ld_in smaller than cols");
  TGM_CHECK_ARG(cols <= 1 || ld_out >= rows, "ld_out smaller than rows");
  if (rows == 0 || cols == 0) return TGM_OK;
  const dim3 grid((unsigned)((cols + 63) / 64), (unsigned)((rows + 63) / 64));
  if (grid.y > 65535) TGM_UNSUPPORTED("tgm_transpose8: too many rows");
  hipLaunchKernelGGL(transpose_t<uint8_t>, grid, dim3(256), 0, (hipStream_t)stream, (const uint8_t*)in, (int)rows,
                     (int)cols, ld_in, (uint8_t*)out, ld_out);
  return launch_status("tgm_transpose8");
}
