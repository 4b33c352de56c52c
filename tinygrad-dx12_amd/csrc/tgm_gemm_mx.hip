// Kernel family 2, block-scaled path: FP4 (E2M1) x FP4 GEMM on gfx950 scaled MFMA.
//
// Replaces the reference's collective LinAlg GEMM (alexandreteles/tinygrad-dx12
// src/tinygrad_dx12/renderer/linalg.py:38-124) for two packed operands.  The reference
// first decodes both operands to the fp32 intermediate (codegen/decomp/dx12.py:115-138,
// 49-106) and multiplies those; here the packed codes and their E8M0 scales feed
// v_mfma_scale_f32_32x32x64_f8f6f4 directly.  FP4 x FP4 products with power-of-two
// scales are exact in fp32, so only the summation order differs from the reference.
//
//   C[m, n] = sum_k deq(A)[m, k] * deq(B)[n, k]
//
// A [M, K] and B [N, K] are stored K-contiguous, two codes per byte (low nibble first),
// with one E8M0 scale byte per 32 K-elements ([M, K/32], [N, K/32]).
//
// MFMA operand layout (32x32x64): lane l supplies row (l % 32) of its operand and the 32
// consecutive K elements [32 * (l / 32), +32) of the 64-element K step -- 16 bytes of
// packed codes, i.e. one MX block, and that block's scale in byte 0 of its scale VGPR.
// D layout: lane l holds column l % 32 and rows 8 * (v / 4) + 4 * (l / 32) + v % 4.
//
// Workgroup: 256 x 256 output tile, eight waves in 4 x 2, each wave 64 x 128 = 2 x 4 MFMA
// tiles (128 fp32 accumulators per lane, two waves per SIMD).  K advances in steps of 256
// elements (128 bytes per row and operand): each step's A and B panels (32 KB each) are
// loaded straight from global memory into a double-buffered LDS tile (buffer_load ... lds),
// XOR-swizzled so the 32 rows one ds_read_b128 touches fall in distinct banks; the E8M0
// scales take the same route four steps at a time into their own double buffer (160 KB of
// LDS in all).  The loads of step s + 2 run while step s + 1's MFMAs do.  Tiles are mapped
// XCD-aware (tile_of).  For K a multiple of 1024 the same pipeline runs persistently, one
// workgroup per CU streaming its tiles' steps back to back (gemm_mx_fp4_stream); other K
// launch one workgroup per tile (gemm_mx_fp4).
#include <type_traits>

#include "tgm_mfma_common.h"

namespace tgm {

constexpr int kBM = 256, kBN = 256;  // output tile
constexpr int kBK = 256;             // K elements per step
constexpr int kRowBytes = kBK / 2;   // FP4 bytes per row and step
constexpr int kPanel = kBM * kRowBytes;          // one operand, one buffer (32 KB)
constexpr int kBuffer = 2 * kPanel;              // A and B panels of one step (64 KB)
constexpr int kBatchSteps = 4;                   // steps per batch of E8M0 scales
constexpr int kBatchRow = kBatchSteps * (kBK / 32);  // scale bytes of one row per batch (32)
constexpr int kBatch = 2 * kBM * kBatchRow;      // A and B scales of one batch (16 KB)
constexpr int kLds = 2 * kBuffer + 2 * kBatch;   // two step buffers, two scale batches: 160 KB
constexpr int kGroupM = 8;
constexpr int kWavesM = 4, kWavesN = 2;  // wave grid of the launched kernel

// WM x WN waves per workgroup; wave tile (256 / WM) x (256 / WN) = FA x FB MFMA tiles.
template <int WM, int WN>
__global__ void __launch_bounds__(WM * WN * 64) gemm_mx_fp4(const uint8_t* __restrict__ a, const uint8_t* __restrict__ sa,
                                                   const uint8_t* __restrict__ b, const uint8_t* __restrict__ sb,
                                                   int M, int N, int K, void* __restrict__ c, int cdt, int64_t ldc) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[kLds];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  constexpr int NW = WM * WN, FA = 8 / WM, FB = 8 / WN;  // 32-row fragments per wave
  constexpr int NI = 32 / NW;                             // panel loads per wave, operand and step
  static_assert(NW == 4 || NW == 8, "scale batches are loaded by 4 or 8 waves");
  const int wm = wave / WN, wn = wave % WN;
  const int tiles_m = (M + kBM - 1) / kBM, tiles_n = (N + kBN - 1) / kBN;
  int tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, kGroupM, tm, tn);
  const int m0 = tm * kBM, n0 = tn * kBN;
  const int nsteps = K / kBK;

  // Global -> LDS: direct loads (buffer_load_dwordx4 ... lds) write 16 bytes per lane at
  // the LDS address of the instruction plus 16 * lane, so a wave instruction fills 64
  // consecutive 16-byte slots of a panel (256 rows x 128 bytes).  Slot s holds row s / 8
  // and 16-byte column (s % 8) ^ ((row >> 1) & 7): the XOR swizzle puts the 32 rows one
  // fragment read touches (same logical column) into distinct banks, and each wave
  // instruction still covers 8 whole 128-byte rows of global memory.  With NW waves, wave w
  // issues the 32 / NW instructions for slots [2048 w / NW, 2048 (w + 1) / NW) of each
  // operand.  The loads go through buffer resources sized to the operands: rows past M or N
  // read zeros (their results are
  // dropped), so no address needs clamping and every load's offset is one per-lane value
  // plus a uniform one.  Offsets are 32-bit (the host keeps each operand under 4 GiB).
  const unsigned kb = (unsigned)(K / 2);
  const unsigned kblk = (unsigned)(K / 32);
  const i32x4v ra = buffer_rsrc(a, (unsigned)M * kb), rb = buffer_rsrc(b, (unsigned)N * kb);
  const i32x4v rsa = buffer_rsrc(sa, (unsigned)M * kblk), rsb = buffer_rsrc(sb, (unsigned)N * kblk);
  // Lane l of load i covers row lrow + 8 i, whose swizzle term ((lrow + 8 i) >> 1) & 7 is
  // ((l >> 4) + 4 i) & 7 = (l >> 4) ^ (4 (i & 1)): the 16-byte column it fetches is
  // (l % 8) ^ (l >> 4), flipped by 4 on odd loads.
  const int lrow = wave * (256 / NW) + (lane >> 3);  // + 8 i
  const unsigned lcol = (unsigned)(((lane & 7) ^ (lane >> 4)) * 16);
  const unsigned voa = (unsigned)(m0 + lrow) * kb, vob = (unsigned)(n0 + lrow) * kb;
  const unsigned lds_base = (unsigned)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)lds;
  // One panel load instruction of step s into buffer buf: piece 2i / 2i + 1 is A / B load i.
  constexpr int NP = 2 * NI;
  auto dma_piece = [&](int s, int buf, int p) __attribute__((always_inline)) {
    const int i = p >> 1;
    const unsigned step_off = (unsigned)(8 * i) * kb + (unsigned)(s * kRowBytes);  // uniform
    const unsigned col = lcol ^ (unsigned)((i & 1) * 64);
    const unsigned la = lds_base + (unsigned)(buf * kBuffer + (p & 1) * kPanel + wave * (2048 / NW) * 16 + i * 1024);
    lds_dma16((p & 1) ? rb : ra, la, ((p & 1) ? vob : voa) + col + step_off);
  };
  // Scales arrive in batches of kBatchSteps steps: batch b's 32 E8M0 bytes of row r (steps
  // 4b .. 4b + 3) land at byte r * 32 of scale buffer b & 1 (A rows, then B rows), two 16-byte
  // lanes per row, 32 rows per instruction.  Fetching a row's 8 bytes of one step at a time
  // costs a cache-line access per row and step -- as many as the operand panels themselves --
  // and measured half again the panels' load time; batches of four cut that to a quarter.
  // Bytes past the end of a row (K not a multiple of 1024) belong to steps that do not exist.
  // The two 16-byte halves of a row's batch (steps 4b, 4b + 1 and steps 4b + 2, 4b + 3) are
  // swapped in LDS on rows with bit 3 set.  A step's 8-byte reads of 32 consecutive rows (32
  // bytes apart) then fall on 16 distinct 8-byte bank pairs of the 64 banks, two rows each,
  // instead of 8 (rows r and r + 8 share banks).  Lane l writes slot l & 1 of row
  // 32 g + (l >> 1) and so fetches half (l & 1) ^ ((l >> 4) & 1).
  const unsigned vbat = (unsigned)(((lane & 1) ^ ((lane >> 4) & 1)) * 16);
  auto issue_batch = [&](int b) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 8 / NW; ++i) {
      const int g = wave * (8 / NW) + i;  // rows [32 g, 32 g + 32)
      const int r = 32 * g + (lane >> 1);
      const unsigned boff = (unsigned)(b * kBatchRow) + vbat;
      const unsigned la = lds_base + (unsigned)(2 * kBuffer + (b & 1) * kBatch + g * 1024);
      lds_dma16(rsa, la, (unsigned)(m0 + r) * kblk + boff);
      lds_dma16(rsb, la + kBM * kBatchRow, (unsigned)(n0 + r) * kblk + boff);
    }
  };
  auto dma_pieces = [&](int s, int buf, int p0, int p1) __attribute__((always_inline)) {
#pragma unroll
    for (int p = 0; p < NP; ++p)
      if (p >= p0 && p < p1) dma_piece(s, buf, p);
  };
  // Scale words of this lane for one step: A rows wm * FA * 32 + t * 32 + l % 32, B likewise.
  u32x2 scl_a[FA], scl_b[FB];

  f32x16 acc[FA][FB];
#pragma unroll
  for (int i = 0; i < FA; ++i)
#pragma unroll
    for (int j = 0; j < FB; ++j) acc[i][j] = f32x16{};

  const int half = lane >> 5;  // K half of the 64-element MFMA step
  // Fragment t of substep u: row (w? * 128 + t * 32 + l % 32), logical 16-byte column
  // 2u + half, stored at column (2u + half) ^ ((row >> 1) & 7) = (2u + half) ^ ((l >> 1) & 7).
  const int sw = (lane >> 1) & 7;
  const int fa_row = (wm * FA * 32 + (lane & 31)) * kRowBytes;
  const int fb_row = (wn * FB * 32 + (lane & 31)) * kRowBytes;
  struct Frags {
    u32x4 a[FA], b[FB];
  };
  // Reads placed one at a time between MFMAs: fragment t (A 0..FA-1, then B) of substep u,
  // and scale word t (same numbering) of a buffer.
  auto read_item = [&](Frags& f, int buf, int u, int t) __attribute__((always_inline)) {
    const unsigned char* la = lds + buf * kBuffer;
    const int col = ((2 * u + half) ^ sw) * 16;
    if (t < FA) f.a[t < FA ? t : 0] = *(const u32x4*)(la + fa_row + col + t * 32 * kRowBytes);
    else f.b[t < FA ? 0 : t - FA] = *(const u32x4*)(la + kPanel + fb_row + col + (t - FA) * 32 * kRowBytes);
  };
  // Step sn's 8 bytes of row r sit in half ((sn % 4) >> 1) ^ ((r >> 3) & 1) of the row's batch; the
  // rows a lane reads are 32 t + (l & 31) past a multiple of 32, so (r >> 3) & 1 = (l >> 3) & 1.
  const int sq = (lane >> 3) & 1;
  auto scale_item = [&](int sn, int t) __attribute__((always_inline)) {  // scales of step sn
    const int st = sn % kBatchSteps;
    const unsigned char* ls =
        lds + 2 * kBuffer + ((sn / kBatchSteps) & 1) * kBatch + ((st >> 1) ^ sq) * 16 + (st & 1) * 8;
    if (t < FA) scl_a[t < FA ? t : 0] = *(const u32x2*)(ls + (wm * FA * 32 + t * 32 + (lane & 31)) * kBatchRow);
    else scl_b[t < FA ? 0 : t - FA] =
        *(const u32x2*)(ls + kBM * kBatchRow + (wn * FB * 32 + (t - FA) * 32 + (lane & 31)) * kBatchRow);
  };
  auto mfmas = [&](const Frags& f, int u, auto&& hook) __attribute__((always_inline)) {
    // scale of block 2u + half of this step: byte (2u + half) % 4 of word (2u + half) / 4
    const int blk = 2 * u + half;
    int xa[FA], xb[FB];
#pragma unroll
    for (int t = 0; t < FA; ++t) xa[t] = (int)((u < 2 ? scl_a[t][0] : scl_a[t][1]) >> (8 * (blk & 3)));
#pragma unroll
    for (int t = 0; t < FB; ++t) xb[t] = (int)((u < 2 ? scl_b[t][0] : scl_b[t][1]) >> (8 * (blk & 3)));
#pragma unroll
    for (int i = 0; i < FA; ++i)
#pragma unroll
      for (int j = 0; j < FB; ++j) {
        const i32x8 fa = {(int)f.a[i][0], (int)f.a[i][1], (int)f.a[i][2], (int)f.a[i][3], 0, 0, 0, 0};
        const i32x8 fb = {(int)f.b[j][0], (int)f.b[j][1], (int)f.b[j][2], (int)f.b[j][3], 0, 0, 0, 0};
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa, fb, acc[i][j], 4, 4, 0, xa[i], 0, xb[j]);
        hook(i * FB + j);
      }
  };
  // Pipeline.  Step s computes from LDS buffer s & 1 in four 64-element substeps u0..u3
  // whose fragments alternate between f0 and f1.  After each of a substep's FA * FB MFMAs
  // the wave issues an even share of the memory work placed on that substep:
  //   u0 (f0): read f1 <- u1; second half of step s + 1's loads (into the other buffer)
  //   u1 (f1): read f0 <- u2
  //   u2 (f0): read f1 <- u3
  //   wait for this wave's loads of step s + 1, barrier: step s + 1 is complete in the other
  //       buffer and every read of this buffer has been issued and completed
  //   u3 (f1): read the scale words and f0 <- u0 of step s + 1; first half of step s + 2's
  //       loads (into this buffer); on steps s = 4b, scale batch b + 1
  // Each piece of memory work sits between scheduling barriers so that the order holds.  Past
  // the last step the loads re-read step nsteps - 1 into a buffer nobody reads again; the body
  // has no branches.
  constexpr int kMaxItems = 2 * (FA + FB) + NP;
  auto substep = [&](const Frags& fc, int u, Frags& fn, int rbuf, int ru, bool scales, int sn, int ds, int dbuf,
                     int p0, int p1) __attribute__((always_inline)) {
    const int nr = (FA + FB) * (scales ? 2 : 1);
    const int ni = nr + (p1 - p0);
    mfmas(fc, u, [&](int idx) __attribute__((always_inline)) {
#pragma unroll
      for (int it = 0; it < kMaxItems; ++it) {
        if (it < ni && it * FA * FB / ni == idx) {
          __builtin_amdgcn_sched_barrier(0);
          if (it >= nr) dma_piece(ds, dbuf, p0 + it - nr);
          else if (!scales) read_item(fn, rbuf, ru, it);
          else if (it < FA + FB) scale_item(sn, it);  // scales first: the next substep starts with them
          else read_item(fn, rbuf, ru, it - (FA + FB));
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    });
  };
  const int s1 = nsteps > 1 ? 1 : 0;
  issue_batch(0);
  dma_pieces(0, 0, 0, NP);
  dma_pieces(s1, 1, 0, NP / 2);
  wait_lds_dma();
  __syncthreads();
  Frags f0, f1;
  // same order as the loop's u3 reads, so that the waits at the loop head can count
#pragma unroll
  for (int t = 0; t < FA + FB; ++t) {
    __builtin_amdgcn_sched_barrier(0);
    scale_item(0, t);
  }
#pragma unroll
  for (int t = 0; t < FA + FB; ++t) {
    __builtin_amdgcn_sched_barrier(0);
    read_item(f0, 0, 0, t);
  }
  __builtin_amdgcn_sched_barrier(0);
  // One step; ``batch`` (a literal at every call) adds the scale batch load.  The loop is
  // unrolled by the batch length so that the batch load needs no branch: a branch in the
  // body splits the schedule and spilled half the accumulators.
  auto step = [&](int s, int cur, bool batch) __attribute__((always_inline)) {
    const int s1n = s + 1 < nsteps ? s + 1 : nsteps - 1;
    const int s2 = s + 2 < nsteps ? s + 2 : nsteps - 1;
    substep(f0, 0, f1, cur, 1, false, 0, s1n, cur ^ 1, NP / 2, NP);
    substep(f1, 1, f0, cur, 2, false, 0, 0, 0, 0, 0);
    substep(f0, 2, f1, cur, 3, false, 0, 0, 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    wait_lds_dma();  // this wave's loads of step s + 1 (and of a scale batch issued at step s - 1)
    __syncthreads();
    substep(f1, 3, f0, cur ^ 1, 0, true, s + 1, s2, cur, 0, NP / 2);
    __builtin_amdgcn_sched_barrier(0);
    // Batch b + 1 goes to the buffer batch b - 1 used; its last scale reads (step 4b - 1's, in
    // step 4b - 2) are behind this step's barrier.  It is complete after the next step's wait.
    if (batch) issue_batch(s / kBatchSteps + 1);
    __builtin_amdgcn_sched_barrier(0);
  };
  static_assert(kBatchSteps == 4, "the step loop is unrolled by four");
  int s = 0;
  for (; s + kBatchSteps <= nsteps; s += kBatchSteps) {
    step(s, 0, true);
    step(s + 1, 1, false);
    step(s + 2, 0, false);
    step(s + 3, 1, false);
  }
  for (; s < nsteps; ++s) step(s, s & 1, false);  // the last batch was issued by the loop above
  wait_lds_dma();
  __syncthreads();  // the epilogue reuses the operand LDS

  // Epilogue: each 32 x 32 accumulator tile through the wave's LDS block (store_tile32).
  float* ep = (float*)lds + wave * 32 * 36;
  // literal indices keep the accumulators in registers
#define TGM_OUT(I, J)                                                                                 \
  if constexpr (I < FA && J < FB)                                                                     \
    store_tile32(acc[I < FA ? I : 0][J < FB ? J : 0], ep, lane, m0 + wm * FA * 32 + I * 32, n0 + wn * FB * 32 + J * 32, \
                 M, N, c, cdt, ldc);
  TGM_OUT(0, 0) TGM_OUT(0, 1) TGM_OUT(0, 2) TGM_OUT(0, 3) TGM_OUT(1, 0) TGM_OUT(1, 1) TGM_OUT(1, 2) TGM_OUT(1, 3)
  TGM_OUT(2, 0) TGM_OUT(2, 1) TGM_OUT(2, 2) TGM_OUT(2, 3) TGM_OUT(3, 0) TGM_OUT(3, 1) TGM_OUT(3, 2) TGM_OUT(3, 3)
#undef TGM_OUT
}

// ---------------------------------------------------------------------------------------------
// Persistent form for K a multiple of 1024 (kBatchSteps steps of 256): one workgroup per CU walks
// the tiles blockIdx.x, blockIdx.x + G, ... (G = gridDim.x, a multiple of 8, so a workgroup's tiles
// stay on its XCD's contiguous range of tile_of) as one stream of K steps.  The step pipeline of
// gemm_mx_fp4 runs across tile boundaries unchanged: the loads of the next tile's first two
// steps are issued during the current tile's last two, so a tile starts with its operands in LDS
// instead of waiting for them, and no workgroup is launched per tile.  At a tile's end the
// accumulators go to C through the idle scale buffer (see the epilogue) with ordinary stores (in
// one process against non-temporal ones: 251.4 against 253.0 us at 8192^3, 134.0 against 137.4 us
// at 4096 x 14336 x 4096; a round of tiles writes as much C per XCD, 32 x 128 KB, as its L2 holds,
// but a store that completes in L2 holds up the next step's load wait for less time).
template <int WM, int WN>
__global__ void __launch_bounds__(WM * WN * 64) gemm_mx_fp4_stream(const uint8_t* __restrict__ a,
                                                                   const uint8_t* __restrict__ sa,
                                                                   const uint8_t* __restrict__ b,
                                                                   const uint8_t* __restrict__ sb, int M, int N, int K,
                                                                   void* __restrict__ c, int cdt, int64_t ldc) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[kLds];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  constexpr int NW = WM * WN, FA = 8 / WM, FB = 8 / WN;
  constexpr int NI = 32 / NW;
  static_assert(NW == 8, "scale batches are loaded by 8 waves");
  const int wm = wave / WN, wn = wave % WN;
  const int tiles_m = (M + kBM - 1) / kBM, tiles_n = (N + kBN - 1) / kBN;
  const int ntiles = tiles_m * tiles_n;
  const int G = gridDim.x;
  const int my_tiles = (ntiles - (int)blockIdx.x + G - 1) / G;  // >= 1 (the host launches G <= ntiles)
  const int nsteps = K / kBK;                                    // a multiple of kBatchSteps
  const int total = my_tiles * nsteps;                           // this workgroup's stream of steps

  const unsigned kb = (unsigned)(K / 2);
  const unsigned kblk = (unsigned)(K / 32);
  const i32x4v ra = buffer_rsrc(a, (unsigned)M * kb), rb = buffer_rsrc(b, (unsigned)N * kb);
  const i32x4v rsa = buffer_rsrc(sa, (unsigned)M * kblk), rsb = buffer_rsrc(sb, (unsigned)N * kblk);
  const int lrow = wave * (256 / NW) + (lane >> 3);
  const unsigned lcol = (unsigned)(((lane & 7) ^ (lane >> 4)) * 16);
  const unsigned lane_a = (unsigned)lrow * kb + lcol;  // + tile row offset, step offset, 8 i kb
  const unsigned lds_base = (unsigned)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)lds;
  // (first row, first column) of this workgroup's t-th tile
  auto tile_origin = [&](int t, int& m0, int& n0) __attribute__((always_inline)) {
    int tm, tn;
    tile_of((int)blockIdx.x + t * G, tiles_m, tiles_n, kGroupM, tm, tn);
    m0 = tm * kBM;
    n0 = tn * kBN;
  };
  // Origins of the current tile (t) and the next (t + 1, or t itself for the last), looked up once
  // per tile: the steps whose loads are issued during tile t belong to one of the two.
  struct Tiles {
    int t, base;        // tile index and its first stream step (t * nsteps)
    int mc, nc, mn, nn;  // (row, column) origins of tiles t and t + 1
  } tl;
  auto set_tile = [&](int t) __attribute__((always_inline)) {
    tl.t = t;
    tl.base = t * nsteps;
    tile_origin(t, tl.mc, tl.nc);
    tile_origin(t + 1 < my_tiles ? t + 1 : t, tl.mn, tl.nn);
    tl.mc = __builtin_amdgcn_readfirstlane(tl.mc);
    tl.nc = __builtin_amdgcn_readfirstlane(tl.nc);
    tl.mn = __builtin_amdgcn_readfirstlane(tl.mn);
    tl.nn = __builtin_amdgcn_readfirstlane(tl.nn);
  };
  // (tile row origin, tile column origin, step within the tile) of stream step gs, clamped to the
  // stream; gs lies in tile tl.t or tl.t + 1
  struct StepAt {
    int m0, n0, st;
  };
  auto step_at = [&](int gs) __attribute__((always_inline)) {
    gs = gs < total ? gs : total - 1;
    const int local = gs - tl.base;
    return local < nsteps ? StepAt{tl.mc, tl.nc, local} : StepAt{tl.mn, tl.nn, local - nsteps};
  };
  // uniform byte offsets of stream step gs in A and B
  struct StepOff {
    unsigned a, b;
  };
  auto step_off = [&](int gs) __attribute__((always_inline)) {
    const StepAt at = step_at(gs);
    return StepOff{(unsigned)__builtin_amdgcn_readfirstlane((int)((unsigned)at.m0 * kb + (unsigned)(at.st * kRowBytes))),
                   (unsigned)__builtin_amdgcn_readfirstlane((int)((unsigned)at.n0 * kb + (unsigned)(at.st * kRowBytes)))};
  };
  constexpr int NP = 2 * NI;
  auto dma_piece = [&](const StepOff& o, int buf, int p) __attribute__((always_inline)) {
    const int i = p >> 1;
    const unsigned col_flip = (unsigned)((i & 1) * 64);
    const unsigned la = lds_base + (unsigned)(buf * kBuffer + (p & 1) * kPanel + wave * (2048 / NW) * 16 + i * 1024);
    const unsigned v = (lane_a ^ col_flip) + (unsigned)(8 * i) * kb + ((p & 1) ? o.b : o.a);
    lds_dma16((p & 1) ? rb : ra, la, v);
  };
  const unsigned vbat = (unsigned)(((lane & 1) ^ ((lane >> 4) & 1)) * 16);
  // scale batch gb of the stream (steps 4 gb .. 4 gb + 3, all of one tile since nsteps % 4 == 0)
  auto issue_batch = [&](int gb) __attribute__((always_inline)) {
    const int gs = gb * kBatchSteps < total ? gb * kBatchSteps : total - kBatchSteps;
    const StepAt at = step_at(gs);  // the batch's first step; all four are in one tile
    const int g = wave;             // rows [32 g, 32 g + 32)
    const int r = 32 * g + (lane >> 1);
    const unsigned boff = (unsigned)(at.st / kBatchSteps * kBatchRow) + vbat;
    const unsigned la = lds_base + (unsigned)(2 * kBuffer + (gb & 1) * kBatch + g * 1024);
    lds_dma16(rsa, la, (unsigned)(at.m0 + r) * kblk + boff);
    lds_dma16(rsb, la + kBM * kBatchRow, (unsigned)(at.n0 + r) * kblk + boff);
  };
  auto dma_pieces = [&](int gs, int buf, int p0, int p1) __attribute__((always_inline)) {
    const StepOff o = step_off(gs);
#pragma unroll
    for (int p = 0; p < NP; ++p)
      if (p >= p0 && p < p1) dma_piece(o, buf, p);
  };
  // E8M0 bytes of the lane's row for one step: the 8 blocks as read from LDS (raw), then the four
  // blocks 2 u + half (u = 0 .. 3) of the lane's K half packed into one word per fragment, whose byte
  // u the MFMA of substep u selects itself (op_sel), so no instruction sits between a scale and its use
  u32x2 sraw_a[FA], sraw_b[FB];
  unsigned sw_a[FA], sw_b[FB];
  f32x16 acc[FA][FB];
#pragma unroll
  for (int i = 0; i < FA; ++i)
#pragma unroll
    for (int j = 0; j < FB; ++j) acc[i][j] = f32x16{};

  const int half = lane >> 5;
  const int sw = (lane >> 1) & 7;
  const int fa_row = (wm * FA * 32 + (lane & 31)) * kRowBytes;
  const int fb_row = (wn * FB * 32 + (lane & 31)) * kRowBytes;
  struct Frags {
    u32x4 a[FA], b[FB];
  };
  auto read_item = [&](Frags& f, int buf, int u, int t) __attribute__((always_inline)) {
    const unsigned char* la = lds + buf * kBuffer;
    const int col = ((2 * u + half) ^ sw) * 16;
    if (t < FA) f.a[t < FA ? t : 0] = *(const u32x4*)(la + fa_row + col + t * 32 * kRowBytes);
    else f.b[t < FA ? 0 : t - FA] = *(const u32x4*)(la + kPanel + fb_row + col + (t - FA) * 32 * kRowBytes);
  };
  const int sq = (lane >> 3) & 1;
  auto scale_item = [&](int sn, int t) __attribute__((always_inline)) {  // raw scales of stream step sn
    const int st = sn % kBatchSteps;
    const unsigned char* ls =
        lds + 2 * kBuffer + ((sn / kBatchSteps) & 1) * kBatch + ((st >> 1) ^ sq) * 16 + (st & 1) * 8;
    if (t < FA) sraw_a[t < FA ? t : 0] = *(const u32x2*)(ls + (wm * FA * 32 + t * 32 + (lane & 31)) * kBatchRow);
    else sraw_b[t < FA ? 0 : t - FA] =
        *(const u32x2*)(ls + kBM * kBatchRow + (wn * FB * 32 + (t - FA) * 32 + (lane & 31)) * kBatchRow);
  };
  // bytes half, 2 + half (word 0) and half, 2 + half (word 1) of the raw pair: blocks 2 u + half
  const unsigned ssel = half ? 0x07050301u : 0x06040200u;
  auto scale_word = [&](int t) __attribute__((always_inline)) {
    if (t < FA) sw_a[t < FA ? t : 0] = __builtin_amdgcn_perm(sraw_a[t < FA ? t : 0][1], sraw_a[t < FA ? t : 0][0], ssel);
    else sw_b[t < FA ? 0 : t - FA] = __builtin_amdgcn_perm(sraw_b[t < FA ? 0 : t - FA][1], sraw_b[t < FA ? 0 : t - FA][0], ssel);
  };
  auto mfmas = [&](const Frags& f, auto uc, auto&& hook) __attribute__((always_inline)) {
    constexpr int u = decltype(uc)::value;  // the MFMA's scale byte select
    unsigned xa[FA], xb[FB];                // this substep's words (the hook may write the next step's)
#pragma unroll
    for (int t = 0; t < FA; ++t) xa[t] = sw_a[t];
#pragma unroll
    for (int t = 0; t < FB; ++t) xb[t] = sw_b[t];
#pragma unroll
    for (int i = 0; i < FA; ++i)
#pragma unroll
      for (int j = 0; j < FB; ++j) {
        const i32x8 fa = {(int)f.a[i][0], (int)f.a[i][1], (int)f.a[i][2], (int)f.a[i][3], 0, 0, 0, 0};
        const i32x8 fb = {(int)f.b[j][0], (int)f.b[j][1], (int)f.b[j][2], (int)f.b[j][3], 0, 0, 0, 0};
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa, fb, acc[i][j], 4, 4, u, (int)xa[i], u,
                                                                    (int)xb[j]);
        hook(i * FB + j);
      }
  };
  // Substep u's items, one after each MFMA share, in this order: the fragment reads of the next
  // substep (from buffer rbuf), then with ``rs`` the raw E8M0 bytes of stream step sn, then load
  // pieces [p0, p1) into buffer dbuf, then with ``words`` the scale words of the step just read.
  constexpr int kMaxItems = 3 * (FA + FB) + NP;
  auto substep = [&](const Frags& fc, auto uc, Frags& fn, int rbuf, int ru, bool rs, int sn, bool words,
                     const StepOff* lo, int dbuf, int p0, int p1) __attribute__((always_inline)) {
    const int nf = FA + FB;
    const int nr = nf + (rs ? FA + FB : 0);
    const int nd = nr + (p1 - p0);
    const int ni = nd + (words ? FA + FB : 0);
    mfmas(fc, uc, [&](int idx) __attribute__((always_inline)) {
#pragma unroll
      for (int it = 0; it < kMaxItems; ++it) {
        if (it < ni && it * FA * FB / ni == idx) {
          __builtin_amdgcn_sched_barrier(0);
          if (it >= nd) scale_word(it - nd);
          else if (it >= nr) dma_piece(*lo, dbuf, p0 + it - nr);
          else if (it >= nf) scale_item(sn, it - nf);
          else read_item(fn, rbuf, ru, it);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    });
  };
  using U0 = std::integral_constant<int, 0>;
  using U1 = std::integral_constant<int, 1>;
  using U2 = std::integral_constant<int, 2>;
  using U3 = std::integral_constant<int, 3>;
  set_tile(0);
  issue_batch(0);
  dma_pieces(0, 0, 0, NP);
  dma_pieces(1, 1, 0, NP / 2);
  wait_lds_dma();
  __syncthreads();
  Frags f0, f1;
#pragma unroll
  for (int t = 0; t < FA + FB; ++t) {
    __builtin_amdgcn_sched_barrier(0);
    scale_item(0, t);
  }
#pragma unroll
  for (int t = 0; t < FA + FB; ++t) {
    __builtin_amdgcn_sched_barrier(0);
    read_item(f0, 0, 0, t);
  }
#pragma unroll
  for (int t = 0; t < FA + FB; ++t) scale_word(t);
  __builtin_amdgcn_sched_barrier(0);
  // Step gs from buffer cur:
  //   u0 (f0): read f1 <- u1; second half of step gs + 1's loads (into the other buffer)
  //   u1 (f1): read f0 <- u2; the raw E8M0 bytes of step gs + 1.  Its batch is complete (a batch is
  //       issued four steps ahead of its first step and waited for by the step after that), and
  //       the batch that will overwrite a buffer is issued only after the barrier of the step whose
  //       scales it last held were read two steps before, so the reads need no barrier of their own
  //       and stay out of the burst of reads that follows the step barrier
  //   u2 (f0): read f1 <- u3
  //   wait for this wave's loads of step gs + 1, barrier
  //   u3 (f1): read f0 <- u0 of step gs + 1 (other buffer); first half of step gs + 2's loads (into
  //       this buffer); the scale words of step gs + 1
  auto step = [&](int gs, int cur, bool batch) __attribute__((always_inline)) {
    const StepOff o1 = step_off(gs + 1), o2 = step_off(gs + 2);
    substep(f0, U0{}, f1, cur, 1, false, 0, false, &o1, cur ^ 1, NP / 2, NP);
    substep(f1, U1{}, f0, cur, 2, true, gs + 1, false, &o1, 0, 0, 0);
    substep(f0, U2{}, f1, cur, 3, false, 0, false, &o1, 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    wait_lds_dma();
    __syncthreads();
    substep(f1, U3{}, f0, cur ^ 1, 0, false, 0, true, &o2, cur, 0, NP / 2);
    __builtin_amdgcn_sched_barrier(0);
    if (batch) issue_batch(gs / kBatchSteps + 1);
    __builtin_amdgcn_sched_barrier(0);
  };
  static_assert(kBatchSteps == 4, "the step loop is unrolled by four");
  int gs = 0;
  for (int t = 0; t < my_tiles; ++t) {
    set_tile(t);
    for (int s = 0; s < nsteps; s += kBatchSteps, gs += kBatchSteps) {
      step(gs, 0, true);
      step(gs + 1, 1, false);
      step(gs + 2, 0, false);
      step(gs + 3, 1, false);
    }
    // Tile t is complete in the accumulators (MFMA D layout: lane l holds column l % 32 and rows
    // 8 (v / 4) + 4 (l / 32) + v % 4 of each 32 x 32 tile).  The scale buffer of the tile's last
    // batch is idle from the last step's barrier until the next tile's first step issues its
    // second batch into it (after that step's barrier, which every wave reaches only after this
    // epilogue): each wave turns its 32 x 32 tiles, rounded to 16 bits, into rows through its 2 KB
    // of that buffer and stores 16-byte row segments.  fp32 output goes out per element.
    const int col0 = tl.nc + wn * FB * 32;
    const int row0 = tl.mc + wm * FA * 32;
    unsigned short* ep = (unsigned short*)(lds + 2 * kBuffer + (((gs - 1) / kBatchSteps) & 1) * kBatch) + wave * 1024;
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
                *(u32x4*)out = *(const u32x4*)(ep + r * 32 + cc);
              } else {  // the ragged edge, element by element from LDS (a rolled loop holds no row in VGPRs)
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

}  // namespace tgm

using namespace tgm;

extern "C" int tgm_gemm_mx(const void* a, int a_fmt, const void* a_scales, int64_t m, const void* b, int b_fmt,
                           const void* b_scales, int64_t n, int64_t k, void* c, int c_dtype, int64_t ldc,
                           void* stream) {
  clear_error();
  TGM_CHECK_ARG(valid_format(a_fmt) && valid_format(b_fmt), "unknown packed format");
  TGM_CHECK_ARG(a && b && c, "null operand");
  TGM_CHECK_ARG(m >= 0 && n >= 0 && k >= 0, "invalid gemm sizes");
  TGM_CHECK_ARG(c_dtype == TGM_BF16 || c_dtype == TGM_F16 || c_dtype == TGM_F32, "output must be bf16, f16 or f32");
  TGM_CHECK_ARG(m <= 1 || ldc >= n, "ldc smaller than N");
  if (m == 0 || n == 0) return TGM_OK;
  const int ta = f8f6f4_code_of_format(a_fmt), tb = f8f6f4_code_of_format(b_fmt);
  if (ta < 0 || tb < 0) TGM_UNSUPPORTED("tgm_gemm_mx: the scaled MFMA takes FP4 and FP6 codes, not integers");
  const bool fp4_pair = a_fmt == TGM_FMT_FP4_E2M1 && b_fmt == TGM_FMT_FP4_E2M1 && a_scales && b_scales;
  if (!fp4_pair || k == 0 || k % kBK != 0) {
    // every other FP4 / FP6 pair (or K a multiple of 128 only): the general scaled-MFMA kernel
    const int64_t rba = k / 8 * (a_fmt == TGM_FMT_FP4_E2M1 ? 4 : 6), rbb = k / 8 * (b_fmt == TGM_FMT_FP4_E2M1 ? 4 : 6);
    return launch_f8f6f4((hipStream_t)stream, ta, a, rba, a_scales, m, tb, b, rbb, b_scales, n, k, c, c_dtype, ldc,
                         "tgm_gemm_mx");
  }
  if (m >= (1ll << 31) || n >= (1ll << 31) || m * (k / 2) >= (1ll << 32) || n * (k / 2) >= (1ll << 32))
    TGM_UNSUPPORTED("tgm_gemm_mx: operands must be under 4 GiB (32-bit offsets)");
  if ((uintptr_t)a % 16 || (uintptr_t)b % 16 || (uintptr_t)a_scales % 8 || (uintptr_t)b_scales % 8)
    TGM_UNSUPPORTED("tgm_gemm_mx: operands must be 16-byte and scales 8-byte aligned");
  const int64_t tiles = ((m + kBM - 1) / kBM) * ((n + kBN - 1) / kBN);
  const int cus = stream_cu_count((hipStream_t)stream);
  if (k % (kBK * kBatchSteps) == 0 && cus >= 8 && tiles >= 8) {
    // persistent: one workgroup per CU (a multiple of 8 of them, so each keeps to its XCD's tiles)
    const int64_t grid = tiles < cus ? tiles / 8 * 8 : cus / 8 * 8;
    hipLaunchKernelGGL((gemm_mx_fp4_stream<kWavesM, kWavesN>), dim3((unsigned)grid), dim3(kWavesM * kWavesN * 64), 0,
                       (hipStream_t)stream, (const uint8_t*)a, (const uint8_t*)a_scales, (const uint8_t*)b,
                       (const uint8_t*)b_scales, (int)m, (int)n, (int)k, c, c_dtype, ldc);
    return launch_status("tgm_gemm_mx");
  }
  // 4 x 2 waves of 64 x 128: two waves per SIMD hide each other's LDS and barrier latency
  hipLaunchKernelGGL((gemm_mx_fp4<kWavesM, kWavesN>), dim3((unsigned)tiles), dim3(kWavesM * kWavesN * 64), 0, (hipStream_t)stream, (const uint8_t*)a,
                     (const uint8_t*)a_scales, (const uint8_t*)b, (const uint8_t*)b_scales, (int)m, (int)n, (int)k, c,
                     c_dtype, ldc);
  return launch_status("tgm_gemm_mx");
}
