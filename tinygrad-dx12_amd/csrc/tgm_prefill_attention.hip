// Causal prompt attention in one kernel (flash-attention form) on bf16 MFMA, with the accuracy
// of fp32 arithmetic.
//
// For every (sequence, q head) and prompt token t at position p = pos[b] + t:
//
//   out[t] = sum_{k <= p} softmax_k(q_t . K_k / sqrt(hd)) V_k        (K, V: the bf16 cache)
//
// The scores and probabilities never leave the chip.  A workgroup takes 128 prompt tokens of
// one (sequence, head), 32 per wave, and walks the cache in blocks of 64 keys up to its last
// token's position.  The products are computed transposed, so that everything a query owns
// sits in one lane (the 32x32 MFMA D layout gives lane l column l % 32):
//
//   S^T[key, query]  = K . Q^T       A = the K block (LDS),     B = q (registers)
//   O^T[dim, query] += V^T . P^T     A = the V^T block (LDS),   B = p (registers)
//
// Accuracy: q (scaled by log2(e) / sqrt(hd), so that the softmax runs on exp2) and each
// probability are split into three bf16 terms
// x = t0 + t1 + t2 (t0 = bf16(x), each later term the bf16 of what the earlier ones leave;
// three terms hold the 24 bits of an fp32 value) and every term meets the bf16 K or V
// operand in its own MFMA.  Products of bf16 values are exact in fp32, so S and O carry only
// fp32 accumulation error, like an fp32 kernel.  The softmax is online per lane in fp32.
//
// D layout and the probability operand: lane (query, half h) holds S^T rows (keys)
// 8 (v / 4) + 4 h + v % 4 of each 32-key tile, v = 0 .. 15.  The P . V MFMA u of a tile
// (16 keys) takes the lane's values v = 8 u .. 8 u + 7 as its B operand, i.e. keys
// 16 u + 4 h + {0..3} and 16 u + 8 + 4 h + {0..3}; the V^T operand reads the same keys (two
// 8-byte pieces of a V^T row), so both sides agree on which key each product belongs to.
//
// LDS (double buffered, one barrier per key block): the K block as 64 rows of hd bf16 with
// 16-byte chunks XOR-swizzled by the row; V^T as hd rows of 64 keys with 8-byte chunks
// XOR-swizzled by (row / 2) % 16, written transposed from the loaded V rows.  The next
// block's global loads are in flight while the current block is computed.
#include <math.h>

#include "../../include/tgm_decoder.h"
#include "tgm_mfma_common.h"

namespace tgm {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 pa_bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 pa_bf16x4;
typedef _Float16 pa_f16x4 __attribute__((ext_vector_type(4)));

constexpr int kPaKeys = 64;      // keys per block
constexpr int kPaQueries = 128;  // prompt tokens per workgroup (32 per wave)
constexpr int kPaTerms = 3;      // bf16 terms per fp32 operand value

// The three bf16 terms of 8 fp32 values.
__device__ __forceinline__ void pa_split(float (&r)[8], pa_bf16x8 (&t)[kPaTerms]) {
#pragma unroll
  for (int s = 0; s < kPaTerms; ++s) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const __bf16 v = (__bf16)r[i];  // round to nearest even
      t[s][i] = v;
      r[i] -= (float)v;  // exact: the residual has at most 16 significant bits
    }
  }
}

// Grid (ceil(T / 128), heads, batch), 256 threads.
template <int HD>
__global__ void __launch_bounds__(256) dec_prefill_attention(const float* __restrict__ qkv, int T, int H, int HK,
                                                             const int32_t* __restrict__ pos,
                                                             const uint16_t* __restrict__ kc,
                                                             const uint16_t* __restrict__ vc, int max_seq, float scale,
                                                             void* __restrict__ out, int odt) {
  constexpr int NJ = HD / 16;                         // 16-wide steps of q . k
  constexpr int ND = HD / 32;                         // 32-row tiles of O^T
  constexpr int KROW = HD * 2, KCH = KROW / 16;       // K block: 64 rows of HD bf16, KCH 16-byte chunks each
  constexpr int VROW = kPaKeys * 2;                   // V^T block: HD rows of 64 bf16
  constexpr int KBYTES = kPaKeys * KROW, STAGE = KBYTES + HD * VROW;
  constexpr int NLD = kPaKeys * KCH / 256;            // 16-byte chunks per thread and block, for K and for V
  static_assert(NLD * 256 == kPaKeys * KCH, "block loads");
  __shared__ __attribute__((aligned(16))) unsigned char lds[2 * STAGE];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, half = lane >> 5, l32 = lane & 31;
  const int h = blockIdx.y, b = blockIdx.z, j = h / (H / HK);
  const int p0 = pos[b];
  const int64_t ld = (int64_t)(H + 2 * HK) * HD;
  // the longest query blocks (the last tokens, which see the most keys) are launched first
  const int qblk = (int)(gridDim.x - 1 - blockIdx.x);
  const int tq = qblk * kPaQueries + wave * 32 + l32;  // this lane's prompt token
  const bool qvalid = tq < T;
  const int tqc = qvalid ? tq : T - 1;
  const int qpos = p0 + tqc;
  const int t_end = min(qblk * kPaQueries + kPaQueries, T);
  const int nkeys = min(p0 + t_end, max_seq);                 // keys 0 .. nkeys - 1 serve the workgroup
  const int nblocks = nkeys > 0 ? (nkeys + kPaKeys - 1) / kPaKeys : 0;
  const int wave_end = min(qblk * kPaQueries + wave * 32 + 32, T);
  const int wave_maxpos = p0 + wave_end - 1;                  // blocks past it are masked for every lane
  const int wave_minpos = p0 + min(qblk * kPaQueries + wave * 32, T - 1);  // blocks up to it need no mask
  const uint16_t* kbase = kc + ((int64_t)b * HK + j) * max_seq * HD;
  const uint16_t* vbase = vc + ((int64_t)b * HK + j) * max_seq * HD;

  // q terms as the B operand of S^T: lane (query, half) holds q[16 s + 8 half + i] * scale.
  pa_bf16x8 qt[NJ][kPaTerms];
  {
    const float* qrow = qkv + ((int64_t)b * T + tqc) * ld + (int64_t)h * HD;
#pragma unroll
    for (int s = 0; s < NJ; ++s) {
      const f32x4 x0 = *(const f32x4*)(qrow + 16 * s + 8 * half);
      const f32x4 x1 = *(const f32x4*)(qrow + 16 * s + 8 * half + 4);
      const float sl = scale * 1.4426950408889634f;  // log2(e): the softmax runs on exp2
      float r[8] = {x0[0] * sl, x0[1] * sl, x0[2] * sl, x0[3] * sl, x1[0] * sl, x1[1] * sl, x1[2] * sl, x1[3] * sl};
      pa_split(r, qt[s]);
    }
  }

  u32x4 kreg[NLD], vreg[NLD];
  auto load_regs = [&](int kb) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      const int c = tid + 256 * i, key = c / KCH, ch = c % KCH;
      const int kk = min(kb * kPaKeys + key, max_seq - 1);  // keys past the cache are masked
      kreg[i] = *(const u32x4*)(kbase + (int64_t)kk * HD + ch * 8);
      vreg[i] = *(const u32x4*)(vbase + (int64_t)kk * HD + ch * 8);
    }
  };
  auto store_lds = [&](int buf) __attribute__((always_inline)) {
    unsigned char* st = lds + buf * STAGE;
    unsigned char* vt = st + KBYTES;
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      const int c = tid + 256 * i, key = c / KCH, ch = c % KCH;
      *(u32x4*)(st + key * KROW + ((ch ^ (key & (KCH - 1))) * 16)) = kreg[i];
      const int c8 = key >> 2, sub = (key & 3) * 2;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int d = ch * 8 + e;
        *(uint16_t*)(vt + d * VROW + ((c8 ^ ((d >> 1) & 15)) * 8) + sub) = (uint16_t)(vreg[i][e >> 1] >> (16 * (e & 1)));
      }
    }
  };

  f32x16 O[ND];
#pragma unroll
  for (int dt = 0; dt < ND; ++dt) O[dt] = f32x16{};
  float m = -INFINITY, l = 0.f;
  if (nblocks > 0) {
    load_regs(0);
    store_lds(0);
  }
  __syncthreads();
  for (int kb = 0; kb < nblocks; ++kb) {
    if (kb + 1 < nblocks) load_regs(kb + 1);
    const unsigned char* st = lds + (kb & 1) * STAGE;
    const unsigned char* vt = st + KBYTES;
    if (kb * kPaKeys <= wave_maxpos) {  // uniform over the wave
      f32x16 S[2] = {f32x16{}, f32x16{}};
#pragma unroll
      for (int s = 0; s < NJ; ++s)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
          const int key = kt * 32 + l32;
          const pa_bf16x8 a = *(const pa_bf16x8*)(st + key * KROW + (((2 * s + half) ^ (key & (KCH - 1))) * 16));
#pragma unroll
          for (int t = 0; t < kPaTerms; ++t) S[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qt[s][t], S[kt], 0, 0, 0);
        }
      // online softmax of this lane's query over the block (the lane pair l, l ^ 32 holds it)
      // (scores are in log2 units: q carries scale * log2(e))
      if (kb * kPaKeys + kPaKeys - 1 > wave_minpos) {  // the block reaches past some query: mask (uniform)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int key = kb * kPaKeys + kt * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
            if (key > qpos) S[kt][v] = -INFINITY;
          }
      }
      float bm = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int v = 0; v < 16; ++v) bm = fmaxf(bm, S[kt][v]);
      bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
      const float mn = fmaxf(m, bm);  // finite: block 0 holds key 0 <= qpos
      float ls = 0.f;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float p = exp2f(S[kt][v] - mn);  // 0 for masked keys
          S[kt][v] = p;
          ls += p;
        }
      if (__any(mn != m)) {  // some lane's maximum moved: rescale (a wave-uniform branch)
        const float alpha = m == -INFINITY ? 0.f : exp2f(m - mn);
        l *= alpha;
#pragma unroll
        for (int dt = 0; dt < ND; ++dt)
#pragma unroll
          for (int v = 0; v < 16; ++v) O[dt][v] *= alpha;
      }
      l += ls;
      m = mn;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          float r[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) r[i] = S[kt][8 * u + i];
          pa_bf16x8 pb[kPaTerms];
          pa_split(r, pb);
          const int c8 = kt * 8 + u * 4 + half;  // keys 16 u + 4 h .. + 4 of tile kt; + 2: the next 8
#pragma unroll
          for (int dt = 0; dt < ND; ++dt) {
            const int d = dt * 32 + l32;
            const unsigned char* row = vt + d * VROW;
            const pa_bf16x4 lo = *(const pa_bf16x4*)(row + ((c8 ^ ((d >> 1) & 15)) * 8));
            const pa_bf16x4 hi = *(const pa_bf16x4*)(row + (((c8 + 2) ^ ((d >> 1) & 15)) * 8));
            const pa_bf16x8 a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
            for (int t = 0; t < kPaTerms; ++t) O[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb[t], O[dt], 0, 0, 0);
          }
        }
    }
    if (kb + 1 < nblocks) store_lds((kb + 1) & 1);
    __syncthreads();
  }
  l += __shfl_xor(l, 32, 64);
  if (!qvalid) return;
  const float inv = 1.0f / l;
  const int64_t o = ((int64_t)b * T + tq) * H * HD + (int64_t)h * HD;
#pragma unroll
  for (int dt = 0; dt < ND; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int64_t e = o + dt * 32 + 8 * g + 4 * half;  // dims 8 g + 4 h .. + 4 of tile dt
      if (odt == TGM_F16) {
        *(pa_f16x4*)((_Float16*)out + e) = pa_f16x4{(_Float16)(O[dt][4 * g] * inv), (_Float16)(O[dt][4 * g + 1] * inv),
                                                    (_Float16)(O[dt][4 * g + 2] * inv), (_Float16)(O[dt][4 * g + 3] * inv)};
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) store_from_f32(out, odt, e + i, O[dt][4 * g + i] * inv);
      }
    }
}

}  // namespace tgm

using namespace tgm;

extern "C" int tgm_dec_prefill_attention(const float* qkv, int64_t rows, int64_t seq_rows, int64_t heads,
                                         int64_t kv_heads, int64_t head_dim, const int32_t* pos, const void* k_cache,
                                         const void* v_cache, int64_t max_seq, void* out, int out_dtype, void* stream) {
  clear_error();
  TGM_CHECK_ARG(qkv && pos && k_cache && v_cache && out, "null operand");
  TGM_CHECK_ARG(rows >= 0 && seq_rows > 0 && rows % seq_rows == 0, "rows must be a multiple of seq_rows");
  TGM_CHECK_ARG(heads > 0 && kv_heads > 0 && heads % kv_heads == 0, "heads must be a multiple of kv_heads");
  TGM_CHECK_ARG(out_dtype == TGM_F16 || out_dtype == TGM_BF16 || out_dtype == TGM_F32, "output must be f16, bf16 or f32");
  TGM_CHECK_ARG(max_seq > 0 && max_seq < (1 << 30) && rows < (1ll << 31), "invalid sizes");
  TGM_CHECK_ARG(heads <= 65535 && rows / seq_rows <= 65535, "at most 65535 heads and sequences");
  if (head_dim != 64 && head_dim != 128) TGM_UNSUPPORTED("tgm_dec_prefill_attention: head_dim must be 64 or 128");
  if ((uintptr_t)qkv % 16 || (uintptr_t)k_cache % 16 || (uintptr_t)v_cache % 16 ||
      (out_dtype == TGM_F16 && (uintptr_t)out % 8))
    TGM_UNSUPPORTED("tgm_dec_prefill_attention: qkv and the caches must be 16-byte aligned, f16 output 8-byte");
  if (rows == 0) return TGM_OK;
  const dim3 grid((unsigned)((seq_rows + kPaQueries - 1) / kPaQueries), (unsigned)heads, (unsigned)(rows / seq_rows));
  const float scale = (float)(1.0 / sqrt((double)head_dim));
  const hipStream_t st = (hipStream_t)stream;
  if (head_dim == 64)
    hipLaunchKernelGGL(dec_prefill_attention<64>, grid, dim3(256), 0, st, qkv, (int)seq_rows, (int)heads,
                       (int)kv_heads, pos, (const uint16_t*)k_cache, (const uint16_t*)v_cache, (int)max_seq, scale, out,
                       out_dtype);
  else
    hipLaunchKernelGGL(dec_prefill_attention<128>, grid, dim3(256), 0, st, qkv, (int)seq_rows, (int)heads,
                       (int)kv_heads, pos, (const uint16_t*)k_cache, (const uint16_t*)v_cache, (int)max_seq, scale, out,
                       out_dtype);
  return launch_status("tgm_dec_prefill_attention");
}
