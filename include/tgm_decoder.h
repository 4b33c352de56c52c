/*
 * Decoder-step kernels around the packed matmul path (libtgm_mi355x.so).
 *
 * The reference has no model code: a decoder built on it would be ordinary tinygrad ops
 * plus PackedTensor.matmul (alexandreteles/tinygrad-dx12 src/tinygrad_dx12/codegen/decomp/
 * dx12.py:108-112, with block_size=128 allowed by dx12.py:30 and :44-47).  These entry
 * points are the non-matmul operations of a Llama-style decoder layer, written for gfx950
 * so that a whole decode step runs on the device:
 *
 *   embed -> [add + RMSNorm -> QKV (INT4 GEMV/GEMM) -> RoPE + KV store -> attention
 *             -> O (INT4) -> add + RMSNorm -> gate|up (FP4) -> SwiGLU -> down (FP4)] x L
 *         -> add + RMSNorm -> output head (bf16 GEMV) -> greedy argmax
 *
 * Sequence positions live in device memory (``pos``, int32 per sequence) and the argmax
 * advances them, so the launches of one decode step do not change from step to step and can
 * be captured once and replayed as a HIP graph.  None of these entry points allocates memory
 * or issues a memset.
 *
 * Layouts (row-major, element strides):
 *   rows         = batch * seq_rows tokens; row r is token r % seq_rows of sequence r / seq_rows
 *   h            = float32 [rows, d] residual stream
 *   qkv          = float32 [rows, (heads + 2 * kv_heads) * head_dim]: q heads, k heads, v heads
 *   k/v caches   = bfloat16 [batch, kv_heads, max_seq, head_dim]
 * Token r of sequence b has position pos[b] + r % seq_rows.
 *
 * Every function returns TGM_OK or a negative tgm_status (message in tgm_last_error()).
 */
#ifndef TGM_DECODER_H
#define TGM_DECODER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* h[r, :] = float(table[tokens[r], :]); table is BF16 [vocab, d] with d a multiple of 8, table
 * and h 16-byte aligned.  Tokens outside [0, vocab) read row 0 (the host validates prompts;
 * generated tokens are in range). */
int tgm_dec_embed(const void* table, int64_t vocab, int64_t d, const int32_t* tokens, int64_t rows, float* h,
                  void* stream);

/* h[r] += delta[r] (delta may be NULL); out[r, i] = h[r, i] / sqrt(mean_i(h[r, i]^2) + eps) * weight[i],
 * computed in fp32 and rounded once to out_dtype (F16, BF16 or F32).  weight is BF16 [d]; d is a
 * multiple of 4 and at most 16384; h, delta and out are 16-byte and weight 8-byte aligned. */
int tgm_dec_add_rmsnorm(float* h, const float* delta, int64_t rows, int64_t d, const void* weight, float eps,
                        void* out, int out_dtype, void* stream);

/* tgm_dec_add_rmsnorm with the residual update given as nparts fp32 parts (part p at
 * parts + p * part_stride floats, each [rows, d]; 1 <= nparts <= 64, part_stride a multiple of 4
 * and at least rows * d): h[r] += parts_0[r] + parts_1[r] + ... (summed in part order), then the
 * same norm.  The parts are what tgm_dec_gemv_parts writes.  The reference has no model code
 * (decoder harness). */
int tgm_dec_add_rmsnorm_parts(float* h, const float* parts, int64_t nparts, int64_t part_stride, int64_t rows,
                              int64_t d, const void* weight, float eps, void* out, int out_dtype, void* stream);

/* A packed GEMV with its K sum cut into `slices` equal slices K_z (k a multiple of 128 * slices,
 * 1 <= slices <= 64): parts + z * m * ldp receives the fp32 [m, ldp] product x[:, K_z] .
 * deq(w[:, K_z])^T, for a consumer that adds the parts (tgm_dec_add_rmsnorm_parts).  FP4 / FP6
 * weights with E8M0/32 (or no) scales, bf16 x [m, ldx], 1 <= m <= 16, operands aligned as for
 * tgm_gemv; otherwise TGM_E_UNSUPPORTED.  For a projection with few output rows and a long K
 * (a decoder's down projection, 4096 x 14336, at 2-16 tokens) each workgroup then stages one
 * slice of x for 64 rows instead of all of x for 16.  The reference has no model code (decoder
 * harness). */
int tgm_dec_gemv_parts(const void* w, int fmt, int64_t n, int64_t k, const void* scales, int scale_dtype,
                       int64_t block_size, const void* x, int x_dtype, int64_t m, int64_t ldx, float* parts,
                       int64_t ldp, int64_t slices, void* stream);

/* Rotary position embedding (rotate-half pairs (i, i + head_dim / 2), angle p * base^(-2 i /
 * head_dim)) applied in place to the q and k heads of qkv; the rotated k heads and the v heads
 * are stored as bf16 into the caches at each token's position.  For the prefill GEMMs it can
 * also write (each may be NULL) bf16 operands split into `parts` (1 to 3) terms, x = t_0 +
 * t_1 + ... with t_0 = bf16(x) and t_s = bf16 of what the earlier terms leave (three terms hold
 * all 24 bits of an fp32 value):
 *   q_out  [batch, heads, seq_rows, parts * head_dim]: the terms of the rotated q side by side;
 *   k_out  [batch, kv_heads, seq_rows, parts * head_dim]: the cached k, `parts` times;
 *   vt_out [batch, kv_heads, head_dim, ld_vt]: the cached v transposed, token t at columns
 *          s * ld_vt / parts + t for each term s (ld_vt / parts >= seq_rows and a multiple of
 *          8, head_dim % 8 == 0, 16-byte aligned; tokens past max_seq are not written);
 * so that one bf16 MFMA GEMM of q_out against k_out gives q . k^T with fp32-like accuracy. */
int tgm_dec_rope_kv(float* qkv, int64_t rows, int64_t seq_rows, int64_t heads, int64_t kv_heads, int64_t head_dim,
                    const int32_t* pos, double rope_base, void* k_cache, void* v_cache, int64_t max_seq, void* q_out,
                    void* k_out, void* vt_out, int64_t ld_vt, int64_t parts, void* stream);

/* Residual add + RMSNorm folded into a one-row packed GEMV (a decoder layer's norm and the
 * projection after it in one launch, for one token):
 *
 *   x = (h + delta) * (1 / sqrt(sum((h + delta)^2) / k + eps)) * norm_weight    (fp32)
 *   y = x . deq(W)^T        (x rounded to f16 for INT4 / UINT4 weights, to bf16 for FP4)
 *
 * with h, delta [k] fp32 (delta may be NULL), norm_weight [k] bf16, and h + delta stored to
 * h_out (may be NULL; must not alias h or delta).  swiglu != 0: W interleaves gate and up rows
 * and y [n / 2] = silu(gate) * up, as tgm_gemv_swiglu.  k = 2048 or 4096; FP4 weights with
 * E8M0/32 (or no) scales, or INT4 / UINT4 with f16, bf16 or f32 group scales per 32, 64 or
 * 128; 16-byte aligned operands; otherwise TGM_E_UNSUPPORTED.  The reference has no model
 * code (decoder harness). */
int tgm_dec_norm_gemv(const float* h, const float* delta, float* h_out, const void* norm_weight, float eps,
                      const void* w, int fmt, int64_t n, int64_t k, const void* scales, int scale_dtype,
                      int64_t block_size, void* y, int y_dtype, int swiglu, void* stream);

/* Causal attention of prompt tokens in one kernel: for every sequence b, q head h and token
 * t (rows b * seq_rows + t of qkv, whose q heads tgm_dec_rope_kv has rotated, at position
 * p = pos[b] + t), out[row, h] = softmax over cache positions k <= p of
 * q . K[k] / sqrt(head_dim), applied to V, with K and V the bf16 caches (kv head
 * h / (heads / kv_heads)), which must already hold positions 0 .. p.  Scores and
 * probabilities stay on chip (flash-attention form on bf16 MFMA); q and the probabilities are
 * split into three bf16 terms each, so the result has the accuracy of fp32 arithmetic.
 * head_dim 64 or 128; qkv and caches 16-byte aligned (else TGM_E_UNSUPPORTED); out f16,
 * bf16 or f32 [rows, heads * head_dim].  The reference has no model code (decoder harness). */
int tgm_dec_prefill_attention(const float* qkv, int64_t rows, int64_t seq_rows, int64_t heads, int64_t kv_heads,
                              int64_t head_dim, const int32_t* pos, const void* k_cache, const void* v_cache,
                              int64_t max_seq, void* out, int out_dtype, void* stream);

/* Causal softmax of prefill scores: for row = z * seq_rows + t (float32, row stride ld_scores),
 * p[j] = softmax over j <= t of scale * scores[row, j] is split into `parts` (1 to 3) bf16 terms
 * as in tgm_dec_rope_kv, term s at probs[row, s * ld_probs / parts + j], all 0 for
 * t < j < ld_probs / parts (ld_probs a multiple of parts, ld_probs / parts >= seq_rows), so that
 * one GEMM of probs against the vt_out of tgm_dec_rope_kv (K = ld_probs) gives P . V.
 * ld_scores must be a multiple of 4, ld_probs / parts of 8, and both buffers 16-byte aligned. */
int tgm_dec_causal_softmax(const float* scores, int64_t rows, int64_t seq_rows, int64_t ld_scores, float scale,
                           void* probs, int64_t ld_probs, int64_t parts, void* stream);

/* Causal grouped-query attention of every q head over its kv head's cache, positions
 * 0 .. pos(token) (softmax of q.k / sqrt(head_dim) in fp32).  head_dim is 64 or 128; heads /
 * kv_heads is 1, 2, 4 or 8.  ``splits`` > 1 (at most 32) divides each token's positions over
 * that many workgroups (split-K over the sequence, merged by a second kernel) and needs
 * ``workspace`` of tgm_dec_attention_workspace() bytes.  out is [rows, heads * head_dim].
 * rope_base > 0 (seq_rows == 1 only) also does tgm_dec_rope_kv's work for each token in the
 * same arithmetic: q and k of qkv are read unrotated, and the token's k (rotated) and v are
 * stored into the caches.  rope_base <= 0: qkv holds rotated q and the caches already hold
 * every position the tokens attend to. */
int64_t tgm_dec_attention_workspace(int64_t rows, int64_t heads, int64_t head_dim, int64_t splits);
int tgm_dec_attention(const float* qkv, int64_t rows, int64_t seq_rows, int64_t heads, int64_t kv_heads,
                      int64_t head_dim, const int32_t* pos, void* k_cache, void* v_cache, int64_t max_seq,
                      double rope_base, int64_t splits, float* workspace, int64_t workspace_bytes, void* out,
                      int out_dtype, void* stream);

/* SwiGLU: out[r, i] = silu(g) * u with g = gate_up[r, 2 i], u = gate_up[r, 2 i + 1] (float32
 * [rows, 2 * ffn], gate and up interleaved as the rows of the gate|up weight are, so that the
 * M = 1 projection can apply it in its epilogue, tgm_gemv_swiglu); out is [rows, ffn]. */
int tgm_dec_silu_mul(const float* gate_up, int64_t rows, int64_t ffn, void* out, int out_dtype, void* stream);

/* Dense bf16 GEMV for the output head: y[m, n] = sum_k x[m, k] * w[n, k] in fp32.  w is BF16
 * [n, k], x BF16 (row stride ldx), y F32 (row stride ldy); m <= 8, k a multiple of 8 and
 * m * k <= 32768. */
int tgm_dec_gemv_bf16(const void* w, int64_t n, int64_t k, const void* x, int64_t m, int64_t ldx, float* y,
                      int64_t ldy, void* stream);

/* Greedy decode: tokens[r] = argmax_n logits[r, n] (row stride ld; the first maximum wins).
 * When pos is given, also history[r * hist_stride + pos[r] + 1 - hist_base] = tokens[r]
 * (when that index lies in [0, hist_stride) and history is given) and pos[r] += 1. */
int tgm_dec_argmax(const float* logits, int64_t rows, int64_t n, int64_t ld, int32_t* tokens, int32_t* pos,
                   int32_t* history, int64_t hist_stride, int64_t hist_base, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TGM_DECODER_H */
