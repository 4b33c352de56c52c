"""CPU restatement of the Llama-style decoder around the packed path (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this module; it checks the device path and is never the thing measured or shipped.

The reference has no model code (a decoder on it would be tinygrad ops around
``PackedTensor.matmul``, src/tinygrad_dx12/codegen/decomp/dx12.py:108-112), so nothing here
follows a reference file line by line.  The math is the standard Llama decoder layer:

    h   = embed[token]
    x   = RMSNorm(h) * w_attn            -> f16           (input of the INT4 projections)
    qkv = x @ deq(Wqkv)^T; q, k rotated by RoPE (rotate-half pairs, base^(-2i/hd))
    k, v stored as bf16 in the cache; attention = softmax(q k^T / sqrt(hd)) v over positions
    0 .. p (GQA: q head h reads kv head h // (heads / kv_heads))      -> f16
    h  += attn @ deq(Wo)^T
    x   = RMSNorm(h) * w_ffn             -> bf16          (input of the FP4 projections)
    g|u = x @ deq(Wgu)^T (gate and up rows interleaved); a = silu(g) * u -> bf16
    h  += a @ deq(Wdown)^T
    logits = bf16(RMSNorm(h) * w_final) @ lm_head^T; next token = first argmax

The rounding points (f16 / bf16 casts of activations and of the KV cache) are the device
path's; everything else is float64.  The dequantised weights come from ``packed_oracle``.

Pinned (tests/test_decoder_oracle.py) by what the mathematics fixes, not by a retyped
formula: RoPE is an isometry, identity at position 0, and makes q.k depend only on the
position difference; RMSNorm output has unit RMS for unit weights; attention over one
position returns v; grouped-query attention equals multi-head attention over repeated kv
heads; prefill of T tokens and prefill of T - n tokens followed by n cached decode steps
give the same logits; the argmax takes the first maximum.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

import packed_oracle as O


def f16(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=np.float64).astype(np.float32).astype(np.float16).astype(np.float64)


def bf16(x: np.ndarray) -> np.ndarray:
    return O.bf16_to_f32(O.bf16_round(np.asarray(x, dtype=np.float64).astype(np.float32))).astype(np.float64)


def rmsnorm(h: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    return h / np.sqrt(np.mean(h * h, axis=-1, keepdims=True) + eps) * w


def rope(x: np.ndarray, positions: np.ndarray, base: float) -> np.ndarray:
    """Rotate-half RoPE of x [..., T, hd] at positions [T]."""
    hd = x.shape[-1]
    half = hd // 2
    inv = base ** (-2.0 * np.arange(half) / hd)
    ang = np.asarray(positions, dtype=np.float64)[:, None] * inv[None, :]
    c, s = np.cos(ang), np.sin(ang)
    x1, x2 = x[..., :half], x[..., half:]
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1)


def silu(g: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):  # exp(-g) = inf for very negative g gives the limit -0
        return g / (1.0 + np.exp(-g))


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, q_pos: np.ndarray) -> np.ndarray:
    """q [H, Tq, hd] at positions q_pos; k, v [HK, Tk, hd] for positions 0 .. Tk - 1.

    Query i attends to positions 0 .. q_pos[i]; heads / kv_heads q heads share a kv head.
    """
    H, HK, hd = q.shape[0], k.shape[0], q.shape[-1]
    rep = H // HK
    kk = np.repeat(k, rep, axis=0)
    vv = np.repeat(v, rep, axis=0)
    s = q @ kk.transpose(0, 2, 1) / np.sqrt(hd)
    mask = np.arange(k.shape[1])[None, :] > np.asarray(q_pos)[:, None]
    s = np.where(mask[None], -np.inf, s)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return p @ vv


@dataclass
class OracleLayer:
    attn_norm: np.ndarray
    wqkv: np.ndarray
    wo: np.ndarray
    ffn_norm: np.ndarray
    w_gate_up: np.ndarray
    w_down: np.ndarray


@dataclass
class OracleWeights:
    embed: np.ndarray
    layers: list[OracleLayer]
    final_norm: np.ndarray
    lm_head: np.ndarray


class OracleDecoder:
    """Float64 decoder with the device path's rounding points and a per-sequence KV cache."""

    def __init__(self, w: OracleWeights, heads: int, kv_heads: int, head_dim: int, ffn: int, eps: float,
                 rope_base: float, batch: int, max_seq: int) -> None:
        self.w, self.H, self.HK, self.hd, self.F = w, heads, kv_heads, head_dim, ffn
        self.eps, self.base = eps, rope_base
        L = len(w.layers)
        self.k = np.zeros((L, batch, kv_heads, max_seq, head_dim))
        self.v = np.zeros((L, batch, kv_heads, max_seq, head_dim))

    def attn_input(self, li: int, h: np.ndarray) -> np.ndarray:
        """The f16 input of layer ``li``'s QKV projection: RMSNorm(h) * w_attn."""
        return f16(rmsnorm(h, self.w.layers[li].attn_norm, self.eps))

    def qkv(self, li: int, x: np.ndarray, start: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
        """q, k rotated to positions start .. start + T - 1 and v, from the projection input x
        [B, T, D]: q [B, H, T, hd], k and v [B, HK, T, hd], unrounded."""
        B, T = x.shape[:2]
        H, HK, hd = self.H, self.HK, self.hd
        pos = np.arange(start, start + T)
        qkv = x @ self.w.layers[li].wqkv.T
        q = qkv[..., :H * hd].reshape(B, T, H, hd).transpose(0, 2, 1, 3)
        k = qkv[..., H * hd:(H + HK) * hd].reshape(B, T, HK, hd).transpose(0, 2, 1, 3)
        v = qkv[..., (H + HK) * hd:].reshape(B, T, HK, hd).transpose(0, 2, 1, 3)
        return rope(q, pos, self.base), rope(k, pos, self.base), v

    def attend(self, li: int, q: np.ndarray, start: int) -> np.ndarray:
        """Causal attention of q [B, H, T, hd] at positions start .. over layer ``li``'s cache,
        as [B, T, H * hd], unrounded."""
        B, H, T, hd = q.shape
        pos = np.arange(start, start + T)
        att = np.stack([attention(q[b], self.k[li, b, :, :start + T], self.v[li, b, :, :start + T], pos)
                        for b in range(B)])
        return att.transpose(0, 2, 1, 3).reshape(B, T, H * hd)

    def attention_delta(self, li: int, h: np.ndarray, start: int) -> np.ndarray:
        """Layer ``li``'s attention half for residual h [B, T, D] at positions start .. start + T - 1:
        stores the new k, v in the layer's cache and returns attn @ Wo^T (what the layer adds to h)."""
        T = h.shape[1]
        q, k, v = self.qkv(li, self.attn_input(li, h), start)
        self.k[li, :, :, start:start + T] = bf16(k)
        self.v[li, :, :, start:start + T] = bf16(v)
        return f16(self.attend(li, q, start)) @ self.w.layers[li].wo.T

    def ffn_input(self, li: int, h: np.ndarray) -> np.ndarray:
        """The bf16 input of layer ``li``'s gate|up projection: RMSNorm(h) * w_ffn."""
        return bf16(rmsnorm(h, self.w.layers[li].ffn_norm, self.eps))

    def swiglu(self, li: int, x: np.ndarray) -> np.ndarray:
        """silu(gate) * up of the gate|up projection of x (gate and up rows interleaved), unrounded."""
        gu = x @ self.w.layers[li].w_gate_up.T
        return silu(gu[..., 0::2]) * gu[..., 1::2]

    def ffn_delta(self, li: int, h: np.ndarray) -> np.ndarray:
        """Layer ``li``'s feed-forward half for residual h: what it adds to h."""
        return bf16(self.swiglu(li, self.ffn_input(li, h))) @ self.w.layers[li].w_down.T

    def head(self, h: np.ndarray) -> np.ndarray:
        """Logits of residual rows h [..., D]."""
        x = bf16(rmsnorm(h, self.w.final_norm, self.eps))
        return x @ self.w.lm_head.T

    def forward(self, tokens: np.ndarray, start: int) -> np.ndarray:
        """Run tokens [B, T] at positions start .. start + T - 1; returns logits [B, T, V]."""
        h = self.w.embed[tokens].astype(np.float64)
        for li in range(len(self.w.layers)):
            h = h + self.attention_delta(li, h, start)
            h = h + self.ffn_delta(li, h)
        return self.head(h)

    def generate(self, prompts: np.ndarray, new_tokens: int) -> tuple[np.ndarray, np.ndarray]:
        """Greedy decode: ([B, new_tokens] token ids, [B, new_tokens, V] logits that chose them)."""
        B, T = prompts.shape
        logits = [self.forward(prompts, 0)[:, -1]]
        toks = [logits[-1].argmax(axis=-1)]
        for i in range(1, new_tokens):
            logits.append(self.forward(toks[-1][:, None], T + i - 1)[:, -1])
            toks.append(logits[-1].argmax(axis=-1))
        return np.stack(toks, axis=1), np.stack(logits, axis=1)
