"""Llama-style decoder on the packed matmul path: prefill and greedy decode on gfx950.

The reference has no model code.  A decoder on it would be ordinary tinygrad ops around
``PackedTensor.matmul`` (alexandreteles/tinygrad-dx12 src/tinygrad_dx12/codegen/decomp/
dx12.py:108-112), with INT4 ``block_size=128`` accepted by dx12.py:30, :44-47.  This module is
that consumer, the one that turns the packed kernels into tokens per second:

* attention projections: INT4 weights with fp16 scales per 128 K-elements; q, k and v rows
  are stacked into one weight so that a token needs one QKV product;
* feed-forward: FP4 E2M1 weights with E8M0 scales per 32; gate and up rows interleaved in one
  weight, so that the one-token GEMV applies SwiGLU in its epilogue;
* embeddings and output head: bf16; RMSNorm weights bf16; residual stream fp32;
* RoPE (rotate-half pairs, base 10000) and grouped-query attention over a bf16 KV cache.

Every operation is a gfx950 kernel of ``libtgm_mi355x.so``: the packed GEMV (decode, up to
16 rows) and GEMM (prefill), plus the decoder-step kernels (include/tgm_decoder.h).  torch
supplies device memory and the stream.  Activations feeding INT4 weights are fp16 and those
feeding FP4 weights bf16, the activation types of the two kernel families.

A decode step reads sequence positions and the previous tokens from device memory and its
argmax writes the next tokens and advances the positions, so its launch sequence never
changes: ``Decoder.generate`` captures one step as a HIP graph and replays it.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from tinygrad_mi355x.codegen.decomp.mi355x import PackedTensor, quantize_mx
from tinygrad_mi355x.runtime import kernels as K
from tinygrad_mi355x.runtime.graph import StreamGraph

F16, BF16, F32 = K.DTYPE_IDS[torch.float16], K.DTYPE_IDS[torch.bfloat16], K.DTYPE_IDS[torch.float32]
GEMV_MAX_ROWS = 16
# Decode attention takes one of two forms (tgm_dec_attention):
#   one pass (splits = 1): a 16-wave workgroup per (token, q head) streams its kv head's cache,
#     about 8-9 ns per position per workgroup on top of ~5 us (one CU per q head bounds it);
#   position splits: the positions spread over workgroups and a second launch merges them,
#     ~8 us at batch 1 almost independent of the length (~9-11 us at batch 8, 100-600 positions).
# One pass is taken when its grid fits one round of CUs and either fills at least half of them or
# the mean decode length is short; never beyond ONE_PASS_MAX_LEN.
ONE_PASS_SHORT_LEN = 384
ONE_PASS_MAX_LEN = 1024


@dataclass(frozen=True)
class DecoderConfig:
    hidden: int = 4096
    heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    ffn: int = 14336
    vocab: int = 32000
    layers: int = 8
    eps: float = 1e-5
    rope_base: float = 10000.0
    attn_group: int = 128  # INT4 scale group along K

    @property
    def qkv_rows(self) -> int:
        return (self.heads + 2 * self.kv_heads) * self.head_dim

    def weight_bytes_per_token(self) -> int:
        """Weight bytes one decode step streams: packed layers plus the bf16 output head."""
        d, f = self.hidden, self.ffn
        attn = (self.qkv_rows + d) * d // 2 + (self.qkv_rows + d) * (d // self.attn_group) * 2
        ffn = 3 * d * f // 2 + 3 * d * f // 32
        norms = 2 * d * 2
        return self.layers * (attn + ffn + norms) + self.vocab * d * 2 + d * 2


@dataclass
class LayerWeights:
    attn_norm: torch.Tensor      # bf16 [D]
    wqkv: PackedTensor           # int4 [(H + 2 HK) hd, D], fp16 scales per attn_group
    wo: PackedTensor             # int4 [D, H hd]
    ffn_norm: torch.Tensor       # bf16 [D]
    w_gate_up: PackedTensor      # fp4 [2 F, D], E8M0 per 32; row 2 i is gate i, row 2 i + 1 is up i
    w_down: PackedTensor         # fp4 [D, F]


@dataclass
class DecoderWeights:
    embed: torch.Tensor          # bf16 [V, D]
    layers: list[LayerWeights]
    final_norm: torch.Tensor     # bf16 [D]
    lm_head: torch.Tensor        # bf16 [V, D]


def random_weights(cfg: DecoderConfig, device: str | torch.device = "cuda", seed: int = 0) -> DecoderWeights:
    """Synthetic random-init weights of the configured shape, generated on the device.

    INT4 codes are uniform over all 16 nibbles with scales in [0.002, 0.005]; FP4 weights are
    N(0, 0.02) MX-quantised along K; norms 1 + 0.1 N(0, 1); embeddings N(0, 1); head N(0, 0.02).
    """
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    d = cfg.hidden

    def int4(n: int, k: int) -> PackedTensor:
        data = torch.randint(0, 256, (n * k // 2,), dtype=torch.uint8, device=device, generator=g)
        scales = (torch.rand((n, k // cfg.attn_group), device=device, generator=g) * 0.003 + 0.002).to(torch.float16)
        return PackedTensor(data, "int4", (n, k), scales, cfg.attn_group)

    def fp4(n: int, k: int) -> PackedTensor:
        return quantize_mx(torch.randn((n, k), device=device, generator=g) * 0.02, "fp4_e2m1")

    def norm() -> torch.Tensor:
        return (1.0 + 0.1 * torch.randn(d, device=device, generator=g)).to(torch.bfloat16)

    layers = []
    for _ in range(cfg.layers):
        layers.append(LayerWeights(norm(), int4(cfg.qkv_rows, d), int4(d, cfg.heads * cfg.head_dim), norm(),
                                   fp4(2 * cfg.ffn, d), fp4(d, cfg.ffn)))
    embed = torch.randn((cfg.vocab, d), device=device, generator=g).to(torch.bfloat16)
    final_norm = norm()
    lm_head = (torch.randn((cfg.vocab, d), device=device, generator=g) * 0.02).to(torch.bfloat16)
    return DecoderWeights(embed, layers, final_norm, lm_head)


_LAYER_FIELDS = ("attn_norm", "wqkv", "wo", "ffn_norm", "w_gate_up", "w_down")


def save_weights(path, w: DecoderWeights, cfg: DecoderConfig) -> None:
    """Write the weights and configuration as a packed-weights file (tinygrad_mi355x.checkpoint)."""
    from dataclasses import asdict

    from tinygrad_mi355x import checkpoint

    tensors = {"embed": w.embed, "final_norm": w.final_norm, "lm_head": w.lm_head}
    for i, layer in enumerate(w.layers):
        for field in _LAYER_FIELDS:
            tensors[f"layers.{i}.{field}"] = getattr(layer, field)
    checkpoint.save(path, tensors, {"decoder": asdict(cfg)})


def load_weights(path, device: str | torch.device = "cuda") -> tuple[DecoderWeights, DecoderConfig]:
    """Read weights written by ``save_weights`` onto ``device``."""
    from tinygrad_mi355x import checkpoint

    tensors, meta = checkpoint.load(path, device)
    if "decoder" not in meta:
        raise ValueError(f"{path} holds no decoder configuration")
    cfg = DecoderConfig(**meta["decoder"])
    try:
        layers = [LayerWeights(*(tensors[f"layers.{i}.{field}"] for field in _LAYER_FIELDS)) for i in range(cfg.layers)]
        weights = DecoderWeights(tensors["embed"], layers, tensors["final_norm"], tensors["lm_head"])
    except KeyError as error:
        raise ValueError(f"{path} lacks decoder tensor {error}") from error
    return weights, cfg


GEMM_TILE_M, GEMM_TILE_N, GEMM_FILL = 128, 256, 192  # packed GEMM output tile; tiles that fill the chip


def _norm_gemv_fits(w: PackedTensor, swiglu: bool) -> bool:
    """Whether tgm_dec_norm_gemv takes this weight: FP4 with E8M0 scales per 32 (required with
    the SwiGLU epilogue) or none, INT4 / UINT4 with f16, bf16 or f32 group scales per 32, 64 or
    128 or none."""
    if w.format == "fp4_e2m1":
        if w.scales is None:
            return not swiglu
        return w.scales.dtype == torch.float8_e8m0fnu and w.block_size == 32
    if w.format in ("int4", "uint4") and not swiglu:
        return w.scales is None or (w.scales.dtype in (torch.float16, torch.bfloat16, torch.float32)
                                    and w.block_size in (32, 64, 128))
    return False


def gemm_splits(m: int, n: int) -> int:
    """K splits for a packed GEMM whose output tiles alone would leave CUs idle (at most 8)."""
    tiles = -(-m // GEMM_TILE_M) * -(-n // GEMM_TILE_N)
    return 1 if tiles >= GEMM_FILL else max(1, min(8, 256 // tiles))


def _packed_product(x: torch.Tensor, m: int, ldx: int, w: PackedTensor, y: torch.Tensor, ldy: int, stream: int,
                    workspace: "_Workspace | None" = None) -> None:
    """y[:m] = x[:m] @ deq(w)^T: packed GEMV for m <= 16 rows, packed GEMM above (with K split
    over ``workspace`` when the output has too few tiles)."""
    n, k = w.shape
    sdt = K.dtype_id(w.scales.dtype) if w.scales is not None else -1
    if m <= GEMV_MAX_ROWS:
        K.call("tgm_gemv", w.data.data_ptr(), K.FORMAT_IDS[w.format], n, k, K.ptr(w.scales), sdt, w.block_size,
               x.data_ptr(), K.dtype_id(x.dtype), m, ldx, y.data_ptr(), K.dtype_id(y.dtype), ldy, stream)
        return
    splits = gemm_splits(m, n) if workspace is not None else 1
    if splits > 1:
        ws = workspace.get(K.load_library().tgm_gemm_w_split_workspace(m, n, splits))
        K.call("tgm_gemm_w_split", x.data_ptr(), K.dtype_id(x.dtype), m, ldx, w.data.data_ptr(),
               K.FORMAT_IDS[w.format], n, k, K.ptr(w.scales), sdt, w.block_size, y.data_ptr(), K.dtype_id(y.dtype),
               ldy, splits, ws.data_ptr(), ws.numel() * 4, stream)
    else:
        K.call("tgm_gemm_w", x.data_ptr(), K.dtype_id(x.dtype), m, ldx, w.data.data_ptr(), K.FORMAT_IDS[w.format], n,
               k, K.ptr(w.scales), sdt, w.block_size, y.data_ptr(), K.dtype_id(y.dtype), ldy, stream)


class _Workspace:
    """A device buffer that grows to the largest request (allocated outside graph capture: only
    the prefill, which is never captured, asks for one)."""

    def __init__(self, device: torch.device) -> None:
        self.device, self.buf = device, None

    def get(self, nbytes: int) -> torch.Tensor:
        if self.buf is None or self.buf.numel() * 4 < nbytes:
            self.buf = torch.empty((max(nbytes, 16) + 3) // 4, dtype=torch.float32, device=self.device)
        return self.buf


class Decoder:
    """Prefill + greedy decode for ``batch`` sequences of up to ``max_seq`` tokens.

    All activations, the KV caches and the attention workspace are allocated once here;
    ``prefill`` and ``step`` launch kernels only.
    """

    def __init__(self, weights: DecoderWeights, cfg: DecoderConfig, batch: int, max_seq: int, max_prompt: int) -> None:
        if cfg.heads % cfg.kv_heads or cfg.head_dim not in (64, 128):
            raise ValueError("heads must be a multiple of kv_heads and head_dim 64 or 128")
        if not 1 <= batch <= 8:
            raise ValueError("batch must be in [1, 8] (the output-head GEMV takes up to 8 rows)")
        if not 1 <= max_prompt <= max_seq:
            raise ValueError("max_prompt must be in [1, max_seq]")
        self.w, self.cfg, self.batch, self.max_seq, self.max_prompt = weights, cfg, batch, max_seq, max_prompt
        dev = weights.embed.device
        K.require_device(weights.embed)
        self.device = dev
        d, rows = cfg.hidden, batch * max_prompt
        f32 = dict(dtype=torch.float32, device=dev)
        self.h = torch.empty((rows, d), **f32)
        self.delta = torch.empty((rows, d), **f32)
        self.xn16 = torch.empty((rows, d), dtype=torch.float16, device=dev)
        self.xnb = torch.empty((rows, d), dtype=torch.bfloat16, device=dev)
        self.qkv = torch.empty((rows, cfg.qkv_rows), **f32)
        self.attn = torch.empty((rows, cfg.heads * cfg.head_dim), dtype=torch.float16, device=dev)
        self.gu = torch.empty((rows, 2 * cfg.ffn), **f32)
        self.act = torch.empty((rows, cfg.ffn), dtype=torch.bfloat16, device=dev)
        self.logits = torch.empty((batch, cfg.vocab), **f32)
        cache = (cfg.layers, batch, cfg.kv_heads, max_seq, cfg.head_dim)
        self.k_cache = torch.zeros(cache, dtype=torch.bfloat16, device=dev)
        self.v_cache = torch.zeros(cache, dtype=torch.bfloat16, device=dev)
        # decode attention: one pass or position splits (ONE_PASS_SHORT_LEN)
        self.position_splits = min(max(1, math.ceil(max_seq / 64)), 32)
        cus = torch.cuda.get_device_properties(dev).multi_processor_count
        mean_len = (max_prompt + max_seq) / 2
        grid = batch * cfg.heads
        one_pass = (grid <= cus and mean_len <= ONE_PASS_MAX_LEN
                    and (2 * grid >= cus or mean_len <= ONE_PASS_SHORT_LEN))
        self.splits = 1 if one_pass else self.position_splits
        self.fuse_rope = True
        # attention of prompts of several tokens:
        #   "fused": one flash-attention kernel on MFMA (scores stay on chip);
        #   "gemm":  two batched MFMA GEMMs around a causal softmax (scores through memory), with
        #            ``prefill_parts`` bf16 terms per operand value (3: the accuracy of fp32);
        #   "split": the per-token decode attention kernel.
        self.prompt_attention = "fused"
        self.prefill_parts = 3
        self._gemm_buffers: dict[str, torch.Tensor] | None = None
        self._split_ws = _Workspace(dev)  # split-K partial products of the prefill GEMMs
        # one token: the gate|up GEMV applies SwiGLU itself when its row-streaming kernel covers the shape
        self.fuse_swiglu = (cfg.hidden % 2048 == 0 and cfg.hidden <= 16384)
        # 2 to 16 tokens: the streaming MFMA GEMV applies it (K a multiple of 128)
        self.fuse_swiglu_rows = cfg.hidden % 128 == 0
        # one token: each RMSNorm runs inside the projection after it (tgm_dec_norm_gemv), the
        # residual stream alternating between h and h_alt
        self.fuse_norm = (batch == 1 and cfg.hidden in (2048, 4096) and self.fuse_swiglu
                          and all(_norm_gemv_fits(L.wqkv, False) and _norm_gemv_fits(L.w_gate_up, True)
                                  for L in weights.layers))
        self.h_alt = torch.empty((batch, d), **f32) if self.fuse_norm else None
        # 5-8 tokens: the down projection's K is cut into slices of 2048 (tgm_dec_gemv_parts) and
        # the next add + RMSNorm sums the parts: a workgroup then stages one slice of the
        # activations for 64 weight rows instead of all 14336 columns for 16 rows
        # (4096 x 14336 at 8 tokens: 13.7 -> 10.8 us)
        wd = weights.layers[0].w_down
        self.down_slices = cfg.ffn // 2048 if (batch >= 5 and cfg.ffn % 2048 == 0 and 2 <= cfg.ffn // 2048 <= 16
                                               and wd.format in ("fp4_e2m1", "fp6_e2m3", "fp6_e3m2")
                                               and (wd.scales is None or wd.block_size == 32)) else 1
        self.delta_parts = torch.empty((self.down_slices, batch, d), **f32) if self.down_slices > 1 else None
        ws = K.load_library().tgm_dec_attention_workspace(batch, cfg.heads, cfg.head_dim, self.position_splits)
        self.workspace = torch.empty(max(ws // 4, 1), **f32)
        self.workspace_bytes = ws
        self.tokens = torch.zeros(rows, dtype=torch.int32, device=dev)
        self.pos = torch.zeros(batch, dtype=torch.int32, device=dev)
        self.history: torch.Tensor | None = None
        self.prompt_len = 0
        self._graph: StreamGraph | None = None
        self.graph_stream: torch.cuda.Stream | None = None
        # when a list (eager runs only): per layer, a dict of copies of the layer's activations --
        # "h" the residual after attention and "delta" the feed-forward output (fp32, the layer's
        # output is their sum), "x16" the normed f16 input of the QKV projection, "attn" the f16
        # attention output, "xb" the normed bf16 input of gate|up and "act" the bf16 SwiGLU
        # output; "x16" and "xb" are None when the norm runs inside the projection
        self.layer_trace: list[dict[str, torch.Tensor | None]] | None = None

    # ---------------------------------------------------------------- building blocks
    def _add_norm(self, rows: int, parts: int, first: bool, weight: torch.Tensor, out: torch.Tensor, odt: int,
                  stream: int) -> None:
        """h += delta (or the ``parts`` down-projection parts; nothing before the first layer),
        then RMSNorm(h) * weight -> out."""
        d = self.cfg.hidden
        if parts:
            K.call("tgm_dec_add_rmsnorm_parts", self.h.data_ptr(), self.delta_parts.data_ptr(), parts, rows * d, rows, d,
                   weight.data_ptr(), self.cfg.eps, out.data_ptr(), odt, stream)
        else:
            K.call("tgm_dec_add_rmsnorm", self.h.data_ptr(), None if first else self.delta.data_ptr(), rows, d,
                   weight.data_ptr(), self.cfg.eps, out.data_ptr(), odt, stream)

    def _down(self, rows: int, L: LayerWeights, stream: int) -> int:
        """The down projection of ``act``: into ``delta``, or as K-slice parts (returns their count)."""
        cfg = self.cfg
        if self.down_slices > 1 and 5 <= rows <= GEMV_MAX_ROWS:
            w = L.w_down
            K.call("tgm_dec_gemv_parts", w.data.data_ptr(), K.FORMAT_IDS[w.format], cfg.hidden, cfg.ffn, K.ptr(w.scales),
                   K.dtype_id(w.scales.dtype) if w.scales is not None else -1, w.block_size, self.act.data_ptr(), BF16,
                   rows, cfg.ffn, self.delta_parts.data_ptr(), cfg.hidden, self.down_slices, stream)
            return self.down_slices
        _packed_product(self.act, rows, cfg.ffn, L.w_down, self.delta, cfg.hidden, stream, self._split_ws)
        return 0

    def _layers(self, rows: int, seq_rows: int, splits: int, stream: int) -> None:
        cfg = self.cfg
        d = cfg.hidden
        fuse_norm = rows == 1 and self.fuse_norm
        parts = 0  # down-projection parts the next norm adds (0: the output is in delta)
        for li, L in enumerate(self.w.layers):
            if fuse_norm:  # h + delta -> h_alt, RMSNorm and the QKV projection in one launch
                w = L.wqkv
                K.call("tgm_dec_norm_gemv", self.h.data_ptr(), self.delta.data_ptr() if li else None,
                       self.h_alt.data_ptr(), L.attn_norm.data_ptr(), cfg.eps, w.data.data_ptr(),
                       K.FORMAT_IDS[w.format], cfg.qkv_rows, d, K.ptr(w.scales),
                       K.dtype_id(w.scales.dtype) if w.scales is not None else -1, w.block_size, self.qkv.data_ptr(),
                       F32, 0, stream)
            else:
                self._add_norm(rows, parts, li == 0, L.attn_norm, self.xn16, F16, stream)
                _packed_product(self.xn16, rows, d, L.wqkv, self.qkv, cfg.qkv_rows, stream, self._split_ws)
            kc, vc = self.k_cache[li], self.v_cache[li]
            fused = seq_rows == 1 and self.fuse_rope  # one new token per sequence: RoPE + cache store in attention
            if seq_rows > 1 and self.prompt_attention == "fused":
                K.call("tgm_dec_rope_kv", self.qkv.data_ptr(), rows, seq_rows, cfg.heads, cfg.kv_heads, cfg.head_dim,
                       self.pos.data_ptr(), cfg.rope_base, kc.data_ptr(), vc.data_ptr(), self.max_seq, None, None,
                       None, 0, 1, stream)
                K.call("tgm_dec_prefill_attention", self.qkv.data_ptr(), rows, seq_rows, cfg.heads, cfg.kv_heads,
                       cfg.head_dim, self.pos.data_ptr(), kc.data_ptr(), vc.data_ptr(), self.max_seq,
                       self.attn.data_ptr(), F16, stream)
            elif seq_rows > 1 and self.prompt_attention == "gemm":
                self._prefill_attention(rows, seq_rows, kc, vc, stream)
            else:
                if not fused:
                    K.call("tgm_dec_rope_kv", self.qkv.data_ptr(), rows, seq_rows, cfg.heads, cfg.kv_heads,
                           cfg.head_dim, self.pos.data_ptr(), cfg.rope_base, kc.data_ptr(), vc.data_ptr(),
                           self.max_seq, None, None, None, 0, 1, stream)
                K.call("tgm_dec_attention", self.qkv.data_ptr(), rows, seq_rows, cfg.heads, cfg.kv_heads,
                       cfg.head_dim, self.pos.data_ptr(), kc.data_ptr(), vc.data_ptr(), self.max_seq,
                       cfg.rope_base if fused else 0.0, splits, self.workspace.data_ptr() if splits > 1 else None,
                       self.workspace_bytes if splits > 1 else 0, self.attn.data_ptr(), F16, stream)
            _packed_product(self.attn, rows, cfg.heads * cfg.head_dim, L.wo, self.delta, d, stream, self._split_ws)
            if fuse_norm:  # h_alt + delta -> h, RMSNorm and the gate|up projection with SwiGLU
                w = L.w_gate_up
                K.call("tgm_dec_norm_gemv", self.h_alt.data_ptr(), self.delta.data_ptr(), self.h.data_ptr(),
                       L.ffn_norm.data_ptr(), cfg.eps, w.data.data_ptr(), K.FORMAT_IDS[w.format], 2 * cfg.ffn, d,
                       K.ptr(w.scales), K.dtype_id(w.scales.dtype), w.block_size, self.act.data_ptr(), BF16, 1, stream)
                _packed_product(self.act, rows, cfg.ffn, L.w_down, self.delta, d, stream, self._split_ws)
                self._trace(rows, fused_norm=True)
                continue
            K.call("tgm_dec_add_rmsnorm", self.h.data_ptr(), self.delta.data_ptr(), rows, d, L.ffn_norm.data_ptr(),
                   cfg.eps, self.xnb.data_ptr(), BF16, stream)
            if (rows == 1 and self.fuse_swiglu) or (1 < rows <= GEMV_MAX_ROWS and self.fuse_swiglu_rows):
                w = L.w_gate_up  # gate|up GEMV with the SwiGLU epilogue
                K.call("tgm_gemv_swiglu", w.data.data_ptr(), K.FORMAT_IDS[w.format], 2 * cfg.ffn, d, K.ptr(w.scales),
                       K.dtype_id(w.scales.dtype), w.block_size, self.xnb.data_ptr(), BF16, rows, d,
                       self.act.data_ptr(), BF16, cfg.ffn, stream)
            elif rows > GEMV_MAX_ROWS and L.w_gate_up.format == "fp4_e2m1":  # GEMM with the SwiGLU epilogue
                w = L.w_gate_up
                K.call("tgm_gemm_w_swiglu", self.xnb.data_ptr(), BF16, rows, d, w.data.data_ptr(),
                       K.FORMAT_IDS[w.format], 2 * cfg.ffn, d, K.ptr(w.scales),
                       K.dtype_id(w.scales.dtype) if w.scales is not None else -1, w.block_size,
                       self.act.data_ptr(), BF16, cfg.ffn, stream)
            else:
                _packed_product(self.xnb, rows, d, L.w_gate_up, self.gu, 2 * cfg.ffn, stream, self._split_ws)
                K.call("tgm_dec_silu_mul", self.gu.data_ptr(), rows, cfg.ffn, self.act.data_ptr(), BF16, stream)
            parts = self._down(rows, L, stream)
            self._trace(rows, parts=parts)
        self._add_norm(rows, parts, False, self.w.final_norm, self.xnb, BF16, stream)

    def _trace(self, rows: int, fused_norm: bool = False, parts: int = 0) -> None:
        if self.layer_trace is not None:
            delta = self.delta[:rows].clone()
            if parts:  # the parts summed in the order the next norm adds them
                delta = self.delta_parts[0, :rows].clone()
                for p in range(1, parts):
                    delta += self.delta_parts[p, :rows]
            self.layer_trace.append({
                "h": self.h[:rows].clone(), "delta": delta, "attn": self.attn[:rows].clone(),
                "act": self.act[:rows].clone(), "x16": None if fused_norm else self.xn16[:rows].clone(),
                "xb": None if fused_norm else self.xnb[:rows].clone()})

    def _prefill_attention(self, rows: int, t: int, kc: torch.Tensor, vc: torch.Tensor, stream: int) -> None:
        """Causal attention of a whole prompt (positions 0 .. t - 1 of every sequence) as two
        batched bf16 MFMA GEMMs around a softmax.  The first operand of each product is split
        into n = ``prefill_parts`` bf16 terms (x = bf16(x) + bf16(rest) + ..., three terms
        hold an fp32 value) side by side along K, against n copies of the second operand, so
        the products keep fp32 accuracy for n times the (small) GEMM work:

        1. RoPE; k and v go to the caches; the q terms [seq, head, t, n hd], k n times [seq,
           kv head, t, n hd] and v transposed n times [seq, kv head, hd, n tp] (tp = t rounded
           up to 64) for the GEMMs;
        2. S = q k^T for every (sequence, head) pair in fp32, the heads / kv_heads q heads of a
           group sharing their kv head's keys;
        3. P = causal softmax(S / sqrt(hd)) as n terms, zero beyond each row's position;
        4. O = P v over the padded key count, written as f16 straight into the [token,
           head * hd] rows of the attention output.
        """
        cfg = self.cfg
        H, HK, hd, n = cfg.heads, cfg.kv_heads, cfg.head_dim, self.prefill_parts
        if not 1 <= n <= 3:
            raise ValueError("prefill_parts must be 1, 2 or 3")
        tp = -(-t // 64) * 64
        z, g = self.batch * H, H // HK
        if self._gemm_buffers is None:  # sized for 3 terms and the longest prompt, allocated once
            tmax = -(-self.max_prompt // 64) * 64
            b16 = dict(dtype=torch.bfloat16, device=self.device)
            self._gemm_buffers = {
                "q": torch.empty((self.batch * H * self.max_prompt * 3 * hd,), **b16),
                "k": torch.empty((self.batch * HK * self.max_prompt * 3 * hd,), **b16),
                "vt": torch.zeros((self.batch * HK * hd * 3 * tmax,), **b16),
                "s": torch.empty((self.batch * H * self.max_prompt * tmax,), dtype=torch.float32, device=self.device),
                "p": torch.empty((self.batch * H * self.max_prompt * 3 * tmax,), **b16)}
        buf = self._gemm_buffers
        K.call("tgm_dec_rope_kv", self.qkv.data_ptr(), rows, t, H, HK, hd, self.pos.data_ptr(), cfg.rope_base,
               kc.data_ptr(), vc.data_ptr(), self.max_seq, buf["q"].data_ptr(), buf["k"].data_ptr(),
               buf["vt"].data_ptr(), n * tp, n, stream)
        K.call("tgm_gemm_dense_batched", buf["q"].data_ptr(), BF16, t, n * hd, t * n * hd, buf["k"].data_ptr(),
               BF16, t, n * hd, t * n * hd, g, n * hd, buf["s"].data_ptr(), F32, tp, t * tp, z, 0, z, stream)
        K.call("tgm_dec_causal_softmax", buf["s"].data_ptr(), z * t, t, tp, 1.0 / math.sqrt(hd),
               buf["p"].data_ptr(), n * tp, n, stream)
        K.call("tgm_gemm_dense_batched", buf["p"].data_ptr(), BF16, t, n * tp, t * n * tp, buf["vt"].data_ptr(), BF16,
               hd, n * tp, hd * n * tp, g, n * tp, self.attn.data_ptr(), F16, H * hd, hd, H, t * H * hd, z, stream)

    def _head(self, first_row: int, row_stride: int, stream: int, advance: bool) -> None:
        """Output head over one normed row per sequence (rows first_row + b * row_stride of the
        normed activations) and the greedy argmax."""
        cfg = self.cfg
        x = self.xnb[first_row]
        K.call("tgm_dec_gemv_bf16", self.w.lm_head.data_ptr(), cfg.vocab, cfg.hidden, x.data_ptr(), self.batch,
               row_stride * cfg.hidden, self.logits.data_ptr(), cfg.vocab, stream)
        hist = self.history
        K.call("tgm_dec_argmax", self.logits.data_ptr(), self.batch, cfg.vocab, cfg.vocab, self.tokens.data_ptr(),
               self.pos.data_ptr() if advance else None, hist.data_ptr() if (advance and hist is not None) else None,
               hist.shape[1] if hist is not None else 0, self.prompt_len, stream)

    # ---------------------------------------------------------------- public API
    def prefill(self, prompts: torch.Tensor) -> torch.Tensor:
        """Run the prompts (int [batch, T], T <= max_prompt) and return the first greedy tokens."""
        if prompts.dim() != 2 or prompts.shape[0] != self.batch or not 1 <= prompts.shape[1] <= self.max_prompt:
            raise ValueError(f"prompts must be [{self.batch}, 1..{self.max_prompt}]")
        if int(prompts.min()) < 0 or int(prompts.max()) >= self.cfg.vocab:
            raise ValueError("prompt tokens out of range")
        if self.prompt_attention not in ("fused", "gemm", "split"):
            raise ValueError(f"prompt_attention must be 'fused', 'gemm' or 'split', not {self.prompt_attention!r}")
        t = prompts.shape[1]
        rows = self.batch * t
        stream = K.stream_of(self.h)
        self.prompt_len = t
        self.tokens[:rows].copy_(prompts.reshape(-1).to(torch.int32))
        self.pos.zero_()
        K.call("tgm_dec_embed", self.w.embed.data_ptr(), self.cfg.vocab, self.cfg.hidden, self.tokens.data_ptr(), rows,
               self.h.data_ptr(), stream)
        self._layers(rows, t, 1, stream)
        self._head(t - 1, t, stream, advance=False)  # the last prompt row of each sequence
        self.pos.fill_(t)
        self._graph = None
        return self.tokens[:self.batch].clone()

    def _decode_step(self) -> None:
        stream = K.stream_of(self.h)
        K.call("tgm_dec_embed", self.w.embed.data_ptr(), self.cfg.vocab, self.cfg.hidden, self.tokens.data_ptr(),
               self.batch, self.h.data_ptr(), stream)
        self._layers(self.batch, 1, self.splits, stream)
        self._head(0, 1, stream, advance=True)

    def step(self) -> None:
        """One eager decode step: consumes ``tokens[:batch]`` at ``pos``, writes the next tokens."""
        self._decode_step()

    def capture(self) -> StreamGraph:
        """Capture one decode step on a side stream as a HIP graph (replayed by ``generate``)."""
        if self._graph is None:
            stream = torch.cuda.Stream(device=self.device)
            stream.wait_stream(torch.cuda.current_stream(self.device))
            with torch.cuda.stream(stream):
                self._graph = StreamGraph(self._decode_step, stream.cuda_stream)
            self.graph_stream = stream
        return self._graph

    def generate(self, prompts: torch.Tensor, new_tokens: int, graph: bool = True) -> torch.Tensor:
        """Greedy generation: [batch, new_tokens] token ids (the first comes from the prefill)."""
        if new_tokens < 1 or prompts.shape[1] + new_tokens - 1 > self.max_seq:
            raise ValueError("prompt + generated tokens exceed max_seq")
        self.history = torch.zeros((self.batch, new_tokens), dtype=torch.int32, device=self.device)
        self.prompt_len = prompts.shape[1]
        self._graph = None
        first = self.prefill(prompts)
        self.history[:, 0] = first
        if new_tokens > 1:
            # the first step runs eagerly: it also performs every kernel's one-time set-up, which
            # must not happen inside a capture
            self._decode_step()
        remaining = new_tokens - 2
        if graph and remaining > 0:
            g = self.capture()
            cur = torch.cuda.current_stream(self.device)
            self.graph_stream.wait_stream(cur)
            for _ in range(remaining):
                g.launch()
            cur.wait_stream(self.graph_stream)
        else:
            for _ in range(max(remaining, 0)):
                self._decode_step()
        return self.history.clone()
