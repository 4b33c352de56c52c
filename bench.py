"""Benchmark of the packed low-bit matmul path on one MI355X.

A step is one FP4 E2M1 (+ E8M0 per 32 K-elements) decode GEMV, W [14336, 4096],
x bf16 [1, 4096] -> y bf16 [1, 14336], fp32 accumulation -- one call of the C-ABI
entry point ``tgm_gemv``.  Every step reads a different copy of the weights (18
copies, 562 MB, more than twice the 256 MB Infinity Cache) so each launch streams
its weights from HBM.  The K timed steps are captured once in a HIP graph and
replayed, and timed with HIP events on the launch stream.

``value`` is the achieved algorithmic bandwidth of the step (bytes of packed weights,
scales, x and y per step / time per step).  Secondary workloads (skinny M=4/16, the
INT4 g32 GEMV, the FP6-weight x bf16 GEMMs and the FP4xFP4 GEMMs) are reported under ``workloads``.
``cpu_baseline`` times the C restatement of the reference's CPU path
(oracle/cpu_path.c: materialise fp32 weights, fp32 GEMV, RNE to bf16) on the host.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "tinygrad-dx12_amd"))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP4_PEAK_TFLOPS = 10100.0
N_COPIES = 18


EXTRAS = ("fp4_gemv_m4", "fp4_gemv_m16", "int4_gemv_n4096", "int4_gemv_n14336", "fp6_e3m2_gemm_m2048", "fp6_e2m3_gemm_m2048", "fp4_gemm_8192",
          "fp4_gemm_4096x14336x4096", "decoder_b1", "decoder_b8")


def parse() -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-extras", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=12.0, help="budget of the CPU baseline sample")
    p.add_argument("--only", choices=sorted(EXTRAS), default=None,
                   help="run only this secondary workload and print its figures (for profiling)")
    p.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                   help="only run --steps device-to-device copies of MIB MiB (reference for HBM byte counters)")
    return p.parse_args()


def gemv_bytes(n: int, k: int, m: int, bits: int, scale_bytes: float, act_bytes: int, out_bytes: int) -> int:
    return n * k * bits // 8 + int(n * (k // 32) * scale_bytes) + m * k * act_bytes + m * n * out_bytes


class Timer:
    """Captures ``steps`` launches of ``launch(i)`` in a HIP graph; replays and times them."""

    def __init__(self, torch, launch, steps: int, warmup: int):
        self.torch, self.launch, self.steps, self.warmup = torch, launch, steps, warmup

    def run(self) -> float:
        torch = self.torch
        for i in range(self.warmup):
            self.launch(i)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        stream = torch.cuda.Stream()
        with torch.cuda.stream(stream):
            with torch.cuda.graph(graph, stream=stream):
                for i in range(self.steps):
                    self.launch(i)
        graph.replay()  # untimed replay: graph upload and first-touch
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            start.record(stream)
            graph.replay()
            end.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(end) / self.steps  # ms per step


def fp4_gemv_workload(torch, K, dev, m: int, steps: int, warmup: int, copies: int = N_COPIES):
    n, k = 14336, 4096
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    ws = [torch.randint(0, 256, (n * k // 2,), dtype=torch.uint8, device=dev, generator=g) for _ in range(copies)]
    ss = [torch.randint(123, 130, (n, k // 32), dtype=torch.uint8, device=dev, generator=g) for _ in range(copies)]
    x = torch.randn((m, k), device=dev, generator=g).to(torch.bfloat16)
    y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
    fmt, bf16, e8m0 = K.FORMAT_IDS["fp4_e2m1"], K.DTYPE_IDS[torch.bfloat16], K.DTYPE_IDS[torch.float8_e8m0fnu]
    lib = K.load_library()

    def launch(i: int) -> None:
        j = i % copies
        K.check("tgm_gemv", lib.tgm_gemv(ws[j].data_ptr(), fmt, n, k, ss[j].data_ptr(), e8m0, 32, x.data_ptr(), bf16,
                                         m, k, y.data_ptr(), bf16, n, K.stream_of(x)))

    ms = Timer(torch, launch, steps, warmup).run()
    nbytes = gemv_bytes(n, k, m, 4, 1, 2, 2)
    return {"workload": f"fp4_e2m1 e8m0/32 GEMV N=14336 K=4096 M={m}", "ms": ms, "bytes": nbytes,
            "GB/s": nbytes / ms / 1e6, "hbm_frac": nbytes / ms / 1e6 / HBM_PEAK_GBS,
            "TFLOPS": 2 * m * n * k / ms / 1e9}


def int4_gemv_workload(torch, K, dev, steps: int, warmup: int, copies: int = 40, n: int = 4096, k: int = 4096):
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    ws = [torch.randint(0, 256, (n * k // 2,), dtype=torch.uint8, device=dev, generator=g) for _ in range(copies)]
    ss = [(torch.rand((n, k // 32), device=dev, generator=g) * 0.015 + 0.005).half() for _ in range(copies)]
    x = torch.randn((1, k), device=dev, generator=g).half()
    y = torch.empty((1, n), dtype=torch.float16, device=dev)
    fmt, f16 = K.FORMAT_IDS["int4"], K.DTYPE_IDS[torch.float16]
    lib = K.load_library()

    def launch(i: int) -> None:
        j = i % copies
        K.check("tgm_gemv", lib.tgm_gemv(ws[j].data_ptr(), fmt, n, k, ss[j].data_ptr(), f16, 32, x.data_ptr(), f16,
                                         1, k, y.data_ptr(), f16, n, K.stream_of(x)))

    ms = Timer(torch, launch, steps, warmup).run()
    nbytes = gemv_bytes(n, k, 1, 4, 2, 2, 2)
    return {"workload": f"int4 g32 fp16-scale GEMV N={n} K={k} M=1 fp16", "ms": ms, "bytes": nbytes,
            "GB/s": nbytes / ms / 1e6, "hbm_frac": nbytes / ms / 1e6 / HBM_PEAK_GBS}


def measured_traffic(profile: str) -> int | None:
    """HBM bytes per launch of the dominant kernel from its committed rocprofv3 summary
    (FETCH_SIZE + WRITE_SIZE per dispatch, each scaled by a plain copy of known size)."""
    path = ROOT / "profiles" / profile
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch="):
            return int(line.split("=", 1)[1])
    return None


def settle(torch, stream, launch, warmup: int, min_ms: float = 60.0) -> None:
    """Untimed launches of a compute-bound kernel: at least ``warmup`` of them and at least
    ``min_ms`` of GPU time, since the clocks keep rising over the first tens of milliseconds of
    sustained MFMA load (a 4096 x 14336 x 4096 FP4 GEMM measured 180 us cold and 157 us after
    about 30 ms of the same work)."""
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    done, spent = 0, 0.0
    while done < warmup or spent < min_ms:
        e0.record(stream)
        for _ in range(5):
            launch()
        e1.record(stream)
        torch.cuda.synchronize()
        done, spent = done + 5, spent + e0.elapsed_time(e1)


def fp4_gemm_workload(torch, K, dev, m: int, n: int, k: int, steps: int, warmup: int):
    """FP4 x FP4 + E8M0/32 GEMM C[M,N] = deq(A) deq(B)^T, bf16 out, timed with HIP events on
    the launch stream (each launch is long enough that launch overhead is negligible).  The
    warmup launches let the clocks settle under MFMA load (the first few run ~15% slower)."""
    g = torch.Generator(device=dev)
    g.manual_seed(2)
    a = torch.randint(0, 256, (m * k // 2,), dtype=torch.uint8, device=dev, generator=g)
    b = torch.randint(0, 256, (n * k // 2,), dtype=torch.uint8, device=dev, generator=g)
    sa = torch.randint(123, 130, (m, k // 32), dtype=torch.uint8, device=dev, generator=g)
    sb = torch.randint(123, 130, (n, k // 32), dtype=torch.uint8, device=dev, generator=g)
    c = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
    fp4, bf16 = K.FORMAT_IDS["fp4_e2m1"], K.DTYPE_IDS[torch.bfloat16]
    lib = K.load_library()
    stream = torch.cuda.current_stream(dev)

    def launch() -> None:
        K.check("tgm_gemm_mx", lib.tgm_gemm_mx(a.data_ptr(), fp4, sa.data_ptr(), m, b.data_ptr(), fp4, sb.data_ptr(), n, k,
                                               c.data_ptr(), bf16, n, stream.cuda_stream))

    settle(torch, stream, launch, warmup)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        launch()
    end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    tflops = 2 * m * n * k / ms / 1e9
    nbytes = (m + n) * k // 2 + (m + n) * k // 32 + m * n * 2
    return {"workload": f"fp4xfp4 e8m0/32 GEMM M={m} N={n} K={k} bf16 out", "ms": ms, "TFLOPS": tflops,
            "mfma_frac": tflops / FP4_PEAK_TFLOPS, "bytes": nbytes, "GB/s": nbytes / ms / 1e6}


def fp6_gemm_workload(torch, K, dev, fmt: str, steps: int, warmup: int, m: int = 2048, n: int = 11008, k: int = 4096):
    """Packed FP6 weight x bf16 activation prefill GEMM C[M,N] = A deq(W)^T (E8M0 per 32),
    bf16 out, on the dequant-to-bf16 MFMA kernel; timed like the FP4 GEMM."""
    g = torch.Generator(device=dev)
    g.manual_seed(4)
    a = torch.randn((m, k), device=dev, generator=g).to(torch.bfloat16)
    w = torch.randint(0, 256, (n * k * 6 // 8,), dtype=torch.uint8, device=dev, generator=g)
    s = torch.randint(123, 130, (n, k // 32), dtype=torch.uint8, device=dev, generator=g)
    c = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
    f, bf16, e8m0 = K.FORMAT_IDS[fmt], K.DTYPE_IDS[torch.bfloat16], K.DTYPE_IDS[torch.float8_e8m0fnu]
    lib = K.load_library()
    stream = torch.cuda.current_stream(dev)

    def launch() -> None:
        K.check("tgm_gemm_w", lib.tgm_gemm_w(a.data_ptr(), bf16, m, k, w.data_ptr(), f, n, k, s.data_ptr(), e8m0, 32,
                                             c.data_ptr(), bf16, n, stream.cuda_stream))

    settle(torch, stream, launch, warmup)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        launch()
    end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    tflops = 2 * m * n * k / ms / 1e9
    nbytes = m * k * 2 + n * k * 6 // 8 + n * (k // 32) + m * n * 2
    return {"workload": f"{fmt} e8m0/32 weight x bf16 GEMM M={m} N={n} K={k} bf16 out", "ms": ms, "TFLOPS": tflops,
            "bf16_mfma_frac": tflops / BF16_PEAK_TFLOPS, "bytes": nbytes, "GB/s": nbytes / ms / 1e6}


def decoder_workload(torch, dev, batch: int, prompt: int = 512, new_tokens: int = 128):
    """Llama-style decoder (8 layers, hidden 4096, 32 / 8 heads x 128, SwiGLU 14336, vocab 32000;
    INT4 g128 attention, FP4 + E8M0 FFN, bf16 head): a 512-token prefill, then greedy decode of
    128 tokens, the decode steps replayed as a HIP graph and timed with HIP events on the
    graph's stream.  Random-init weights and prompts."""
    from tinygrad_mi355x.decoder import Decoder, DecoderConfig, random_weights

    cfg = DecoderConfig()
    w = random_weights(cfg, dev, seed=0)
    dec = Decoder(w, cfg, batch, prompt + new_tokens, prompt)
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    prompts = torch.randint(0, cfg.vocab, (batch, prompt), device=dev, generator=g)
    cur = torch.cuda.current_stream(dev)
    dec.history = torch.zeros((batch, new_tokens), dtype=torch.int32, device=dev)
    t_warm = time.perf_counter()
    while True:  # untimed prefills, at least 60 ms of them, while the clocks settle
        dec.prefill(prompts)
        torch.cuda.synchronize()
        if time.perf_counter() - t_warm >= 0.06:
            break
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(cur)
    dec.prefill(prompts)
    e1.record(cur)
    torch.cuda.synchronize()
    prefill_ms = e0.elapsed_time(e1)
    dec.step()  # first decode step eagerly (kernel set-up), then the graph
    graph = dec.capture()
    s = dec.graph_stream
    s.wait_stream(cur)
    steps = new_tokens - 2
    e0.record(s)
    for _ in range(steps):
        graph.launch()
    e1.record(s)
    torch.cuda.synchronize()
    step_ms = e0.elapsed_time(e1) / steps
    mean_ctx = prompt + 1 + (steps + 1) / 2
    kv_bytes = int(cfg.layers * batch * cfg.kv_heads * mean_ctx * cfg.head_dim * 2 * 2)
    step_bytes = cfg.weight_bytes_per_token() + kv_bytes
    return {"workload": f"8-layer decoder (hidden 4096, INT4 attention, FP4 FFN) batch {batch}: {prompt}-token prefill + greedy decode of {new_tokens} tokens "
                        "(decode steps replayed as a HIP graph)",
            "decode_ms_per_step": step_ms, "tokens_per_s": batch / step_ms * 1e3,
            "bytes_per_step": step_bytes, "GB/s": step_bytes / step_ms / 1e6,
            "hbm_frac": step_bytes / step_ms / 1e6 / HBM_PEAK_GBS,
            "prefill_ms": prefill_ms, "prefill_tokens_per_s": batch * prompt / prefill_ms * 1e3,
            "final_pos": int(dec.pos[0])}


def cpu_baseline(budget_s: float) -> dict:
    """The reference CPU path restated in C (oracle/cpu_path.c), timed on the host cores."""
    import numpy as np

    lib = ctypes.CDLL(str(ROOT / "oracle" / "liboracle_cpu.so"))
    n, k, m = 14336, 4096, 1
    rng = np.random.default_rng(0)
    data = rng.integers(0, 256, n * k // 2).astype(np.uint8)
    e = (127 + rng.integers(-4, 3, (n, k // 32))).astype(np.int64)
    scales = np.ldexp(np.float32(1.0), (e - 127)).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x = ((x.view(np.uint32) + 0x8000) & 0xFFFF0000).view(np.float32)  # bf16-valued activations
    wdeq = np.empty(n * k, np.float32)
    yf = np.empty(m * n, np.float32)
    y = np.empty(m * n, np.uint16)
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    i64 = ctypes.c_int64

    def once() -> float:
        t = time.perf_counter()
        lib.oracle_cpu_path(p(data), i64(data.size), 2, i64(n), i64(k), p(scales), i64(32), p(x), i64(m), p(wdeq),
                            p(yf), p(y), 16)
        return time.perf_counter() - t

    once()  # warm the pages
    times, start = [], time.perf_counter()
    while time.perf_counter() - start < budget_s and len(times) < 200:
        times.append(once())
    med = statistics.median(times)
    nbytes = gemv_bytes(n, k, m, 4, 1, 2, 2)
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"full fp4 e8m0/32 GEMV 14336x4096 M=1 (dequant to fp32 + fp32 GEMV + bf16), "
                      f"median of {len(times)} runs, {med * 1e3:.1f} ms each"}


def copy_calibration(torch, mib: int, steps: int) -> None:
    """Plain device copies of a known size: FETCH_SIZE / WRITE_SIZE per dispatch of this copy
    kernel calibrate the counters against bytes actually moved."""
    n = mib << 20
    src = torch.randint(0, 256, (n,), dtype=torch.uint8, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": n, "steps": steps}))


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark runs on one GPU; --gpus must be 1 (multi-GPU sharding is design-only)"}))
        return 2
    import torch

    from tinygrad_mi355x.runtime import kernels as K

    dev = torch.device("cuda:0")
    if args.copy_calibration:
        copy_calibration(torch, args.copy_calibration, args.steps)
        return 0
    K.load_library()
    half = max(args.steps // 2, 1)
    extras = {
        "fp4_gemv_m4": lambda: fp4_gemv_workload(torch, K, dev, 4, half, args.warmup),
        "fp4_gemv_m16": lambda: fp4_gemv_workload(torch, K, dev, 16, half, args.warmup),
        "int4_gemv_n4096": lambda: int4_gemv_workload(torch, K, dev, half, args.warmup),
        "int4_gemv_n14336": lambda: int4_gemv_workload(torch, K, dev, half, args.warmup, copies=12, n=14336),
        "fp6_e3m2_gemm_m2048": lambda: fp6_gemm_workload(torch, K, dev, "fp6_e3m2", 20, 20),
        "fp6_e2m3_gemm_m2048": lambda: fp6_gemm_workload(torch, K, dev, "fp6_e2m3", 20, 20),
        "fp4_gemm_8192": lambda: fp4_gemm_workload(torch, K, dev, 8192, 8192, 8192, 20, 20),
        "fp4_gemm_4096x14336x4096": lambda: fp4_gemm_workload(torch, K, dev, 4096, 14336, 4096, 20, 20),
        "decoder_b1": lambda: decoder_workload(torch, dev, 1),
        "decoder_b8": lambda: decoder_workload(torch, dev, 8),
    }
    if args.only:
        print(json.dumps({args.only: extras[args.only]()}))
        return 0
    torch.cuda.synchronize()
    wall = time.perf_counter()
    primary = fp4_gemv_workload(torch, K, dev, 1, args.steps, args.warmup)
    workloads = {}
    if not args.no_extras:
        for name in EXTRAS:
            workloads[name] = extras[name]()
    torch.cuda.synchronize()
    gpu_wall = time.perf_counter() - wall
    cpu = None if args.no_cpu_baseline else cpu_baseline(args.cpu_seconds)
    gbs = primary["GB/s"]
    line = {
        "metric": "low-bit GEMV GB/s (% HBM peak) + FP4 GEMM TFLOPS (% MFMA peak), 1 GPU",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(primary["ms"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp4_e2m1 x bf16 -> fp32 acc -> bf16",
        "data": "synthetic (uniform E2M1 codes, E8M0 exponents 123..129, N(0,1) bf16 activations), 18 rotating weight copies",
        "config": {"workload": primary["workload"], "N": 14336, "K": 4096, "M": 1, "block": 32,
                   "launch": "hip graph of the timed steps", "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic("gemv_fp4_e2m1_n14336_k4096_m1.txt")},
        "cpu_baseline": cpu,
        "workloads": {name: {k: (round(v, 6) if isinstance(v, float) else v) for k, v in w.items()}
                      for name, w in workloads.items()},
        "gpu_wall_s": round(gpu_wall, 2),
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
