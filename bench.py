"""Benchmark of the packed low-bit matmul path on one MI355X.

A step is one FP4 E2M1 (+ E8M0 per 32 K-elements) decode GEMV, W [14336, 4096],
x bf16 [1, 4096] -> y bf16 [1, 14336], fp32 accumulation -- one call of the C-ABI
entry point ``tgm_gemv``.  Consecutive steps read different copies of the weights (a
copy set of at least 600 MB, over twice the 256 MB Infinity Cache, walked in order, so a
copy is read again only after every other copy has been), so each launch streams its
weights from HBM.  A trial is exactly K steps captured in one HIP graph, replayed and
timed with HIP events on the launch stream; ``value`` comes from the median of several
trials (each trial's graph continues the rotation where the previous one stopped).

``value`` is the achieved algorithmic bandwidth of the step (bytes of packed weights,
scales, x and y per step / time per step); every workload's algorithmic bytes and flops are
the Estimates of the kernel program it launches (tinygrad_mi355x/codegen/program.py).  Secondary workloads (skinny M=4/16, the
INT4 g32 GEMVs, the FP6-weight x bf16 GEMMs, the FP4xFP4 GEMMs and the 8-layer
decoder) are reported under ``workloads``, each with its own roofline.
``cpu_baseline`` times the C restatement of the reference's CPU path
(oracle/cpu_path.c: materialise fp32 weights, fp32 GEMV, RNE to bf16 / fp16) on the host
cores, for the headline GEMV and, under the INT4 4096 x 4096 workload, for that GEMV.

``--summarize-profile DIR --only W`` turns the rocprofv3 runs of workload W (the commands
it prints in its header) into the summary committed under ``profiles/``.
"""

from __future__ import annotations

import argparse
import csv
import ctypes
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "tinygrad-dx12_amd"))

from tinygrad_mi355x.codegen import program as P  # noqa: E402  (torch-free: kernel programs and their estimates)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP4_PEAK_TFLOPS = 10100.0
ROTATION_BYTES = 600_000_000  # every GEMV copy set: > 2 x the 256 MB Infinity Cache
MIN_TRIALS = 5

EXTRAS = ("fp4_gemv_m4", "fp4_gemv_m16", "int4_gemv_n4096", "int4_gemv_n14336", "fp6_e3m2_gemm_m2048",
          "fp6_e2m3_gemm_m2048", "fp4_gemm_8192", "fp4_gemm_4096x14336x4096", "decoder_b1", "decoder_b8",
          "read_ceiling_31232000", "read_ceiling_9453568", "read_ceiling_470000000", "mfma_fp4_ceiling_8192",
          "launch_floor_448", "fp4_gemv_shard_n1792_m1", "fp4_gemv_shard_n1792_m4", "fp4_gemv_shard_n1792_m16",
          "bf16_gemm_8192", "fp8_gemm_8192", "uop_rowsum_16384x4096", "uop_gemm_bf16_4096_relu")
PRIMARY = "fp4_gemv_m1"

# workload -> (committed rocprof summary, substring of the dominant kernel's name)
PROFILES = {
    "fp4_gemv_m1": ("gemv_fp4_e2m1_n14336_k4096_m1.txt", "gemv_rows_fp4"),
    "fp4_gemv_m4": ("gemv_fp4_e2m1_n14336_k4096_m4.txt", "gemv_quads"),
    "fp4_gemv_m16": ("gemv_fp4_e2m1_n14336_k4096_m16.txt", "gemv_stream"),
    "int4_gemv_n4096": ("gemv_int4_g32_n4096_k4096_m1.txt", "gemv_rows_int4"),
    "int4_gemv_n14336": ("gemv_int4_g32_n14336_k4096_m1.txt", "gemv_rows_int4"),
    "fp6_e3m2_gemm_m2048": ("gemm_w_fp6_e3m2_m2048_n11008_k4096.txt", "gemm_w_stream"),
    "fp6_e2m3_gemm_m2048": ("gemm_w_fp6_e2m3_m2048_n11008_k4096.txt", "gemm_w_stream"),
    "fp4_gemm_8192": ("gemm_mx_fp4_m8192_n8192_k8192.txt", "gemm_mx"),
    "fp4_gemm_4096x14336x4096": ("gemm_mx_fp4_m4096_n14336_k4096.txt", "gemm_mx"),
    "bf16_gemm_8192": ("gemm_dense_bf16_m8192_n8192_k8192.txt", "gemm_dense"),
    "fp8_gemm_8192": ("gemm_dense_fp8_e4m3_m8192_n8192_k8192.txt", "gemm_dense"),
    "read_ceiling_31232000": ("probe_read_31232000.txt", "probe_read"),
    "read_ceiling_9453568": ("probe_read_9453568.txt", "probe_read"),
    "uop_rowsum_16384x4096": ("uop_rowsum_f32_16384x4096.txt", "uop_rowsum"),
    "uop_gemm_bf16_4096_relu": ("uop_schedule_gemm_dense_bf16_4096_relu.txt", "gemm_dense"),
    "read_ceiling_470000000": ("probe_read_470000000.txt", "probe_read"),
    "mfma_fp4_ceiling_8192": ("probe_mfma_fp4_1024x512.txt", "probe_mfma_fp4"),
    "launch_floor_448": ("probe_launch_448x256.txt", "probe_launch"),
    "fp4_gemv_shard_n1792_m1": ("gemv_fp4_e2m1_n1792_k4096_m1.txt", "gemv_rows_fp4"),
    "fp4_gemv_shard_n1792_m4": ("gemv_fp4_e2m1_n1792_k4096_m4.txt", "gemv_quads"),
    "fp4_gemv_shard_n1792_m16": ("gemv_fp4_e2m1_n1792_k4096_m16.txt", "gemv_stream"),
}


def parse() -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200, help="steps per timed trial (K)")
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-extras", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=12.0, help="budget of each CPU baseline sample")
    p.add_argument("--only", choices=sorted((PRIMARY,) + EXTRAS), default=None,
                   help="run only this workload and print its figures (for profiling)")
    p.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                   help="only run --steps device-to-device copies of MIB MiB (reference for HBM byte counters)")
    p.add_argument("--summarize-decoder", type=Path, default=None, metavar="DIR",
                   help="summarise the rocprofv3 kernel trace under DIR of a decoder_b1 / decoder_b8 run (--only) "
                        "per decode step or per prefill (--part)")
    p.add_argument("--part", choices=("decode", "prefill"), default="decode")
    p.add_argument("--summarize-profile", type=Path, default=None, metavar="DIR",
                   help="summarise the rocprofv3 output folders under DIR for the --only workload")
    return p.parse_args()


def median_trials(torch, launch, steps: int, warmup: int, copies: int) -> tuple[float, int, int]:
    """Median ms per step over trials of exactly ``steps`` launches.

    ``launch(i)`` runs step ``i`` on copy ``i % copies``.  Trial ``r`` is a HIP graph of steps
    [r * steps, (r + 1) * steps); the trial count makes the trials cover the copy ring a whole
    number of times (and is at least MIN_TRIALS), so every copy is reread only after all the
    others, also across the untimed first pass over every graph (graph upload) and the timed
    second pass.  Returns (median ms per step, trials, timed dispatches).
    """
    for i in range(warmup):
        launch(i)
    torch.cuda.synchronize()
    cycle = copies // math.gcd(steps, copies)
    trials = cycle * max(1, -(-MIN_TRIALS // cycle))
    stream = torch.cuda.Stream()
    graphs = []
    for r in range(trials):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream), torch.cuda.graph(g, stream=stream):
            for i in range(steps):
                launch(r * steps + i)
        graphs.append(g)
    with torch.cuda.stream(stream):
        for g in graphs:  # untimed pass: graph upload and first touch
            g.replay()
    torch.cuda.synchronize()
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in graphs]
    with torch.cuda.stream(stream):
        for g, (e0, e1) in zip(graphs, events):
            e0.record(stream)
            g.replay()
            e1.record(stream)
    torch.cuda.synchronize()
    ms = statistics.median(e0.elapsed_time(e1) for e0, e1 in events) / steps
    return ms, trials, trials * steps


def copies_for(nbytes: int) -> int:
    return max(2, -(-ROTATION_BYTES // nbytes))


def hbm_roofline(nbytes: int, ms: float) -> dict:
    achieved = nbytes / ms / 1e6
    return {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4)}


def mfma_roofline(flops: int, ms: float, peak: float, what: str) -> dict:
    achieved = flops / ms / 1e9
    return {"bound": "mfma", "achieved": round(achieved, 2), "peak": peak, "unit": "TFLOP/s",
            "frac": round(achieved / peak, 4), "peak_of": what}


def fp4_gemv_workload(torch, K, dev, m: int, steps: int, warmup: int, n: int = 14336) -> dict:
    """FP4 E2M1 + E8M0/32 GEMV W [N, 4096] (N = 14336; 1792 is one GPU's eighth of it when the rows
    are split over 8 GPUs), bf16 X [M, 4096] -> bf16 Y [M, N]: codes uniform over the 16 E2M1
    values, E8M0 bytes 127 + [-4, 2], X ~ N(0, 1) rounded to bf16."""
    k = 4096
    nbytes = P.weight_program(P.PackedDesc("fp4_e2m1", (n, k), n * k // 2, 1, "float8_e8m0fnu"), m, "bfloat16", k,
                              "bfloat16", n).estimates.mem
    copies = copies_for(nbytes)
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    ws = [torch.randint(0, 256, (n * k // 2,), dtype=torch.uint8, device=dev, generator=g) for _ in range(copies)]
    ss = [torch.randint(123, 130, (n, k // 32), dtype=torch.uint8, device=dev, generator=g) for _ in range(copies)]
    x = torch.randn((m, k), device=dev, generator=g).to(torch.bfloat16)
    y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
    # one program per weight copy (each binds its copy's scales); slots (out, a, b) = (Y, W, X)
    progs = [P.weight_program(P.PackedDesc("fp4_e2m1", (n, k), n * k // 2, s.data_ptr(), "float8_e8m0fnu"), m,
                              "bfloat16", k, "bfloat16", n) for s in ss]

    def launch(i: int) -> None:
        j = i % copies
        progs[j].launch(y.data_ptr(), ws[j].data_ptr(), x.data_ptr(), K.stream_of(x))

    ms, trials, timed = median_trials(torch, launch, steps, warmup, copies)
    return {"workload": f"fp4_e2m1 e8m0/32 GEMV N={n} K=4096 M={m}", "ms": ms, "bytes": nbytes,
            "GB/s": nbytes / ms / 1e6, "TFLOPS": 2 * m * n * k / ms / 1e9, "copies": copies,
            "copy_set_bytes": copies * nbytes, "trials": trials, "steps_per_trial": steps,
            "timed_dispatches": timed, "roofline": hbm_roofline(nbytes, ms)}


def int4_gemv_workload(torch, K, dev, n: int, steps: int, warmup: int, k: int = 4096) -> dict:
    """INT4 g32 GEMV W [N, 4096] with fp16 scales ~ U(0.005, 0.02), fp16 x [1, 4096] -> fp16 y."""
    nbytes = P.weight_program(P.PackedDesc("int4", (n, k), n * k // 2, 1, "float16"), 1, "float16", k, "float16",
                              n).estimates.mem
    copies = copies_for(nbytes)
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    ws = [torch.randint(0, 256, (n * k // 2,), dtype=torch.uint8, device=dev, generator=g) for _ in range(copies)]
    ss = [(torch.rand((n, k // 32), device=dev, generator=g) * 0.015 + 0.005).half() for _ in range(copies)]
    x = torch.randn((1, k), device=dev, generator=g).half()
    y = torch.empty((1, n), dtype=torch.float16, device=dev)
    progs = [P.weight_program(P.PackedDesc("int4", (n, k), n * k // 2, s.data_ptr(), "float16"), 1, "float16", k,
                              "float16", n) for s in ss]

    def launch(i: int) -> None:
        j = i % copies
        progs[j].launch(y.data_ptr(), ws[j].data_ptr(), x.data_ptr(), K.stream_of(x))

    ms, trials, timed = median_trials(torch, launch, steps, warmup, copies)
    return {"workload": f"int4 g32 fp16-scale GEMV N={n} K={k} M=1 fp16", "ms": ms, "bytes": nbytes,
            "GB/s": nbytes / ms / 1e6, "copies": copies, "copy_set_bytes": copies * nbytes, "trials": trials,
            "steps_per_trial": steps, "timed_dispatches": timed, "roofline": hbm_roofline(nbytes, ms)}


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


def median_launch_ms(torch, stream, launch, steps: int) -> float:
    """Median over ``steps`` back-to-back launches, each bracketed by HIP events on ``stream``."""
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for e0, e1 in events:
        e0.record(stream)
        launch()
        e1.record(stream)
    torch.cuda.synchronize()
    return statistics.median(e0.elapsed_time(e1) for e0, e1 in events)


def fp4_gemm_workload(torch, K, dev, m: int, n: int, k: int, steps: int, warmup: int, vendor: bool = False,
                      zero: bool = False) -> dict:
    """FP4 x FP4 + E8M0/32 GEMM C[M,N] = deq(A) deq(B)^T, bf16 out: A [M, K] and B [N, K] drawn
    N(0, 1) and MX-quantised along K (round to nearest even, shared exponent per 32)."""
    from tinygrad_mi355x.codegen.decomp.mi355x import quantize_mx

    g = torch.Generator(device=dev)
    g.manual_seed(2)
    a = quantize_mx(torch.randn((m, k), device=dev, generator=g), "fp4_e2m1")
    b = quantize_mx(torch.randn((n, k), device=dev, generator=g), "fp4_e2m1")
    c = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
    stream = torch.cuda.current_stream(dev)
    prog = P.mx_program(a.desc(), b.desc(), "bfloat16", n)

    def launch() -> None:
        prog.launch(c.data_ptr(), a.data.data_ptr(), b.data.data_ptr(), stream.cuda_stream)

    settle(torch, stream, launch, warmup)
    ms = median_launch_ms(torch, stream, launch, steps)
    zero_ms = zero_operand_ms(torch, stream, prog, c, a.data, b.data, steps, warmup) if zero else None
    flops, nbytes = prog.estimates.ops, prog.estimates.mem
    return {"workload": f"fp4xfp4 e8m0/32 GEMM M={m} N={n} K={k} bf16 out", "ms": ms, "TFLOPS": flops / ms / 1e9,
            "flops": flops, "bytes": nbytes, "GB/s": nbytes / ms / 1e6, "timed_dispatches": steps,
            "zero_operands_ms": zero_ms, "zero_operands_TFLOPS": flops / zero_ms / 1e9 if zero_ms else None,
            "roofline": mfma_roofline(flops, ms, FP4_PEAK_TFLOPS, "dense MXFP4 MFMA"),
            "vendor": vendor_fp4_gemm(m, n, k, steps) if vendor else None}


def zero_operand_ms(torch, stream, prog, c, a, b, steps: int, warmup: int) -> float:
    """The same kernel program on all-zero operand bytes of the same sizes (same scales, same
    launch): the instruction stream, memory traffic and stalls are those of the real product, only
    the operand bits stop toggling.  The difference to the real time is what the operands'
    switching power costs through the clock the chip can hold (not part of any workload's value).
    Run in the full bench line only: its launches follow the timed ones, and a profile of a single
    workload takes its last launches as the timed ones."""
    za, zb = torch.zeros_like(a), torch.zeros_like(b)

    def launch() -> None:
        prog.launch(c.data_ptr(), za.data_ptr(), zb.data_ptr(), stream.cuda_stream)

    settle(torch, stream, launch, warmup)
    return median_launch_ms(torch, stream, launch, steps)


VENDOR_BAR = ROOT / "tinygrad-dx12_amd" / "tinygrad_mi355x" / "_lib" / "ck_mx_gemm_bar"


def vendor_fp4_gemm(m: int, n: int, k: int, steps: int) -> dict | None:
    """The vendor's MXFP4 GEMM on this machine: ROCm's Composable Kernel prebuilt instances
    (libdevice_gemm_operations.a; this ROCm's hipBLASLt ships no FP4 kernels for gfx950), every
    instance timed like this benchmark's GEMMs, beside tgm_gemm_mx on the same operands in the same
    child process (random FP4 codes, every E8M0 scale 2^0 since Composable Kernel reads its scales
    in its own shuffled order; both outputs checked at 64 sampled elements against exact sums)."""
    import subprocess

    if not VENDOR_BAR.exists():
        return None
    lib = ROOT / "tinygrad-dx12_amd" / "tinygrad_mi355x" / "_lib" / "libtgm_mi355x.so"
    try:
        proc = subprocess.run([str(VENDOR_BAR), str(m), str(n), str(k), str(steps), str(lib)], capture_output=True,
                              text=True, timeout=240)
    except subprocess.TimeoutExpired:
        return {"error": "timed out"}
    lines = [x for x in proc.stdout.splitlines() if x.startswith("{")]
    if proc.returncode != 0 or not lines:
        return {"error": (proc.stdout + proc.stderr).strip().splitlines()[-1:] or ["no output"]}
    r = json.loads(lines[-1])
    flops = 2 * m * n * k
    best = min(x for x in (r["ck_best_us"], r["ck_preshuffled_best_us"]) if x > 0)
    return {"library": "Composable Kernel (ROCm 7.2 libdevice_gemm_operations, MXFP4 instances, fp16 out)",
            "best_ms": best / 1e3, "TFLOPS": flops / best / 1e6, "frac": round(flops / best / 1e6 / FP4_PEAK_TFLOPS, 4),
            "best_instance": r["ck_best_instance"] if best == r["ck_best_us"] else r["ck_preshuffled_best_instance"],
            "natural_layout_best_ms": r["ck_best_us"] / 1e3, "natural_layout_max_rel_err": r["ck_best_err"],
            "preshuffled_b_best_ms": r["ck_preshuffled_best_us"] / 1e3 if r["ck_preshuffled_best_us"] > 0 else None,
            "instances": r["ck_instances"], "this_library_same_run_ms": r["tgm_us"] / 1e3,
            "this_library_max_rel_err": r["tgm_err"],
            "vendor_ms_over_this_library_ms": round(best / r["tgm_us"], 4) if r["tgm_us"] > 0 else None}


def fp6_gemm_workload(torch, K, dev, fmt: str, steps: int, warmup: int, m: int = 2048, n: int = 11008,
                      k: int = 4096) -> dict:
    """Packed FP6 weight x bf16 activation prefill GEMM C[M,N] = A deq(W)^T, bf16 out: A ~ N(0, 1)
    in bf16, W [N, K] drawn N(0, 0.02) and MX-quantised along K to ``fmt`` (E8M0 per 32)."""
    from tinygrad_mi355x.codegen.decomp.mi355x import quantize_mx

    g = torch.Generator(device=dev)
    g.manual_seed(4)
    a = torch.randn((m, k), device=dev, generator=g).to(torch.bfloat16)
    w = quantize_mx(torch.randn((n, k), device=dev, generator=g) * 0.02, fmt)
    c = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
    stream = torch.cuda.current_stream(dev)
    prog = P.weight_program(w.desc(), m, "bfloat16", k, "bfloat16", n)  # slots (out, a, b) = (C, W, A)

    def launch() -> None:
        prog.launch(c.data_ptr(), w.data.data_ptr(), a.data_ptr(), stream.cuda_stream)

    settle(torch, stream, launch, warmup)
    ms = median_launch_ms(torch, stream, launch, steps)
    flops, nbytes = prog.estimates.ops, prog.estimates.mem
    return {"workload": f"{fmt} e8m0/32 weight x bf16 GEMM M={m} N={n} K={k} bf16 out", "ms": ms,
            "TFLOPS": flops / ms / 1e9, "flops": flops, "bytes": nbytes, "GB/s": nbytes / ms / 1e6,
            "timed_dispatches": steps,
            "roofline": mfma_roofline(flops, ms, BF16_PEAK_TFLOPS, "dense bf16 MFMA (the activations stay bf16)")}


def dense_gemm_workload(torch, K, dev, dtype: str, n: int, steps: int, warmup: int, zero: bool = False) -> dict:
    """Ordinary product C[N,N] = A B^T (A, B [N, N], K-contiguous) on this library's kernel
    (tgm_gemm_dense for bf16, tgm_gemm_fp8 for float8_e4m3fn with per-tensor scales 1), bf16 out,
    with hipBLASLt timed on the same operands in the same run for comparison (torch.matmul for
    bf16, torch._scaled_mm for fp8)."""
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    tdt = getattr(torch, dtype)
    a = torch.randn((n, n), device=dev, generator=g).to(tdt)
    b = torch.randn((n, n), device=dev, generator=g).to(tdt)
    c = torch.empty((n, n), dtype=torch.bfloat16, device=dev)
    one = torch.ones((), dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev)
    fp8 = dtype.startswith("float8")
    prog = (P.dense_program(dtype, n, n, dtype, n, n, n, "bfloat16", n, one.data_ptr(), one.data_ptr()) if fp8
            else P.dense_program(dtype, n, n, dtype, n, n, n, "bfloat16", n))

    def launch() -> None:
        prog.launch(c.data_ptr(), a.data_ptr(), b.data_ptr(), stream.cuda_stream)

    settle(torch, stream, launch, warmup)
    ms = median_launch_ms(torch, stream, launch, steps)
    zero_ms = zero_operand_ms(torch, stream, prog, c, a, b, steps, warmup) if zero else None
    bt = b.t()  # column-major [K, N] view: hipBLASLt's natural B layout for C = A B^T
    if fp8:
        def library() -> None:
            torch._scaled_mm(a, bt, scale_a=one, scale_b=one, out_dtype=torch.bfloat16)
    else:
        bt_c = bt.contiguous()

        def library() -> None:
            torch.matmul(a, bt_c)
    settle(torch, stream, library, warmup)
    lib_ms = median_launch_ms(torch, stream, library, steps)
    flops, nbytes = prog.estimates.ops, prog.estimates.mem
    peak = 5000.0 if fp8 else BF16_PEAK_TFLOPS
    return {"workload": f"{dtype} x {dtype} GEMM M=N=K={n} bf16 out ({prog.name})", "ms": ms,
            "TFLOPS": flops / ms / 1e9, "flops": flops, "bytes": nbytes, "timed_dispatches": steps,
            "hipblaslt_ms": lib_ms, "hipblaslt_TFLOPS": flops / lib_ms / 1e9,
            "zero_operands_ms": zero_ms, "zero_operands_TFLOPS": flops / zero_ms / 1e9 if zero_ms else None,
            "roofline": mfma_roofline(flops, ms, peak, "dense fp8 MFMA" if fp8 else "dense bf16 MFMA")}


def _plugin_graph_ms(graph, steps: int, warmup: int) -> float:
    """Median GPU ms of one replay of a schedule graph on the plugin device's stream."""
    for _ in range(max(warmup, 1)):
        graph()
    return statistics.median(graph(wait=True) for _ in range(steps)) * 1e3


def uop_rowsum_workload(steps: int, warmup: int, rows: int = 16384, cols: int = 4096) -> dict:
    """A rendered UOp kernel: the row sums of an fp32 [16384, 4096] matrix (a REDUCE of 4096
    points per row, folded by one workgroup per row: strided register accumulators, then an LDS
    tree), on the plugin device, as a schedule of two launches over two copies of the matrix
    (537 MB, past the 256 MB Infinity Cache) replayed as one HIP graph; ms per launch."""
    from tinygrad_mi355x.runtime import ops_mi355x as R
    from tinygrad_mi355x.runtime.schedule import LinearGraph
    from tinygrad_mi355x.uop.ops import AxisType, KernelInfo, Ops, UOp, dtypes

    dev = R.get_device("MI355X")
    f32 = dtypes.float32
    x, o = UOp.param(1, f32, rows * cols, "MI355X"), UOp.param(0, f32, rows, "MI355X")
    r, c = UOp.range(rows, 0), UOp.range(cols, 1, AxisType.REDUCE)
    sink = o.index(r).store(x.index(r * cols + c).reduce(c, arg=Ops.ADD)).end(r).sink(
        arg=KernelInfo(name="uop_rowsum"))
    out, a, b = (UOp.new_buffer("MI355X", n, f32) for n in (rows, rows * cols, rows * cols))
    bound = {u: dev.allocator.alloc(u.max_numel() * 4) for u in (out, a, b)}
    graph = LinearGraph(dev, UOp.linear(UOp.call(sink, out, a), UOp.call(sink, out, b)), bound)
    ms = _plugin_graph_ms(graph, steps, warmup) / 2
    graph.close()
    nbytes = rows * cols * 4 + rows * 4
    return {"workload": f"UOp schedule: rendered row sums of fp32 [{rows}, {cols}] (workgroup-folded REDUCE)",
            "ms": ms, "bytes": nbytes, "GB/s": nbytes / ms / 1e6, "timed_dispatches": 2 * steps,
            "roofline": hbm_roofline(nbytes, ms)}


def uop_gemm_workload(steps: int, warmup: int, n: int = 4096) -> dict:
    """A UOp schedule C = relu(A B) (A [n, n], B [n, n] row-major [K, N], bf16, fp32 accumulation,
    bf16 out) lowered by the matmul rewrite to tgm_transpose16 (B -> [N, K]), tgm_gemm_dense into an
    fp32 buffer and the rendered ReLU epilogue, replayed as one HIP graph on the plugin device; ms
    per replay of the whole schedule."""
    import numpy as np

    from tinygrad_mi355x.codegen.uop_matmul import lower_matmul
    from tinygrad_mi355x.runtime import ops_mi355x as R
    from tinygrad_mi355x.runtime.schedule import LinearGraph
    from tinygrad_mi355x.uop.ops import AxisType, KernelInfo, Ops, UOp, dtypes

    dev = R.get_device("MI355X")
    bf = dtypes.bfloat16
    out_p, a_p, b_p = (UOp.param(i, bf, n * n, "MI355X") for i in range(3))
    row, col, i = UOp.range(n, 1), UOp.range(n, 2), UOp.range(n, 0, AxisType.REDUCE)
    prod = a_p.index(row * n + i).cast(dtypes.float32) * b_p.index(i * n + col).cast(dtypes.float32)
    value = prod.reduce(i, arg=Ops.ADD).maximum(0.0).cast(bf)
    sink = out_p.index(row * n + col).store(value).end(row, col).sink(arg=KernelInfo(name="uop_mm_relu"))
    bufs = [UOp.new_buffer("MI355X", n * n, bf) for _ in range(3)]
    linear = lower_matmul(UOp.linear(UOp.call(sink, *bufs)))
    kinds = [c.src[0].arg.name if c.src[0].op is Ops.PROGRAM else "rendered" for c in linear.src]
    rng = np.random.default_rng(6)
    bound = {}
    for u in bufs:
        bound[u] = dev.allocator.alloc(n * n * 2)
        host = (rng.standard_normal(n * n).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
        dev.allocator._copyin(bound[u], memoryview(host).cast("B"))
    graph = LinearGraph(dev, linear, bound)
    ms = _plugin_graph_ms(graph, steps, max(warmup, 20))
    graph.close()
    flops = 2 * n ** 3
    return {"workload": f"UOp schedule relu(A @ B), bf16 {n}^3, lowered to {' + '.join(kinds)}", "ms": ms,
            "TFLOPS": flops / ms / 1e9, "flops": flops, "bytes": 3 * n * n * 2, "timed_dispatches": steps,
            "roofline": mfma_roofline(flops, ms, BF16_PEAK_TFLOPS, "dense bf16 MFMA")}


def read_ceiling_workload(torch, K, dev, nbytes: int, steps: int, warmup: int) -> dict:
    """tgm_probe_read: ``nbytes`` read with the decode GEMV's access shape and discarded, over a
    rotating copy set timed like the GEMV -- the single-launch read ceiling for that many bytes
    (31,232,000 B: the FP4 decode GEMV's algorithmic bytes; 9,453,568 B: the INT4 g32 4096 x 4096
    GEMV's)."""
    copies = copies_for(nbytes)
    pool = torch.empty((copies, nbytes), dtype=torch.uint8, device=dev)
    pool.fill_(1)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    lib = K.load_library()

    def launch(i: int) -> None:
        K.check("tgm_probe_read", lib.tgm_probe_read(pool[i % copies].data_ptr(), nbytes, sink.data_ptr(),
                                                     K.stream_of(sink)))

    ms, trials, timed = median_trials(torch, launch, steps, warmup, copies)
    return {"workload": f"streaming read of {nbytes} B (the decode GEMV's access shape)", "ms": ms, "bytes": nbytes,
            "GB/s": nbytes / ms / 1e6, "copies": copies, "trials": trials, "steps_per_trial": steps,
            "timed_dispatches": timed, "roofline": hbm_roofline(nbytes, ms)}


def launch_floor_workload(torch, K, dev, groups: int, steps: int, warmup: int) -> dict:
    """tgm_probe_launch: an empty kernel of ``groups`` x 256 threads (448: the FP4 decode GEMV's
    grid at N = 14336), timed exactly like the GEMV (graphs of ``steps`` launches, median trial):
    the fixed cost every launch pays with no work.  A GEMV of B bytes cannot beat
    floor + B / 8 TB/s per step; ``ceiling_frac_31232000`` is that bound for the headline GEMV."""
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    lib = K.load_library()

    def launch(i: int) -> None:
        K.check("tgm_probe_launch", lib.tgm_probe_launch(groups, 256, sink.data_ptr(), K.stream_of(sink)))

    ms, trials, timed = median_trials(torch, launch, steps, warmup, 20)
    headline = 31_232_000
    ceiling_ms = ms + headline / (HBM_PEAK_GBS * 1e6)
    return {"workload": f"empty kernel, {groups} x 256 threads (the launch floor under the decode GEMV)",
            "ms": ms, "trials": trials, "steps_per_trial": steps, "timed_dispatches": timed,
            "ceiling_ms_31232000": ceiling_ms,
            "ceiling_frac_31232000": round(headline / ceiling_ms / 1e6 / HBM_PEAK_GBS, 4)}


def mfma_ceiling_workload(torch, K, dev, steps: int, warmup: int) -> dict:
    """tgm_probe_mfma_fp4 on the 8192^3 FP4 GEMM's grid (1024 workgroups of 8 waves, 2^23 FP4
    MFMAs = the GEMM's 1.0995e12 flops), operands from registers changing every round: the FP4
    MFMA ceiling with no data movement, timed like the GEMM."""
    blocks, iters = 1024, 128
    flops = blocks * 8 * iters * (1 << 20)
    sink = torch.zeros(4, dtype=torch.float32, device=dev)
    lib = K.load_library()
    stream = torch.cuda.current_stream(dev)

    def launch() -> None:
        K.check("tgm_probe_mfma_fp4", lib.tgm_probe_mfma_fp4(blocks, iters, sink.data_ptr(), stream.cuda_stream))

    settle(torch, stream, launch, warmup)
    ms = median_launch_ms(torch, stream, launch, steps)
    return {"workload": "FP4 scaled MFMA from registers, operands changing every round, on the 8192^3 GEMM's grid",
            "ms": ms, "TFLOPS": flops / ms / 1e9, "flops": flops, "timed_dispatches": steps,
            "roofline": mfma_roofline(flops, ms, FP4_PEAK_TFLOPS, "dense MXFP4 MFMA")}


def decoder_workload(torch, dev, batch: int, prompt: int = 512, new_tokens: int = 128) -> dict:
    """Llama-style decoder (8 layers, hidden 4096, 32 / 8 heads x 128, SwiGLU 14336, vocab 32000;
    INT4 g128 attention, FP4 + E8M0 FFN, bf16 head): a 512-token prefill, then greedy decode of
    128 tokens, the decode steps replayed as a HIP graph, each replay bracketed by HIP events on
    the graph's stream (median step reported).  Random-init weights and prompts."""
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
    prefills = []
    for _ in range(3):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(cur)
        dec.prefill(prompts)
        e1.record(cur)
        torch.cuda.synchronize()
        prefills.append(e0.elapsed_time(e1))
    prefill_ms = statistics.median(prefills)
    dec.step()  # first decode step eagerly (kernel set-up), then the graph
    graph = dec.capture()
    s = dec.graph_stream
    s.wait_stream(cur)
    steps = new_tokens - 2
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for e0, e1 in events:
        e0.record(s)
        graph.launch()
        e1.record(s)
    torch.cuda.synchronize()
    step_ms = statistics.median(e0.elapsed_time(e1) for e0, e1 in events)
    mean_ctx = prompt + 1 + (steps + 1) / 2
    kv_bytes = int(cfg.layers * batch * cfg.kv_heads * mean_ctx * cfg.head_dim * 2 * 2)
    step_bytes = cfg.weight_bytes_per_token() + kv_bytes
    return {"workload": f"8-layer decoder (hidden 4096, INT4 attention, FP4 FFN) batch {batch}: {prompt}-token "
                        f"prefill + greedy decode of {new_tokens} tokens (decode steps replayed as a HIP graph)",
            "decode_ms_per_step": step_ms, "tokens_per_s": batch / step_ms * 1e3,
            "bytes_per_step": step_bytes, "GB/s": step_bytes / step_ms / 1e6,
            "prefill_ms": prefill_ms, "prefill_tokens_per_s": batch * prompt / prefill_ms * 1e3,
            "final_pos": int(dec.pos[0]), "roofline": hbm_roofline(step_bytes, step_ms)}


def _host_description() -> dict:
    model = ""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"cpu_model": model, "nproc": os.cpu_count()}


def _time_cpu(once, budget_s: float, max_runs: int = 200) -> tuple[float, int]:
    once()  # warm the pages
    times, start = [], time.perf_counter()
    while time.perf_counter() - start < budget_s and len(times) < max_runs:
        times.append(once())
    return statistics.median(times), len(times)


def cpu_baseline_fp4(budget_s: float) -> dict:
    """The reference CPU path restated in C (oracle/cpu_path.c) on the headline GEMV: FP4 E2M1 +
    E8M0/32 W [14336, 4096] decoded to fp32 (materialised), fp32 GEMV, RNE to bf16."""
    import numpy as np

    lib = ctypes.CDLL(str(ROOT / "oracle" / "liboracle_cpu.so"))
    n, k, m = 14336, 4096, 1
    rng = np.random.default_rng(0)
    data = rng.integers(0, 256, n * k // 2).astype(np.uint8)
    e = (127 + rng.integers(-4, 3, (n, k // 32))).astype(np.int64)
    scales = np.ldexp(np.float32(1.0), (e - 127)).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x = ((x.view(np.uint32) + 0x8000) & 0xFFFF0000).view(np.float32)  # bf16-valued activations
    wdeq, yf, y = np.empty(n * k, np.float32), np.empty(m * n, np.float32), np.empty(m * n, np.uint16)
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    i64 = ctypes.c_int64

    def once() -> float:
        t = time.perf_counter()
        lib.oracle_cpu_path(p(data), i64(data.size), 2, i64(n), i64(k), p(scales), i64(32), p(x), i64(m), p(wdeq),
                            p(yf), p(y), 16)
        return time.perf_counter() - t

    med, runs = _time_cpu(once, budget_s)
    nbytes = P.weight_program(P.PackedDesc("fp4_e2m1", (n, k), n * k // 2, 1, "float8_e8m0fnu"), m, "bfloat16", k,
                              "bfloat16", n).estimates.mem
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"the full fp4 e8m0/32 GEMV 14336x4096 M=1 (dequant to fp32 + fp32 GEMV + bf16), "
                      f"median of {runs} runs, {med * 1e3:.1f} ms each", "ms": round(med * 1e3, 3),
            **_host_description()}


def cpu_baseline_int4(budget_s: float) -> dict:
    """The reference CPU path on the INT4 GEMV of the CPU-device configuration, exactly: seed 0,
    x fp16 [1, 4096] ~ N(0, 1); codes uniform in [-8, 7] packed 2 per byte; fp16 group-32 scales
    ~ U(0.005, 0.02); y = fp16(x . deq(W)^T) with fp32 accumulation."""
    import numpy as np

    lib = ctypes.CDLL(str(ROOT / "oracle" / "liboracle_cpu.so"))
    n = k = 4096
    rng = np.random.default_rng(0)
    x = rng.standard_normal((1, k)).astype(np.float16).astype(np.float32)
    codes = rng.integers(-8, 8, (n, k))
    scales = rng.uniform(0.005, 0.02, (n, k // 32)).astype(np.float16).astype(np.float32)
    flat = (codes & 0xF).astype(np.uint8).reshape(-1)
    data = (flat[0::2] | (flat[1::2] << 4)).astype(np.uint8)
    wdeq, yf, y = np.empty(n * k, np.float32), np.empty(n, np.float32), np.empty(n, np.uint16)
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    i64 = ctypes.c_int64

    def once() -> float:
        t = time.perf_counter()
        lib.oracle_cpu_path(p(data), i64(data.size), 0, i64(n), i64(k), p(scales), i64(32), p(x), i64(1), p(wdeq),
                            p(yf), p(y), 17)
        return time.perf_counter() - t

    med, runs = _time_cpu(once, budget_s)
    nbytes = P.weight_program(P.PackedDesc("int4", (n, k), n * k // 2, 1, "float16"), 1, "float16", k, "float16",
                              n).estimates.mem
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"the whole int4 g32 GEMV 4096x4096 M=1 fp16 (dequant to fp32 + fp32 GEMV + fp16), "
                      f"median of {runs} runs, {med * 1e3:.2f} ms each", "ms": round(med * 1e3, 4),
            **_host_description()}


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


def measured_traffic(workload: str) -> int | None:
    """HBM bytes per launch of a workload's dominant kernel from its committed rocprofv3 summary
    (FETCH_SIZE + WRITE_SIZE per dispatch, each scaled by a plain copy of known size)."""
    entry = PROFILES.get(workload)
    path = ROOT / "profiles" / entry[0] if entry else None
    if path is None or not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch="):
            return int(line.split("=", 1)[1])
    return None


# ----------------------------------------------------------------------------- profile summaries
def profile_commands(workload: str) -> list[str]:
    """The rocprofv3 runs a summary is made from (OUT = the folder given to --summarize-profile)."""
    run = f"python3 bench.py --only {workload} --steps 20 --warmup 5"
    if workload.startswith("launch_floor"):  # an empty kernel moves no bytes: its trace is the figure
        return [f"rocprofv3 --kernel-trace --stats --output-format csv -d OUT/kt -o run -- {run}"]
    cmds = [f"rocprofv3 --kernel-trace --stats --output-format csv -d OUT/kt -o run -- {run}",
            f"rocprofv3 --pmc FETCH_SIZE --output-format csv -d OUT/fetch -o run -- {run}",
            f"rocprofv3 --pmc WRITE_SIZE --output-format csv -d OUT/write -o run -- {run}"]
    if "gemm" in workload or "mfma" in workload:
        cmds.append(f"rocprofv3 --pmc MfmaUtil SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE --output-format csv "
                    f"-d OUT/mfma -o run -- {run}")
    cmds += ["rocprofv3 --pmc FETCH_SIZE --output-format csv -d OUT/cfetch -o copy -- python3 bench.py "
             "--copy-calibration 64 --steps 10",
             "rocprofv3 --pmc WRITE_SIZE --output-format csv -d OUT/cwrite -o copy -- python3 bench.py "
             "--copy-calibration 64 --steps 10"]
    return cmds


def _csv_rows(folder: Path, suffix: str) -> list[dict]:
    files = sorted(folder.rglob(f"*{suffix}"))
    if not files:
        raise FileNotFoundError(f"no *{suffix} under {folder}")
    with open(files[0], newline="") as fh:
        return list(csv.DictReader(fh))


def _counter(folder: Path, counter: str, pattern: str) -> tuple[float, int]:
    values: dict[str, float] = {}
    for r in _csv_rows(folder, "counter_collection.csv"):
        if pattern in r["Kernel_Name"] and r["Counter_Name"] == counter:
            key = r.get("Dispatch_Id") or r.get("Correlation_Id") or str(len(values))
            values[key] = values.get(key, 0.0) + float(r["Counter_Value"])
    if not values:
        raise ValueError(f"{counter} has no dispatch of a kernel matching {pattern!r} in {folder}")
    return statistics.median(values.values()), len(values)


def summarize_profile(folder: Path, workload: str) -> str:
    """Text summary of the rocprofv3 runs of ``workload`` under ``folder`` (see profile_commands)."""
    name, pattern = PROFILES[workload]
    run = json.loads((folder / "kt" / "bench.json").read_text())[workload]
    trace = [r for r in _csv_rows(folder / "kt", "kernel_trace.csv") if pattern in r["Kernel_Name"]]
    durations = [int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in trace]
    timed = durations[-run["timed_dispatches"]:]
    if workload.startswith("launch_floor"):
        starts = sorted(int(r["Start_Timestamp"]) for r in trace)[-run["timed_dispatches"]:]
        gaps = [b - a for a, b in zip(starts, starts[1:])]
        return "\n".join([f"# {name[:-4]}", "# rocprofv3 on one MI355X (gfx950); commands run from the repository "
                          "root, OUT = any output folder:", *[f"#   {c}" for c in profile_commands(workload)],
                          "#   (the kernel-trace run's stdout saved as OUT/kt/bench.json)",
                          f"#   python3 bench.py --summarize-profile OUT --only {workload}",
                          f"workload: {run['workload']}", f"kernel: {trace[-1]['Kernel_Name'][:150]}",
                          f"kernel_trace: dispatches={len(durations)} timed={len(timed)}",
                          f"timed dispatch duration: mean_ns={statistics.mean(timed):.0f} "
                          f"median_ns={statistics.median(timed):.0f}",
                          f"start-to-start of consecutive timed dispatches: median_ns={statistics.median(gaps):.0f}",
                          f"bench_ms_per_step_under_trace={run['ms']:.6f} (kernel tracing adds a fixed cost per "
                          "dispatch; the untraced floor is the bench line's launch_floor_448 ms)"]) + "\n"
    fetch, nf = _counter(folder / "fetch", "FETCH_SIZE", pattern)
    write, nw = _counter(folder / "write", "WRITE_SIZE", pattern)
    cfetch, _ = _counter(folder / "cfetch", "FETCH_SIZE", "copyBuffer")
    cwrite, _ = _counter(folder / "cwrite", "WRITE_SIZE", "copyBuffer")
    kf, kw = 65536 / cfetch, 65536 / cwrite
    traffic = int(round((fetch * kf + write * kw) * 1024))
    mean_ns, median_ns = statistics.mean(timed), statistics.median(timed)
    lines = [f"# {name[:-4]}", "# rocprofv3 on one MI355X (gfx950); commands run from the repository root, "
             "OUT = any output folder:"]
    lines += [f"#   {c}" for c in profile_commands(workload)]
    lines += [f"#   (the kernel-trace run's stdout saved as OUT/kt/bench.json)",
              f"#   python3 bench.py --summarize-profile OUT --only {workload}",
              f"workload: {run['workload']}",
              f"kernel: {trace[-1]['Kernel_Name'][:150]}",
              f"kernel_trace: dispatches={len(durations)} timed={len(timed)} (the last {len(timed)} dispatches: "
              f"the timed launches of the bench run)",
              f"timed: mean_ns={mean_ns:.0f} median_ns={median_ns:.0f} min_ns={min(timed)} max_ns={max(timed)}",
              f"bench_ms_per_step_under_trace={run.get('ms', run.get('decode_ms_per_step')):.6f}",
              f"pmc FETCH_SIZE median per dispatch: {fetch:.1f} KiB ({nf} dispatches); WRITE_SIZE: {write:.1f} KiB "
              f"({nw} dispatches)",
              f"copy calibration (64 MiB device copy, copyBuffer kernel): FETCH_SIZE {cfetch:.1f} KiB -> factor "
              f"{kf:.4f}; WRITE_SIZE {cwrite:.1f} KiB -> factor {kw:.4f}",
              f"traffic_bytes_per_launch={traffic}"]
    if "bytes" in run:
        lines += [f"algorithmic_bytes_per_launch={run['bytes']}",
                  f"traffic/algorithmic={traffic / run['bytes']:.4f}"]
    roof = run["roofline"]
    if roof["bound"] == "hbm":
        lines.append(f"achieved_GBps_from_timed_median={run['bytes'] / median_ns:.1f} "
                     f"(frac {run['bytes'] / median_ns / HBM_PEAK_GBS:.4f} of {HBM_PEAK_GBS:.0f})")
    else:
        flops = run["flops"]
        lines.append(f"algorithmic_flops_per_launch={flops}")
        lines.append(f"achieved_TFLOPS_from_timed_median={flops / median_ns / 1e3:.1f} "
                     f"(frac {flops / median_ns / 1e3 / roof['peak']:.4f} of {roof['peak']:.0f}, {roof['peak_of']})")
        util, nb = _counter(folder / "mfma", "MfmaUtil", pattern)
        busy, _ = _counter(folder / "mfma", "SQ_VALU_MFMA_BUSY_CYCLES", pattern)
        active, _ = _counter(folder / "mfma", "GRBM_GUI_ACTIVE", pattern)
        lines.append(f"pmc MfmaUtil median {util:.2f} % ({nb} dispatches): rocprofv3's derived metric, "
                     f"sum(SQ_VALU_MFMA_BUSY_CYCLES) / (max over XCCs of GRBM_GUI_ACTIVE x SIMD count)")
        lines.append(f"pmc SQ_VALU_MFMA_BUSY_CYCLES median {busy:.0f} (summed over SIMDs), GRBM_GUI_ACTIVE {active:.0f} "
                     f"(summed over the 8 XCCs)")
        lines.append(f"shader clock during the kernel = GRBM_GUI_ACTIVE / 8 / timed median = "
                     f"{active / 8 / median_ns:.3f} GHz; peak at that clock = {roof['peak'] * active / 8 / median_ns / 2.4:.0f} "
                     f"TFLOP/s (the nominal peak is quoted at 2.4 GHz)")
    return "\n".join(lines) + "\n"


def _kernel_label(name: str) -> str:
    return name if len(name) <= 100 else name[:100]


def summarize_decoder(folder: Path, workload: str, part: str) -> str:
    """Per-kernel time of the decoder's timed work in a rocprofv3 kernel trace of
    ``bench.py --only decoder_bN`` (stdout saved as DIR/bench.json).  Every prefill and every
    decode step starts with one dec_embed launch; prefills are the segments that run a prompt
    GEMM or prompt attention.  ``decode``: the last 100 steps (the timed graph replays);
    ``prefill``: the second of the three timed prefills."""
    rows = sorted(_csv_rows(folder, "kernel_trace.csv"), key=lambda r: int(r["Start_Timestamp"]))
    starts = [i for i, r in enumerate(rows) if "dec_embed" in r["Kernel_Name"]]
    segments = [rows[a:b] for a, b in zip(starts, starts[1:] + [len(rows)])]
    is_prefill = [any("prefill_attention" in r["Kernel_Name"] or "gemm_w" in r["Kernel_Name"] for r in seg)
                  for seg in segments]
    if part == "prefill":
        chosen = [seg for seg, pf in zip(segments, is_prefill) if pf][-2:-1]
    else:
        last = max(i for i, pf in enumerate(is_prefill) if pf)
        chosen = segments[last + 2:][-100:]  # after the eager first step
    per: dict[str, list[float]] = {}
    for seg in chosen:
        for r in seg:
            per.setdefault(_kernel_label(r["Kernel_Name"]), []).append(
                (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    n = len(chosen)
    busy = sum(sum(v) for v in per.values()) / n
    span = statistics.mean((int(seg[-1]["End_Timestamp"]) - int(seg[0]["Start_Timestamp"])) / 1e3 for seg in chosen)
    run = json.loads((folder / "bench.json").read_text())[workload]
    unit = "step" if part == "decode" else "prefill"
    lines = [f"# {workload}_{part}",
             "# rocprofv3 kernel trace of the 8-layer decoder bench (hidden 4096, INT4 attention, FP4 feed-forward) on one "
             "MI355X (gfx950); commands, from the "
             "repository root (OUT = any output folder):",
             f"#   rocprofv3 --kernel-trace --stats --output-format csv -d OUT -o run -- python3 bench.py --only {workload} "
             "> OUT/bench.json",
             f"#   python3 bench.py --summarize-decoder OUT --only {workload} --part {part}",
             "# Under the tracer every launch is slower (small kernels ~4-5 us each); the untraced step time is the "
             "bench's decode_ms_per_step.",
             f"bench line under the tracer: decode {run['decode_ms_per_step']:.3f} ms/step, prefill "
             f"{run['prefill_ms']:.2f} ms",
             f"summarised: {n} {unit}{'s' if n != 1 else ''}; kernels per {unit}: "
             f"{sum(len(v) for v in per.values()) / n:.1f}; "
             f"busy {busy:.1f} us/{unit}; span {span:.1f} us/{unit}",
             "",
             f"{'us/' + unit:>11}  calls   avg us  kernel"]
    for name, v in sorted(per.items(), key=lambda kv: -sum(kv[1])):
        lines.append(f"{sum(v) / n:11.2f} {len(v) / n:6.1f} {statistics.mean(v):8.2f}  {name}")
    return "\n".join(lines) + "\n"


# ----------------------------------------------------------------------------- main
def main() -> int:
    args = parse()
    if args.summarize_decoder is not None:
        if not (args.only or "").startswith("decoder"):
            print("--summarize-decoder needs --only decoder_b1 or decoder_b8", file=sys.stderr)
            return 2
        print(summarize_decoder(args.summarize_decoder, args.only, args.part), end="")
        return 0
    if args.summarize_profile is not None:
        if not args.only:
            print("--summarize-profile needs --only WORKLOAD", file=sys.stderr)
            return 2
        print(summarize_profile(args.summarize_profile, args.only), end="")
        return 0
    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark runs on one GPU; --gpus must be 1 (multi-GPU sharding is "
                                   "design-only)"}))
        return 2
    import torch

    from tinygrad_mi355x.runtime import kernels as K

    dev = torch.device("cuda:0")
    if args.copy_calibration:
        copy_calibration(torch, args.copy_calibration, args.steps)
        return 0
    K.load_library()
    steps, warmup = args.steps, args.warmup
    gemm_steps = max(min(steps, 50), 10)
    workloads = {
        "fp4_gemv_m1": lambda: fp4_gemv_workload(torch, K, dev, 1, steps, warmup),
        "fp4_gemv_m4": lambda: fp4_gemv_workload(torch, K, dev, 4, steps, warmup),
        "fp4_gemv_m16": lambda: fp4_gemv_workload(torch, K, dev, 16, steps, warmup),
        "int4_gemv_n4096": lambda: int4_gemv_workload(torch, K, dev, 4096, steps, warmup),
        "int4_gemv_n14336": lambda: int4_gemv_workload(torch, K, dev, 14336, steps, warmup),
        "fp6_e3m2_gemm_m2048": lambda: fp6_gemm_workload(torch, K, dev, "fp6_e3m2", gemm_steps, 20),
        "fp6_e2m3_gemm_m2048": lambda: fp6_gemm_workload(torch, K, dev, "fp6_e2m3", gemm_steps, 20),
        # the vendor comparison (a child process) and the zero-operand timing are left out of --only runs
        # (profiles take a run's last launches as its timed ones)
        "fp4_gemm_8192": lambda: fp4_gemm_workload(torch, K, dev, 8192, 8192, 8192, gemm_steps, 20, not args.only,
                                                   not args.only),
        "fp4_gemm_4096x14336x4096": lambda: fp4_gemm_workload(torch, K, dev, 4096, 14336, 4096, gemm_steps, 20,
                                                               not args.only),
        "decoder_b1": lambda: decoder_workload(torch, dev, 1),
        "decoder_b8": lambda: decoder_workload(torch, dev, 8),
        "read_ceiling_31232000": lambda: read_ceiling_workload(torch, K, dev, 31_232_000, steps, warmup),
        "read_ceiling_9453568": lambda: read_ceiling_workload(torch, K, dev, 9_453_568, steps, warmup),
        "read_ceiling_470000000": lambda: read_ceiling_workload(torch, K, dev, 470_000_000, steps, warmup),
        "mfma_fp4_ceiling_8192": lambda: mfma_ceiling_workload(torch, K, dev, gemm_steps, 20),
        "launch_floor_448": lambda: launch_floor_workload(torch, K, dev, 448, steps, warmup),
        "fp4_gemv_shard_n1792_m1": lambda: fp4_gemv_workload(torch, K, dev, 1, steps, warmup, 1792),
        "fp4_gemv_shard_n1792_m4": lambda: fp4_gemv_workload(torch, K, dev, 4, steps, warmup, 1792),
        "fp4_gemv_shard_n1792_m16": lambda: fp4_gemv_workload(torch, K, dev, 16, steps, warmup, 1792),
        "bf16_gemm_8192": lambda: dense_gemm_workload(torch, K, dev, "bfloat16", 8192, gemm_steps, 20, not args.only),
        "fp8_gemm_8192": lambda: dense_gemm_workload(torch, K, dev, "float8_e4m3fn", 8192, gemm_steps, 20),
        "uop_rowsum_16384x4096": lambda: uop_rowsum_workload(steps, warmup),
        "uop_gemm_bf16_4096_relu": lambda: uop_gemm_workload(gemm_steps, 20),
    }
    if args.only:
        print(json.dumps({args.only: workloads[args.only]()}))
        return 0
    torch.cuda.synchronize()
    wall = time.perf_counter()
    primary = workloads[PRIMARY]()
    extras = {} if args.no_extras else {name: workloads[name]() for name in EXTRAS}
    torch.cuda.synchronize()
    gpu_wall = time.perf_counter() - wall
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline_fp4(args.cpu_seconds)
        if "int4_gemv_n4096" in extras:
            extras["int4_gemv_n4096"]["cpu_baseline"] = cpu_baseline_int4(args.cpu_seconds)
    for name, w in extras.items():
        if name in PROFILES and "roofline" in w:
            w["roofline"]["traffic"] = measured_traffic(name)
    roofline = dict(primary["roofline"], traffic=measured_traffic(PRIMARY))
    floor = extras.get("launch_floor_448")
    if floor:
        # what one launch of this many bytes can reach here: the empty kernel's time on the same
        # grid, in the same graphs, plus the bytes at the HBM peak
        roofline["launch_floor_ms"] = round(floor["ms"], 6)
        roofline["single_launch_ceiling_frac"] = floor["ceiling_frac_31232000"]
    line = {
        "metric": "low-bit GEMV GB/s (% HBM peak) + FP4 GEMM TFLOPS (% MFMA peak), 1 GPU",
        "value": roofline["achieved"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(primary["ms"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp4_e2m1 x bf16 -> fp32 acc -> bf16",
        "data": (f"synthetic (uniform E2M1 codes, E8M0 exponents 123..129, N(0,1) bf16 activations), "
                 f"{primary['copies']} rotating weight copies ({primary['copy_set_bytes'] / 1e6:.0f} MB)"),
        "config": {"workload": primary["workload"], "N": 14336, "K": 4096, "M": 1, "block": 32,
                   "launch": (f"median of {primary['trials']} trials, each a HIP graph of exactly {steps} steps "
                              f"timed with HIP events"),
                   "parallelism": "single GPU"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "workloads": {name: {k: (round(v, 6) if isinstance(v, float) else v) for k, v in w.items()}
                      for name, w in extras.items()},
        "gpu_wall_s": round(gpu_wall, 2),
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
