"""Ablations of the FP4 x FP4 GEMM (csrc/tgm_gemm_mx.hip): where its time goes.

Each variant is the committed kernel source with one literal edit, built into a library of its
own under _build/ablation/<variant>/ (linked with the other objects of the last build_library()
run) and timed by bench.py in a child process pointed at that library (MI355X_KERNEL_LIB), all
in one call so that every variant runs on the same GPU:

    python tinygrad-dx12_amd/ablation/gemm_mx.py build          # here (hipcc cross-compiles)
    python tinygrad-dx12_amd/ablation/gemm_mx.py run [--rounds 2] [--steps 50]   # on the GPU

Variants that remove work compute wrong products by design: they exist to be timed.  No edit
changes an address, a loop bound or a wait count, so every variant reads and writes exactly
the memory the committed kernel does and every wait ends.

    baseline                the committed kernel
    l2_hot_panels           every K step of a tile loads the tile's first two steps' panels
                            again (a working set that stays in L2): the cost of global-load
                            latency and L2 misses
    no_step_barrier         the persistent kernel's barrier between steps removed (LDS races)
    quarter_fragment_reads  three of four substeps skip their LDS fragment reads and reuse
                            registers: the cost of the LDS operand traffic
    reads_in_use_order      each substep's fragment reads issued in the order the next
                            substep's MFMAs consume them (A0, B0 .. B3, A1)
    front_loaded_reads      fragment and scale reads spread over the first half of a substep's
                            MFMAs, the panel loads over the second half
    front_loaded_in_use_order   both
    no_c_stores             the epilogue's C stores left out (no output): the cost of the
                            tile switch's store drain (every step waits on vmcnt(0), which
                            counts stores as well as loads).  (Ordinary against non-temporal C
                            stores, measured the same way: 251.4 against 253.0 us at 8192^3;
                            the kernel now uses ordinary ones.)
    group_m_4 / group_m_16  XCD tile groups 4 or 16 row panels deep instead of 8
    no_scale_reads          the E8M0 words are never read from LDS (each substep keeps the
                            prologue's): the cost of the scale reads
    no_scale_batches        the E8M0 batches are never loaded into LDS: the cost of their loads
    bf16_mfma               the bf16 MFMA (same cycles per instruction) on the same fragments
                            instead of the scaled FP4 MFMA: the cost of the instruction itself
    launch_per_tile         the launch-per-tile kernel instead of the persistent one
    waves_2x2               launch per tile, 4 waves of 128 x 128 (one wave per SIMD)
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parents[1]
ROOT = PKG.parent
sys.path.insert(0, str(PKG))

from tinygrad_mi355x.build import ARCH, BUILD, FLAGS, HIPCC, LIB, build_library  # noqa: E402

SRC = PKG / "csrc" / "tgm_gemm_mx.hip"
OUT = BUILD / "ablation"
WORKLOADS = ("fp4_gemm_8192", "fp4_gemm_4096x14336x4096")

STREAM = "gemm_mx_fp4_stream(const uint8_t"
PERSISTENT = "if (k % (kBK * kBatchSteps) == 0 && cus >= 8 && tiles >= 8) {"
# fragment reads in the order the next substep's MFMAs consume them: A0, B0 .. B3, A1 (FA = 2)
READ_IN_USE_ORDER = "else read_item(fn, rbuf, ru, it == 0 ? 0 : it == FA + FB - 1 ? 1 : it + 1);"
# fragment and scale reads spread over the first half of a substep's MFMAs, panel loads over the second
FRONT_LOADED = ("(it < nr ? it * (FA * FB / 2) / nr : FA * FB / 2 + (it - nr) * (FA * FB / 2) / (ni - nr + 1)) "
                "== idx")  # reads (and raw scales) in the first half of a substep's MFMAs, the rest in the second
C_STORE = "*(u32x4*)out = *(const u32x4*)(ep + r * 32 + cc);"
SCALE_READ_A = "if (t < FA) sraw_a[t < FA ? t : 0] = *(const u32x2*)(ls + (wm * FA * 32 + t * 32 + (lane & 31)) * kBatchRow);"
SCALE_READ_B = ("else sraw_b[t < FA ? 0 : t - FA] =\n"
                "        *(const u32x2*)(ls + kBM * kBatchRow + (wn * FB * 32 + (t - FA) * 32 + (lane & 31)) * kBatchRow);")
MX_MFMA = ("acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa, fb, acc[i][j], 4, 4, u, (int)xa[i], u,\n"
           "                                                                    (int)xb[j]);")
BF16_MFMA = ("acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(__attribute__((__vector_size__(16))) __bf16, f.a[i]),\n"
             "            __builtin_bit_cast(__attribute__((__vector_size__(16))) __bf16, f.b[j]), acc[i][j], 0, 0, 0); (void)fa; (void)fb; (void)xa; (void)xb;")
# (anchor that must precede the edit, old text, new text)
VARIANTS: dict[str, list[tuple[str, str, str]]] = {
    "baseline": [],
    "l2_hot_panels": [(STREAM, "(unsigned)at.m0 * kb + (unsigned)(at.st * kRowBytes)",
                       "(unsigned)at.m0 * kb + (unsigned)((at.st & 1) * kRowBytes)"),
                      (STREAM, "(unsigned)at.n0 * kb + (unsigned)(at.st * kRowBytes)",
                       "(unsigned)at.n0 * kb + (unsigned)((at.st & 1) * kRowBytes)")],
    "no_step_barrier": [(STREAM, "    wait_lds_dma();\n    __syncthreads();\n    substep(f1, U3{},",
                         "    wait_lds_dma();\n    __builtin_amdgcn_sched_barrier(0);\n    substep(f1, U3{},")],
    "quarter_fragment_reads": [(STREAM, "else read_item(fn, rbuf, ru, it);",
                                "else { if (ru == 0) read_item(fn, rbuf, ru, it); }")],
    "reads_in_use_order": [(STREAM, "else read_item(fn, rbuf, ru, it);", READ_IN_USE_ORDER)],
    "front_loaded_reads": [(STREAM, "it * FA * FB / ni == idx", FRONT_LOADED)],
    "front_loaded_in_use_order": [(STREAM, "it * FA * FB / ni == idx", FRONT_LOADED),
                                  (STREAM, "else read_item(fn, rbuf, ru, it);", READ_IN_USE_ORDER)],
    "no_c_stores": [(STREAM, C_STORE, "(void)out;")],
    "no_scale_reads": [(STREAM, SCALE_READ_A, "if (t < FA) { }"), (STREAM, SCALE_READ_B, "else { }")],
    "no_scale_batches": [(STREAM, "    lds_dma16(rsa, la, (unsigned)(at.m0 + r) * kblk + boff);\n"
                                  "    lds_dma16(rsb, la + kBM * kBatchRow, (unsigned)(at.n0 + r) * kblk + boff);",
                          "    (void)la; (void)r; (void)boff;")],
    "bf16_mfma": [(STREAM, MX_MFMA, BF16_MFMA)],
    "group_m_4": [("constexpr int kGroupM = 8;", "constexpr int kGroupM = 8;", "constexpr int kGroupM = 4;")],
    "group_m_16": [("constexpr int kGroupM = 8;", "constexpr int kGroupM = 8;", "constexpr int kGroupM = 16;")],
    "launch_per_tile": [("extern \"C\"", PERSISTENT, "if (false) {")],
    "waves_2x2": [("extern \"C\"", PERSISTENT, "if (false) {"),
                  ("extern \"C\"", "hipLaunchKernelGGL((gemm_mx_fp4<kWavesM, kWavesN>), dim3((unsigned)tiles), "
                                   "dim3(kWavesM * kWavesN * 64)",
                   "hipLaunchKernelGGL((gemm_mx_fp4<2, 2>), dim3((unsigned)tiles), dim3(256)")],
}


def patched(name: str) -> str:
    src = SRC.read_text()
    for anchor, old, new in VARIANTS[name]:
        start = src.index(anchor)
        at = src.find(old, start)
        if at < 0:
            raise SystemExit(f"{name}: {old!r} not found after {anchor!r}: the kernel changed, update the ablation")
        src = src[:at] + new + src[at + len(old):]
    return src


def build(names: list[str]) -> None:
    build_library()
    others = [p for p in sorted(BUILD.glob("*.o")) if p.name != "tgm_gemm_mx.o"]
    for name in names:
        d = OUT / name
        d.mkdir(parents=True, exist_ok=True)
        src = d / "tgm_gemm_mx.hip"
        src.write_text(patched(name))
        obj, lib = d / "tgm_gemm_mx.o", d / LIB.name
        for cmd in ([HIPCC, *FLAGS, "-c", str(src), "-o", str(obj)],
                    [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, others), str(obj), "-o", str(lib)]):
            proc = subprocess.run(cmd, capture_output=True, text=True)
            if proc.returncode != 0:
                raise SystemExit(f"{name}: {proc.stderr}")
        print(f"built {lib}", flush=True)


def time_variant(name: str, workload: str, steps: int) -> float:
    env = dict(os.environ, MI355X_KERNEL_LIB=str(OUT / name / LIB.name))
    cmd = [sys.executable, str(ROOT / "bench.py"), "--only", workload, "--steps", str(steps), "--warmup", "10",
           "--no-cpu-baseline"]
    proc = subprocess.run(cmd, env=env, capture_output=True, text=True, timeout=240)
    if proc.returncode != 0:
        raise SystemExit(f"{name} {workload}: {proc.stderr[-2000:]}")
    return json.loads(proc.stdout.strip().splitlines()[-1])[workload]["ms"] * 1e3


def run(names: list[str], rounds: int, steps: int) -> None:
    times: dict[tuple[str, str], list[float]] = {}
    for r in range(rounds):
        for name in names:
            for w in WORKLOADS:
                us = time_variant(name, w, steps)
                times.setdefault((name, w), []).append(us)
                print(f"round {r} {name} {w}: {us:.1f} us", flush=True)
    print("\n| variant | " + " | ".join(WORKLOADS) + " |")
    print("| --- |" + " --- |" * len(WORKLOADS))
    for name in names:
        cells = []
        for w in WORKLOADS:
            med, base = statistics.median(times[(name, w)]), statistics.median(times[("baseline", w)])
            cells.append(f"{med:.1f} us ({med / base:.3f})")
        print(f"| {name} | " + " | ".join(cells) + " |")


if __name__ == "__main__":
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("action", choices=("build", "run"))
    ap.add_argument("--rounds", type=int, default=2)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--variants", nargs="+", choices=sorted(VARIANTS), default=list(VARIANTS),
                    help="variants to build or time (baseline is always included)")
    a = ap.parse_args()
    names = ["baseline"] + [v for v in a.variants if v != "baseline"]
    build(names) if a.action == "build" else run(names, a.rounds, a.steps)
