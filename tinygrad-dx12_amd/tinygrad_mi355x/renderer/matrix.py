"""Fixed gfx950 matrix-kernel table (no torch).

The reference asks the D3D12 runtime at run time which LinAlg operations exist
(alexandreteles/tinygrad-dx12 src/tinygrad_dx12/codegen/linalg.py:18-34, :90-133;
runtime/support/dx12.py:298-336) and renders HLSL for the accepted one
(renderer/linalg.py:38-166).  On MI355X the set of kernels is known at build time: each
family is one C-ABI entry point of libtgm_mi355x.so with a fixed tile and workgroup size.
"""

from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class MatrixKernel:
    """One native kernel family: the scope name it answers to, its tile and workgroup size."""

    name: str  # C-ABI entry point
    scope: str  # reference scope it replaces
    tile: tuple[int, int, int]  # (rows of W / C per workgroup, activation rows, K per step)
    threads: int


# Family 1: fused dequant GEMV / skinny GEMM (replaces thread_source and the N=1 linalg_source).
GEMV = MatrixKernel("tgm_gemv", "Wave", (16, 16, 128), 256)
# Family 2: dequant-to-bf16 MFMA GEMM (replaces linalg_source for one packed operand).
GEMM_W = MatrixKernel("tgm_gemm_w", "ThreadGroup", (256, 128, 128), 512)
# Family 2: scaled-MFMA GEMM of two packed FP4 / FP6 operands, each with E8M0 block-32 scales or
# unscaled.  One entry point, two kernels: FP4 x FP4 with both scales and K a multiple of 256
# runs 256 x 256 tiles with K steps of 256 (GEMM_MX); every other pair, or K a multiple of 128
# only, runs 256 x 128 tiles with K steps of 128 (GEMM_MX_GENERAL).  ``mx_kernel`` picks.
GEMM_MX = MatrixKernel("tgm_gemm_mx", "ThreadGroup", (256, 256, 256), 512)
GEMM_MX_GENERAL = MatrixKernel("tgm_gemm_mx", "ThreadGroup", (256, 128, 128), 512)
# Family 2: ordinary bf16 x bf16 / f16 x f16 MFMA GEMM (the reference's LinAlg lowering of an
# ordinary matrix product, codegen/matmul.py:156-246).
GEMM_DENSE = MatrixKernel("tgm_gemm_dense", "ThreadGroup", (256, 128, 64), 512)
# The same entry point's persistent kernel for one large product (K a multiple of 128 and at least
# one round of 256 x 256 tiles on the device's CUs): 256 x 256 tiles, K steps of 64, one workgroup
# per CU walking its tiles.  ``dense_kernel`` picks.
GEMM_DENSE_STREAM = MatrixKernel("tgm_gemm_dense", "ThreadGroup", (256, 256, 64), 512)
# Family 2: ordinary FP8 x FP8 GEMM, the FP8 values decoded exactly to bf16 in registers for the
# dense GEMM's MFMA (the reference's LinAlg takes FP8 operands as they are, renderer/linalg.py:12-13).
GEMM_FP8 = MatrixKernel("tgm_gemm_fp8", "ThreadGroup", (256, 128, 128), 512)
# Exact-width fallback (the reference's ordinary matmul); never a "native" candidate.
PLAIN = MatrixKernel("tgm_gemm_plain", "tiled", (16, 16, 1), 256)

GEMV_MAX_ROWS = 16
MI355X_CUS = 256  # compute units of one MI355X


def dense_kernel(m: int, n: int, k: int, batch: int = 1, cus: int = MI355X_CUS) -> MatrixKernel:
    """The kernel tgm_gemm_dense launches for a bf16 / f16 product (tgm_gemm_dense.hip's choice)."""
    tiles = -(-m // GEMM_DENSE_STREAM.tile[0]) * -(-n // GEMM_DENSE_STREAM.tile[1])
    stream = batch == 1 and k > 0 and k % 128 == 0 and cus >= 8 and tiles >= cus
    return GEMM_DENSE_STREAM if stream else GEMM_DENSE


def mx_kernel(a_format: str, a_scaled: bool, b_format: str, b_scaled: bool, k: int) -> MatrixKernel:
    """The kernel tgm_gemm_mx launches for a pair of packed operands (both E8M0/32-scaled or not)."""
    fp4_pair = a_format == b_format == "fp4_e2m1" and a_scaled and b_scaled
    return GEMM_MX if fp4_pair and k > 0 and k % GEMM_MX.tile[2] == 0 else GEMM_MX_GENERAL
