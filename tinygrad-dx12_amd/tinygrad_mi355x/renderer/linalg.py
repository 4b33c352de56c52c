"""Fixed gfx950 matrix-kernel table and accumulator policy.

The reference asks the D3D12 runtime at run time which LinAlg operations exist
(alexandreteles/tinygrad-dx12 src/tinygrad_dx12/codegen/linalg.py:18-34, :90-133;
runtime/support/dx12.py:298-336) and renders HLSL for the accepted one
(renderer/linalg.py:38-166).  On MI355X the set of kernels is known at build time,
so selection is a static table over operand kinds; the kernels themselves are
compiled into libtgm_mi355x.so.
"""

from __future__ import annotations

import torch

from tinygrad_mi355x import dtype as D
from tinygrad_mi355x.renderer.matrix import (GEMM_DENSE, GEMM_FP8, GEMM_MX, GEMM_MX_GENERAL, GEMM_W, GEMV,  # noqa: F401
                                             GEMV_MAX_ROWS, PLAIN, MatrixKernel, mx_kernel)


def _accumulator(a: torch.dtype, b: torch.dtype) -> torch.dtype:
    """Default matrix accumulator: strong(sum_acc(strong(least_upper(a, b)))) (renderer/linalg.py:33-35)."""
    return D.strong_dtype(D.sum_acc_dtype(D.strong_dtype(D.least_upper_dtype(a, b))))


DENSE_DTYPES = (torch.bfloat16, torch.float16)
FP8_DTYPES = (torch.float8_e4m3fn, torch.float8_e5m2)
ACTIVATION_DTYPES = (torch.bfloat16, torch.float16, torch.float32)
OUTPUT_DTYPES = (torch.bfloat16, torch.float16, torch.float32)
WEIGHT_SCALE_DTYPES = (torch.float8_e8m0fnu, torch.float16, torch.bfloat16, torch.float32)
