"""Torch adapter of the kernel library binding (``runtime/library.py``).

The library binding itself is torch-free; this module adds what the torch-facing API needs:
torch dtype ids, the current torch stream of a tensor's device and the device check.  There
is no CPU implementation behind it: when the library is missing or no MI355X is visible,
every call raises.
"""

from __future__ import annotations

import torch

from tinygrad_mi355x.runtime import library as L
from tinygrad_mi355x.runtime.support import hip as _hip
from tinygrad_mi355x.runtime.library import (ABI_VERSION, EXPORTS, FORMAT_IDS, LIB_NAME, LIB_PATH, TGM_E_INVALID,  # noqa: F401
                                             TGM_E_UNSUPPORTED, TGM_OK, UnsupportedKernel, check, library_path,
                                             load_library)

_hip.check_single_runtime()  # torch's runtime and the one the plugin opened must be one

_SIGNATURES = L.SIGNATURES
# enum tgm_dtype by torch dtype
DTYPE_IDS = {getattr(torch, name): i for name, i in L.DTYPE_IDS.items()}


def call(name: str, *args) -> None:
    L.call(name, *args)


def dtype_id(dt: torch.dtype) -> int:
    if dt not in DTYPE_IDS:
        raise ValueError(f"dtype {dt} is not supported by the MI355X kernels")
    return DTYPE_IDS[dt]


def require_device(t: torch.Tensor) -> None:
    """The packed kernels run only on a HIP device; there is no CPU implementation."""
    if t.device.type != "cuda":
        raise RuntimeError(
            f"the MI355X packed path needs tensors on the HIP device (torch 'cuda'), got {t.device}; "
            "this backend has no CPU implementation")


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
