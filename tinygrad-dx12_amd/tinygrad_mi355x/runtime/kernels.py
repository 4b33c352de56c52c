"""ctypes binding of the gfx950 kernel library ``libtgm_mi355x.so`` (include/tgm_packed.h,
include/tgm_decoder.h).

This is the only route from Python into the packed kernels.  There is no CPU
implementation behind it: when the library is missing or no MI355X is visible,
every call raises.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

LIB_NAME = "libtgm_mi355x.so"
LIB_PATH = Path(__file__).resolve().parent.parent / "_lib" / LIB_NAME
ABI_VERSION = 1

# enum tgm_format
FORMAT_IDS = {"int4": 0, "uint4": 1, "fp4_e2m1": 2, "fp6_e2m3": 3, "fp6_e3m2": 4}
# enum tgm_dtype
DTYPE_IDS = {
    torch.bool: 0, torch.int8: 1, torch.uint8: 2, torch.int16: 3, torch.uint16: 4, torch.int32: 5,
    torch.uint32: 6, torch.int64: 7, torch.uint64: 8, torch.float8_e4m3fn: 9, torch.float8_e5m2: 10,
    torch.float16: 11, torch.bfloat16: 12, torch.float32: 13, torch.float64: 14, torch.float8_e8m0fnu: 15,
}
TGM_OK, TGM_E_INVALID, TGM_E_UNSUPPORTED = 0, -1, -2


class UnsupportedKernel(RuntimeError):
    """No kernel of the requested family covers this operand combination."""


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None

_I64, _INT, _P = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p
_SIGNATURES = {
    "tgm_unpack": (_P, _I64, _INT, _I64, _I64, _P, _INT, _I64, _P, _INT, _P),
    "tgm_gemv": (_P, _INT, _I64, _I64, _P, _INT, _I64, _P, _INT, _I64, _I64, _P, _INT, _I64, _P),
    "tgm_gemm_w": (_P, _INT, _I64, _I64, _P, _INT, _I64, _I64, _P, _INT, _I64, _P, _INT, _I64, _P),
    "tgm_gemm_w_swiglu": (_P, _INT, _I64, _I64, _P, _INT, _I64, _I64, _P, _INT, _I64, _P, _INT, _I64, _P),
    "tgm_gemm_w_split": (_P, _INT, _I64, _I64, _P, _INT, _I64, _I64, _P, _INT, _I64, _P, _INT, _I64, _I64, _P, _I64,
                         _P),
    "tgm_gemm_w_split_noalloc": (_P, _INT, _I64, _I64, _P, _INT, _I64, _I64, _P, _INT, _I64, _P, _INT, _I64, _I64,
                                 _P),
    "tgm_gemm_mx": (_P, _INT, _P, _I64, _P, _INT, _P, _I64, _I64, _P, _INT, _I64, _P),
    "tgm_gemm_fp8": (_P, _INT, _I64, _I64, _P, _INT, _I64, _I64, _I64, _P, _P, _P, _INT, _I64, _P),
    "tgm_gemm_plain": (_P, _INT, _I64, _I64, _P, _INT, _I64, _I64, _P, _INT, _I64, _I64, _I64, _I64, _I64, _INT, _P),
    "tgm_quantize_mx": (_P, _INT, _I64, _I64, _INT, _I64, _P, _P, _P),
    "tgm_pack_codes": (_P, _I64, _INT, _P, _P),
    "tgm_gemm_dense": (_P, _INT, _I64, _I64, _P, _INT, _I64, _I64, _I64, _P, _INT, _I64, _P),
    "tgm_gemm_dense_batched": (_P, _INT, _I64, _I64, _I64, _P, _INT, _I64, _I64, _I64, _I64, _I64, _P, _INT, _I64, _I64,
                               _I64, _I64, _I64, _P),
    "tgm_gemv_swiglu": (_P, _INT, _I64, _I64, _P, _INT, _I64, _P, _INT, _I64, _I64, _P, _INT, _I64, _P),
    "tgm_transpose16": (_P, _I64, _I64, _I64, _P, _I64, _P),
    "tgm_transpose8": (_P, _I64, _I64, _I64, _P, _I64, _P),
    # decoder-step kernels (include/tgm_decoder.h)
    "tgm_dec_embed": (_P, _I64, _I64, _P, _I64, _P, _P),
    "tgm_dec_add_rmsnorm": (_P, _P, _I64, _I64, _P, ctypes.c_float, _P, _INT, _P),
    "tgm_dec_rope_kv": (_P, _I64, _I64, _I64, _I64, _I64, _P, ctypes.c_double, _P, _P, _I64, _P, _P, _P, _I64, _I64,
                        _P),
    "tgm_dec_causal_softmax": (_P, _I64, _I64, _I64, ctypes.c_float, _P, _I64, _I64, _P),
    "tgm_dec_prefill_attention": (_P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _I64, _P, _INT, _P),
    "tgm_dec_norm_gemv": (_P, _P, _P, _P, ctypes.c_float, _P, _INT, _I64, _I64, _P, _INT, _I64, _P, _INT, _INT, _P),
    "tgm_dec_attention": (_P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _I64, ctypes.c_double, _I64, _P, _I64, _P, _INT,
                          _P),
    "tgm_dec_silu_mul": (_P, _I64, _I64, _P, _INT, _P),
    "tgm_dec_gemv_bf16": (_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _P),
    "tgm_dec_argmax": (_P, _I64, _I64, _I64, _P, _P, _P, _I64, _I64, _P),
}
EXPORTS = ("tgm_abi_version", "tgm_last_error", "tgm_dec_attention_workspace", "tgm_gemm_w_split_workspace",
           "tgm_gemm_w_split_noalloc_capacity", *_SIGNATURES)


def library_path() -> Path:
    return Path(os.environ.get("MI355X_KERNEL_LIB", str(LIB_PATH)))


def load_library() -> ctypes.CDLL:
    """Load (once) and type the kernel library; raises if it is missing or stale.

    torch is imported first so that the HIP runtime torch ships is the one the
    library binds to (both carry the soname libamdhip64.so.7).
    """
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not path.exists():
            raise RuntimeError(f"MI355X kernel library {path} is not built; run __graft_entry__.build()")
        lib = ctypes.CDLL(str(path))
        lib.tgm_abi_version.restype = ctypes.c_int
        lib.tgm_abi_version.argtypes = ()
        lib.tgm_last_error.restype = ctypes.c_char_p
        lib.tgm_last_error.argtypes = ()
        if lib.tgm_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{path} has ABI {lib.tgm_abi_version()}, expected {ABI_VERSION}")
        for name, args in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        lib.tgm_dec_attention_workspace.argtypes = (_I64, _I64, _I64, _I64)
        lib.tgm_dec_attention_workspace.restype = _I64
        lib.tgm_gemm_w_split_workspace.argtypes = (_I64, _I64, _I64)
        lib.tgm_gemm_w_split_workspace.restype = _I64
        lib.tgm_gemm_w_split_noalloc_capacity.argtypes = ()
        lib.tgm_gemm_w_split_noalloc_capacity.restype = _I64
        _lib = lib
        return lib


def check(name: str, status: int) -> None:
    """Map a tgm status to the reference's exception conventions (ValueError / RuntimeError)."""
    if status == TGM_OK:
        return
    message = (load_library().tgm_last_error() or b"").decode(errors="replace")
    if status == TGM_E_INVALID:
        raise ValueError(f"{name}: {message}")
    if status == TGM_E_UNSUPPORTED:
        raise UnsupportedKernel(f"{name}: {message}")
    raise RuntimeError(f"{name} failed: {status} ({message})")


def call(name: str, *args) -> None:
    check(name, getattr(load_library(), name)(*args))


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
