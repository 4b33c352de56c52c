"""ctypes binding of the gfx950 kernel library ``libtgm_mi355x.so`` (include/tgm_packed.h,
include/tgm_decoder.h), with no torch dependency.

This is the only route from Python into the packed kernels: the plugin-buffer path
(``codegen/program.py``) calls it with plugin buffer addresses and the device stream, the
torch adapter (``runtime/kernels.py``) with tensor addresses and torch's stream.  There is no
CPU implementation behind it: when the library is missing or no MI355X is visible, every call
raises.  The library links the HIP runtime by soname (libamdhip64.so.7); the runtime binding
(``support/hip.py``) is opened first, so the library binds to the one runtime the process
shares with torch.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_NAME = "libtgm_mi355x.so"
LIB_PATH = Path(__file__).resolve().parent.parent / "_lib" / LIB_NAME
ABI_VERSION = 1

# enum tgm_format
FORMAT_IDS = {"int4": 0, "uint4": 1, "fp4_e2m1": 2, "fp6_e2m3": 3, "fp6_e3m2": 4}
# enum tgm_dtype, by dtype name (the torch / tinygrad spelling) and its element size in bytes
DTYPE_IDS = {
    "bool": 0, "int8": 1, "uint8": 2, "int16": 3, "uint16": 4, "int32": 5, "uint32": 6, "int64": 7, "uint64": 8,
    "float8_e4m3fn": 9, "float8_e5m2": 10, "float16": 11, "bfloat16": 12, "float32": 13, "float64": 14,
    "float8_e8m0fnu": 15,
}
DTYPE_SIZES = {
    "bool": 1, "int8": 1, "uint8": 1, "int16": 2, "uint16": 2, "int32": 4, "uint32": 4, "int64": 8, "uint64": 8,
    "float8_e4m3fn": 1, "float8_e5m2": 1, "float16": 2, "bfloat16": 2, "float32": 4, "float64": 8,
    "float8_e8m0fnu": 1,
}
TGM_OK, TGM_E_INVALID, TGM_E_UNSUPPORTED = 0, -1, -2


class UnsupportedKernel(RuntimeError):
    """No kernel of the requested family covers this operand combination."""


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None

_I64, _INT, _P = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p
SIGNATURES = {
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
    "tgm_device_arch": (_INT, ctypes.c_char_p, _I64),
    "tgm_probe_read": (_P, _I64, _P, _P),
    "tgm_probe_mfma_fp4": (_I64, _I64, _P, _P),
    "tgm_probe_launch": (_I64, _I64, _P, _P),
    "tgm_probe_bf16_rounding": (ctypes.c_uint32, _I64, _P, _P, _P),
    # decoder-step kernels (include/tgm_decoder.h)
    "tgm_dec_embed": (_P, _I64, _I64, _P, _I64, _P, _P),
    "tgm_dec_add_rmsnorm": (_P, _P, _I64, _I64, _P, ctypes.c_float, _P, _INT, _P),
    "tgm_dec_add_rmsnorm_parts": (_P, _P, _I64, _I64, _I64, _I64, _P, ctypes.c_float, _P, _INT, _P),
    "tgm_dec_gemv_parts": (_P, _INT, _I64, _I64, _P, _INT, _I64, _P, _INT, _I64, _I64, _P, _I64, _I64, _P),
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
           "tgm_gemm_w_split_noalloc_capacity", *SIGNATURES)


def library_path() -> Path:
    return Path(os.environ.get("MI355X_KERNEL_LIB", str(LIB_PATH)))


def load_library() -> ctypes.CDLL:
    """Load (once) and type the kernel library; raises if it is missing or stale."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not path.exists():
            raise RuntimeError(f"MI355X kernel library {path} is not built; run __graft_entry__.build()")
        from tinygrad_mi355x.runtime.support import hip

        hip.library()  # the process's one HIP runtime, before the library's soname is resolved
        lib = ctypes.CDLL(str(path))
        lib.tgm_abi_version.restype = ctypes.c_int
        lib.tgm_abi_version.argtypes = ()
        lib.tgm_last_error.restype = ctypes.c_char_p
        lib.tgm_last_error.argtypes = ()
        if lib.tgm_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{path} has ABI {lib.tgm_abi_version()}, expected {ABI_VERSION}")
        for name, args in SIGNATURES.items():
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


def device_arch(ordinal: int) -> str:
    """Architecture name of HIP device ``ordinal`` without target features (e.g. "gfx950")."""
    buf = ctypes.create_string_buffer(256)
    call("tgm_device_arch", ordinal, buf, len(buf))
    return buf.value.decode().split(":")[0]
