"""HIP C++ kernel renderer for gfx950.

Counterpart of ``DX12Renderer`` (alexandreteles/tinygrad-dx12
src/tinygrad_dx12/renderer/cstyle.py:303-380): it holds the target, the launch limits
and the supported arithmetic dtypes, serialises rendering with a lock, keeps the
per-renderer matrix rejection cache, and owns the device's compiler.

It renders two things:

* a linear UOp listing (``uop/linearize.py``'s ``LinearKernel``, or a sequence of linear UOps)
  to a complete kernel, statement by statement (``renderer/uop_hip.py``);
* a kernel *description* (``KernelSpec``): a name, typed buffer and scalar parameters and a body
  of HIP C++ statements over the index variables ``gidx0..2`` (workgroup ids) and ``lidx0..2``
  (work-item ids) -- the prologue and signature tinygrad's C-style renderers wrap around
  rendered UOps (``render_kernel``), for hand-written bodies.

The packed matmul kernels themselves are prebuilt in libtgm_mi355x.so.
"""

from __future__ import annotations

import threading
from dataclasses import dataclass, field

from tinygrad_mi355x.renderer.uop_hip import VALUE_TYPES as UOP_VALUE_TYPES
from tinygrad_mi355x.renderer.uop_hip import render_uops
from tinygrad_mi355x.runtime.support.compiler_hip import MI355XCompiler

# dtype name -> HIP C++ element type
TYPE_MAP = {
    "bool": "bool", "int8": "signed char", "uint8": "unsigned char", "int16": "short", "uint16": "unsigned short",
    "int32": "int", "uint32": "unsigned int", "int64": "long long", "uint64": "unsigned long long",
    "float16": "_Float16", "bfloat16": "__hip_bfloat16", "float32": "float", "float64": "double",
}


def dtype_name(dt) -> str:
    """The name of a dtype given by name or as a torch / tinygrad dtype object (no import of either)."""
    return dt if isinstance(dt, str) else str(dt).rsplit(".", 1)[-1]
SCALAR_TYPES = {"i32": "int", "u32": "unsigned int", "i64": "long long", "u64": "unsigned long long", "f32": "float",
                "f64": "double"}


@dataclass(frozen=True)
class BufferParam:
    name: str
    dtype: object  # a dtype name ("float32") or a dtype object whose str() ends in one
    mutable: bool = False


@dataclass(frozen=True)
class KernelSpec:
    """A kernel to render: buffers, scalar parameters (name, kind) and body statements."""

    name: str
    buffers: tuple[BufferParam, ...]
    scalars: tuple[tuple[str, str], ...] = ()
    body: tuple[str, ...] = ()
    local_size: tuple[int, int, int] = (256, 1, 1)
    includes: tuple[str, ...] = field(default_factory=tuple)


class MI355XRenderer:
    """Renders HIP C++ for gfx950 and compiles it with the device's compiler."""

    device = "MI355X"
    global_max = (2**31 - 1, 65535, 65535)  # HIP grid limits (workgroups per dimension)
    local_max = (1024, 1024, 1024)
    local_total_max = 1024
    shared_max = 160 * 1024  # LDS per workgroup on gfx950
    wave_size = 64

    def __init__(self, arch: str = "gfx950") -> None:
        self.arch = arch
        self._render_lock = threading.RLock()
        self.matrix_failures: dict[str, str] = {}
        self.compiler = MI355XCompiler(arch)

    def supported_dtypes(self) -> set[str]:
        """Names of the arithmetic dtypes rendered kernels may use (packed formats are storage, not
        arithmetic): the C++ types of hand-written bodies, and in UOp listings also FP8 E4M3FN /
        E5M2 (computed in fp32 and rounded to the format after every operation, as bf16 is)."""
        return set(TYPE_MAP) | set(UOP_VALUE_TYPES)

    def render(self, spec) -> str:
        """Complete ``extern "C" __global__`` source for a ``KernelSpec``, a ``LinearKernel`` or a
        sequence of linear UOps."""
        if not isinstance(spec, KernelSpec):
            with self._render_lock:
                if hasattr(spec, "uops") and hasattr(spec, "local_size"):
                    return render_uops(spec.uops, spec.name, spec.local_size)
                return render_uops(list(spec))
        if any(dtype_name(b.dtype) not in TYPE_MAP for b in spec.buffers):
            raise ValueError(f"kernel {spec.name}: unsupported buffer dtype")
        if any(kind not in SCALAR_TYPES for _, kind in spec.scalars):
            raise ValueError(f"kernel {spec.name}: unsupported scalar kind")
        lx, ly, lz = spec.local_size
        if min(spec.local_size) < 1 or lx * ly * lz > self.local_total_max:
            raise ValueError(f"kernel {spec.name}: invalid local size {spec.local_size}")
        with self._render_lock:
            params = [f"{'' if b.mutable else 'const '}{TYPE_MAP[dtype_name(b.dtype)]}* __restrict__ {b.name}"
                      for b in spec.buffers]
            params += [f"{SCALAR_TYPES[kind]} {name}" for name, kind in spec.scalars]
            lines = ["#include <hip/hip_runtime.h>", "#include <hip/hip_bf16.h>", *spec.includes,
                     f'extern "C" __global__ void __launch_bounds__({lx * ly * lz}) {spec.name}({", ".join(params)}) {{',
                     "  const int gidx0 = blockIdx.x, gidx1 = blockIdx.y, gidx2 = blockIdx.z;",
                     "  const int lidx0 = threadIdx.x, lidx1 = threadIdx.y, lidx2 = threadIdx.z;",
                     "  (void)gidx0; (void)gidx1; (void)gidx2; (void)lidx0; (void)lidx1; (void)lidx2;",
                     *(f"  {s}" for s in spec.body), "}"]
            return "\n".join(lines) + "\n"
