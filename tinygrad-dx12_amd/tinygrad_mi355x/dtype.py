"""Dtype promotion used by the packed path, over ``torch.dtype``.

The reference delegates promotion to tinygrad (``least_upper_dtype``,
``strong_dtype``, ``sum_acc_dtype``; alexandreteles/tinygrad-dx12
src/tinygrad_dx12/codegen/decomp/dx12.py:6, renderer/linalg.py:33-35).  tinygrad is
not a dependency here, so the same lattice is expressed over torch dtypes:

* every dtype promotes along a fixed parent graph, and the least upper bound of a
  set is the lowest-priority dtype reachable from all of them;
* ``sum_acc_dtype`` widens unsigned types to at least uint32, signed types and bool
  to at least int32, and floats to at least float32 (ARCHITECTURE.md:294-299).

``float8_e8m0fnu`` (OCP MX scale) is an extension: it promotes straight to
float32, so ``least_upper_dtype(float32, e8m0) == float32`` and E8M0 scale tensors
behave as the numeric scales the reference requires (dx12.py:20-23).
"""

from __future__ import annotations

import functools

import torch

# Priority order (lowest first) used to break ties between common parents.
_ORDER = [
    torch.bool, torch.int8, torch.uint8, torch.int16, torch.uint16, torch.int32, torch.uint32,
    torch.int64, torch.uint64, torch.float8_e4m3fn, torch.float8_e5m2, torch.float8_e8m0fnu,
    torch.float16, torch.bfloat16, torch.float32, torch.float64,
]
_PRIORITY = {dt: i for i, dt in enumerate(_ORDER)}

_PARENTS: dict[torch.dtype, tuple[torch.dtype, ...]] = {
    torch.bool: (torch.int8, torch.uint8),
    torch.int8: (torch.int16,),
    torch.int16: (torch.int32,),
    torch.int32: (torch.int64,),
    torch.int64: (torch.float8_e4m3fn, torch.float8_e5m2),
    torch.uint8: (torch.int16, torch.uint16),
    torch.uint16: (torch.int32, torch.uint32),
    torch.uint32: (torch.int64, torch.uint64),
    torch.uint64: (torch.float8_e4m3fn, torch.float8_e5m2),
    torch.float8_e4m3fn: (torch.float16, torch.bfloat16),
    torch.float8_e5m2: (torch.float16, torch.bfloat16),
    torch.float8_e8m0fnu: (torch.float32,),
    torch.float16: (torch.float32,),
    torch.bfloat16: (torch.float32,),
    torch.float32: (torch.float64,),
    torch.float64: (),
}

FLOATS = {torch.float8_e4m3fn, torch.float8_e5m2, torch.float8_e8m0fnu, torch.float16, torch.bfloat16,
          torch.float32, torch.float64}
UNSIGNED = {torch.uint8, torch.uint16, torch.uint32, torch.uint64}
SIGNED = {torch.int8, torch.int16, torch.int32, torch.int64}
FP8 = (torch.float8_e4m3fn, torch.float8_e5m2)


@functools.cache
def _ancestors(dt: torch.dtype) -> frozenset:
    out = {dt}
    for parent in _PARENTS[dt]:
        out |= _ancestors(parent)
    return frozenset(out)


def least_upper_dtype(*dts: torch.dtype) -> torch.dtype:
    """Lowest dtype that every argument promotes to."""
    for dt in dts:
        if dt not in _PARENTS:
            raise ValueError(f"dtype {dt} has no promotion rule on this backend")
    common = frozenset.intersection(*(_ancestors(dt) for dt in dts))
    return min(common, key=_PRIORITY.__getitem__)


def strong_dtype(dt: torch.dtype) -> torch.dtype:
    """torch tensors carry no weak (literal-derived) dtypes, so this is the identity."""
    return dt


def sum_acc_dtype(dt: torch.dtype) -> torch.dtype:
    """Default reduction dtype: uint32+, int32+ (and bool), float32+."""
    if dt in UNSIGNED:
        return least_upper_dtype(dt, torch.uint32)
    if dt in SIGNED or dt is torch.bool:
        return least_upper_dtype(dt, torch.int32)
    return least_upper_dtype(dt, torch.float32)


def is_float(dt: torch.dtype) -> bool:
    return dt in FLOATS


def itemsize(dt: torch.dtype) -> int:
    return torch.empty((), dtype=dt).element_size()
