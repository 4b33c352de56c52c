"""Kernel-level UOp graphs: the IR a tinygrad device backend receives, without tinygrad.

The reference renders tinygrad's UOps to HLSL (alexandreteles/tinygrad-dx12
src/tinygrad_dx12/renderer/cstyle.py:303-678) and rewrites scheduled matrix reductions to
LinAlg GEMMs (codegen/matmul.py:51-246).  tinygrad is not a dependency of this package, so the
graph it hands a backend is stated here in the vocabulary of tinygrad's published UOp
specification (tinygrad_spec/tinyspec.tex): a UOp is ``(op, dtype, src, arg)``; a scheduled
kernel is a ``SINK`` of ``STORE``s into ``INDEX``ed ``PARAM``s, closed over their ``RANGE``s by
``END``, with ``REDUCE`` removing reduction ranges; a schedule is a ``LINEAR`` of ``CALL``s whose
first source is the kernel and whose other sources bind the kernel's ``PARAM`` slots in order.
Codegen ops (``SPECIAL``, ``DEFINE_REG``, ``DEFINE_LOCAL``, ``LOAD``, ``IF`` / ``ENDIF``,
``BARRIER``) appear only in linear kernel listings.  The builder calls follow tinygrad's
(``UOp.param``, ``UOp.range``, ``index``, ``store``, ``reduce``, ``end``, ``sink``), so a graph is
written here as a tinygrad user would write it.

UOps are hash-consed: building the same (op, dtype, src, arg) twice returns the same object,
so identity is structural equality and a UOp can key a dict.
"""

from __future__ import annotations

import itertools
import math
import threading
import weakref
from dataclasses import dataclass
from enum import Enum, auto
from typing import Any


# ----------------------------------------------------------------------------- dtypes
@dataclass(frozen=True)
class DType:
    """A scalar storage dtype: ``kind`` is "b" (bool), "i" (signed), "u" (unsigned) or "f" (float)."""

    name: str
    itemsize: int
    kind: str

    def __repr__(self) -> str:
        return f"dtypes.{self.name}"


class dtypes:  # noqa: N801 -- tinygrad's spelling
    bool = DType("bool", 1, "b")
    int8 = DType("int8", 1, "i")
    uint8 = DType("uint8", 1, "u")
    int16 = DType("int16", 2, "i")
    uint16 = DType("uint16", 2, "u")
    int32 = DType("int32", 4, "i")
    uint32 = DType("uint32", 4, "u")
    int64 = DType("int64", 8, "i")
    uint64 = DType("uint64", 8, "u")
    float16 = DType("float16", 2, "f")
    bfloat16 = DType("bfloat16", 2, "f")
    float32 = DType("float32", 4, "f")
    float64 = DType("float64", 8, "f")
    fp8e4m3 = DType("float8_e4m3fn", 1, "f")
    fp8e5m2 = DType("float8_e5m2", 1, "f")
    # tinygrad's aliases
    half, float, double, int, uint, char, uchar = float16, float32, float64, int32, uint32, int8, uint8
    index = int32  # range and address arithmetic

    @staticmethod
    def is_float(dt: DType) -> bool:
        return dt.kind == "f"

    @staticmethod
    def is_int(dt: DType) -> bool:
        return dt.kind in "iu"

    @staticmethod
    def is_unsigned(dt: DType) -> bool:
        return dt.kind == "u"

    @staticmethod
    def min(dt: DType):
        if dt.kind == "f":
            return -math.inf
        if dt.kind == "b":
            return False
        return 0 if dt.kind == "u" else -(1 << (8 * dt.itemsize - 1))

    @staticmethod
    def max(dt: DType):
        if dt.kind == "f":
            return math.inf
        if dt.kind == "b":
            return True
        return (1 << (8 * dt.itemsize - (0 if dt.kind == "u" else 1))) - 1


ALL_DTYPES = (dtypes.bool, dtypes.int8, dtypes.uint8, dtypes.int16, dtypes.uint16, dtypes.int32, dtypes.uint32,
              dtypes.int64, dtypes.uint64, dtypes.float16, dtypes.bfloat16, dtypes.float32, dtypes.float64,
              dtypes.fp8e4m3, dtypes.fp8e5m2)
FP8_DTYPES = (dtypes.fp8e4m3, dtypes.fp8e5m2)


# ----------------------------------------------------------------------------- ops
class Ops(Enum):
    # sources
    PARAM = auto(); BUFFER = auto(); CONST = auto(); DEFINE_VAR = auto()  # noqa: E702
    # ordering
    RANGE = auto(); END = auto(); SINK = auto(); CALL = auto(); LINEAR = auto(); PROGRAM = auto()  # noqa: E702
    # memory
    INDEX = auto(); LOAD = auto(); STORE = auto()  # noqa: E702
    # reduce
    REDUCE = auto()
    # unary
    CAST = auto(); BITCAST = auto(); NEG = auto(); RECIPROCAL = auto(); TRUNC = auto()  # noqa: E702
    EXP2 = auto(); LOG2 = auto(); SIN = auto(); SQRT = auto()  # noqa: E702
    # binary
    ADD = auto(); SUB = auto(); MUL = auto(); FDIV = auto(); IDIV = auto(); MOD = auto(); MAX = auto()  # noqa: E702
    CMPLT = auto(); CMPNE = auto(); CMPEQ = auto()  # noqa: E702
    AND = auto(); OR = auto(); XOR = auto(); SHL = auto(); SHR = auto()  # noqa: E702
    # ternary
    WHERE = auto(); MULACC = auto()  # noqa: E702
    # codegen
    SPECIAL = auto(); DEFINE_REG = auto(); DEFINE_LOCAL = auto(); BARRIER = auto(); IF = auto()  # noqa: E702
    ENDIF = auto()


class AxisType(Enum):
    GLOBAL = auto()
    LOCAL = auto()
    LOOP = auto()
    REDUCE = auto()


UNARY = {Ops.NEG, Ops.RECIPROCAL, Ops.TRUNC, Ops.EXP2, Ops.LOG2, Ops.SIN, Ops.SQRT}
BINARY = {Ops.ADD, Ops.SUB, Ops.MUL, Ops.FDIV, Ops.IDIV, Ops.MOD, Ops.MAX, Ops.CMPLT, Ops.CMPNE, Ops.CMPEQ,
          Ops.AND, Ops.OR, Ops.XOR, Ops.SHL, Ops.SHR}
TERNARY = {Ops.WHERE, Ops.MULACC}
ALU = UNARY | BINARY | TERNARY
COMPARISONS = {Ops.CMPLT, Ops.CMPNE, Ops.CMPEQ}
REDUCE_OPS = {Ops.ADD, Ops.MAX, Ops.MUL}


@dataclass(frozen=True)
class ParamArg:
    """A kernel parameter: its slot, element count and device."""

    slot: int
    size: int
    device: str | None = None


@dataclass(frozen=True)
class BufferArg:
    """A schedule buffer: a unique id, element count and device."""

    uid: int
    size: int
    device: str | None = None


@dataclass(frozen=True)
class KernelInfo:
    """Kernel metadata: the name, and any optimisation choices a user made explicitly."""

    name: str = "kernel"
    applied_opts: tuple = ()
    opts_to_apply: tuple | None = None


_buffer_ids = itertools.count()


class _Interned(type):
    """Hash-consing: one object per (op, dtype, src, arg), also when threads build graphs at once."""

    _cache: weakref.WeakValueDictionary = weakref.WeakValueDictionary()
    _lock = threading.Lock()

    def __call__(cls, op: Ops, dtype: DType | None = None, src: tuple = (), arg: Any = None):
        src = tuple(src)
        # floats key by their bits: -0.0 and 0.0 are distinct constants
        key = (op, dtype, tuple(id(s) for s in src), ("f", arg.hex()) if isinstance(arg, float) else arg)
        with cls._lock:
            found = cls._cache.get(key)
            if found is not None:
                return found
            obj = super().__call__(op, dtype, src, arg)
            cls._cache[key] = obj
            return obj


def _as_uop(x, dtype: DType) -> "UOp":
    return x if isinstance(x, UOp) else UOp.const(dtype, x)


class UOp(metaclass=_Interned):
    __slots__ = ("op", "dtype", "src", "arg", "__weakref__")

    def __init__(self, op: Ops, dtype: DType | None, src: tuple, arg: Any) -> None:
        self.op, self.dtype, self.src, self.arg = op, dtype, src, arg

    def __repr__(self) -> str:
        arg = "" if self.arg is None else f", arg={self.arg!r}"
        return f"UOp({self.op.name}, {self.dtype}, src=<{len(self.src)}>{arg})"

    def __reduce__(self):
        raise TypeError("UOps are not pickled")

    # ------------------------------------------------------------------ graph utilities
    def toposort(self) -> list["UOp"]:
        """Every UOp this one depends on, itself last, each after its sources."""
        order: list[UOp] = []
        seen: set[int] = set()
        stack: list[tuple[UOp, bool]] = [(self, False)]
        while stack:
            node, expanded = stack.pop()
            if expanded:
                order.append(node)
                continue
            if id(node) in seen:
                continue
            seen.add(id(node))
            stack.append((node, True))
            stack.extend((s, False) for s in reversed(node.src) if id(s) not in seen)
        return order

    def replace(self, **kwargs) -> "UOp":
        fields = {"op": self.op, "dtype": self.dtype, "src": self.src, "arg": self.arg}
        fields.update(kwargs)
        return UOp(fields["op"], fields["dtype"], fields["src"], fields["arg"])

    def substitute(self, mapping: dict["UOp", "UOp"]) -> "UOp":
        """This graph with every occurrence of a key of ``mapping`` replaced by its value."""
        done: dict[UOp, UOp] = {}
        for node in self.toposort():
            if node in mapping:
                done[node] = mapping[node]
            else:
                src = tuple(done[s] for s in node.src)
                done[node] = node if all(a is b for a, b in zip(src, node.src)) else node.replace(src=src)
        return done[self]

    @property
    def val(self):
        if self.op is not Ops.CONST:
            raise ValueError("only a CONST has a value")
        return self.arg

    def max_numel(self) -> int:
        if self.op in (Ops.PARAM, Ops.BUFFER, Ops.DEFINE_LOCAL, Ops.DEFINE_REG):
            return self.arg.size if isinstance(self.arg, (ParamArg, BufferArg)) else int(self.arg)
        raise ValueError(f"{self.op.name} has no storage size")

    # ------------------------------------------------------------------ builders
    @staticmethod
    def const(dtype: DType, value) -> "UOp":
        if dtype.kind == "f":
            value = float(value)
        elif dtype.kind == "b":
            value = bool(value)
        else:
            value = int(value)
        return UOp(Ops.CONST, dtype, (), value)

    def const_like(self, value) -> "UOp":
        return UOp.const(self.dtype, value)

    @staticmethod
    def param(slot: int, dtype: DType, size, device: str | None = None) -> "UOp":
        size = math.prod(size) if isinstance(size, tuple) else int(size)
        return UOp(Ops.PARAM, dtype, (), ParamArg(int(slot), size, device))

    @staticmethod
    def new_buffer(device: str | None, size: int, dtype: DType) -> "UOp":
        return UOp(Ops.BUFFER, dtype, (), BufferArg(next(_buffer_ids), int(size), device))

    @staticmethod
    def variable(name: str, lo: int, hi: int, dtype: DType = dtypes.int32) -> "UOp":
        return UOp(Ops.DEFINE_VAR, dtype, (), (name, int(lo), int(hi)))

    @staticmethod
    def range(bound, axis_id: int, axis_type: AxisType = AxisType.LOOP) -> "UOp":
        return UOp(Ops.RANGE, dtypes.index, (_as_uop(bound, dtypes.index),), (int(axis_id), axis_type))

    def index(self, idx, gate: "UOp | None" = None) -> "UOp":
        src = (self, _as_uop(idx, dtypes.index)) + (() if gate is None else (gate,))
        return UOp(Ops.INDEX, self.dtype, src)

    def store(self, value) -> "UOp":
        if self.op is not Ops.INDEX:
            raise ValueError("store goes through an INDEX")
        return UOp(Ops.STORE, None, (self, _as_uop(value, self.dtype)))

    def load(self, alt=None) -> "UOp":
        src = (self,) if alt is None else (self, _as_uop(alt, self.dtype))
        return UOp(Ops.LOAD, self.dtype, src)

    def cast(self, dtype: DType) -> "UOp":
        return self if dtype == self.dtype else UOp(Ops.CAST, dtype, (self,))

    def bitcast(self, dtype: DType) -> "UOp":
        return UOp(Ops.BITCAST, dtype, (self,))

    def reduce(self, *ranges: "UOp", arg: Ops = Ops.ADD) -> "UOp":
        if arg not in REDUCE_OPS:
            raise ValueError(f"no reduction {arg}")
        return UOp(Ops.REDUCE, self.dtype, (self, *ranges), arg)

    def end(self, *ranges: "UOp") -> "UOp":
        return UOp(Ops.END, None, (self, *ranges))

    def sink(self, *more: "UOp", arg: Any = None) -> "UOp":
        return UOp(Ops.SINK, None, (self, *more), arg)

    @staticmethod
    def call(body: "UOp", *args: "UOp") -> "UOp":
        return UOp(Ops.CALL, None, (body, *args))

    @staticmethod
    def linear(*calls: "UOp") -> "UOp":
        return UOp(Ops.LINEAR, None, tuple(calls))

    def alu(self, op: Ops, *others) -> "UOp":
        if op is Ops.WHERE:  # (cond, a, b): the value dtype is that of a (or b)
            a, b = others
            dt = a.dtype if isinstance(a, UOp) else b.dtype
            a, b = _as_uop(a, dt), _as_uop(b, dt)
            if self.dtype != dtypes.bool or a.dtype != b.dtype:
                raise ValueError("WHERE needs a bool condition and equal value dtypes")
            return UOp(op, dt, (self, a, b))
        srcs = (self, *(_as_uop(o, self.dtype) for o in others))
        if any(s.dtype != self.dtype for s in srcs):
            raise ValueError(f"{op.name} needs equal source dtypes, got {[s.dtype for s in srcs]}")
        return UOp(op, dtypes.bool if op in COMPARISONS else self.dtype, srcs)

    def __add__(self, x): return self.alu(Ops.ADD, x)  # noqa: E704
    def __radd__(self, x): return _as_uop(x, self.dtype).alu(Ops.ADD, self)  # noqa: E704
    def __sub__(self, x): return self.alu(Ops.SUB, x)  # noqa: E704
    def __rsub__(self, x): return _as_uop(x, self.dtype).alu(Ops.SUB, self)  # noqa: E704
    def __mul__(self, x): return self.alu(Ops.MUL, x)  # noqa: E704
    def __rmul__(self, x): return _as_uop(x, self.dtype).alu(Ops.MUL, self)  # noqa: E704
    def __truediv__(self, x): return self.alu(Ops.FDIV, x)  # noqa: E704
    def __floordiv__(self, x): return self.alu(Ops.IDIV, x)  # noqa: E704
    def __mod__(self, x): return self.alu(Ops.MOD, x)  # noqa: E704
    def __lt__(self, x): return self.alu(Ops.CMPLT, x)  # noqa: E704
    def __gt__(self, x): return _as_uop(x, self.dtype).alu(Ops.CMPLT, self)  # noqa: E704
    def __and__(self, x): return self.alu(Ops.AND, x)  # noqa: E704
    def __or__(self, x): return self.alu(Ops.OR, x)  # noqa: E704
    def __xor__(self, x): return self.alu(Ops.XOR, x)  # noqa: E704
    def __lshift__(self, x): return self.alu(Ops.SHL, x)  # noqa: E704
    def __rshift__(self, x): return self.alu(Ops.SHR, x)  # noqa: E704
    def __neg__(self): return UOp(Ops.NEG, self.dtype, (self,))  # noqa: E704
    __hash__ = object.__hash__

    def __eq__(self, other) -> bool:  # identity (hash-consed); comparisons build with ne / eq
        return self is other

    def ne(self, x) -> "UOp":
        return self.alu(Ops.CMPNE, x)

    def eq(self, x) -> "UOp":
        return self.alu(Ops.CMPEQ, x)

    def maximum(self, x) -> "UOp":
        return self.alu(Ops.MAX, x)

    def where(self, a, b) -> "UOp":
        return self.alu(Ops.WHERE, a, b)

    def exp2(self) -> "UOp": return UOp(Ops.EXP2, self.dtype, (self,))  # noqa: E704
    def log2(self) -> "UOp": return UOp(Ops.LOG2, self.dtype, (self,))  # noqa: E704
    def sqrt(self) -> "UOp": return UOp(Ops.SQRT, self.dtype, (self,))  # noqa: E704
    def sin(self) -> "UOp": return UOp(Ops.SIN, self.dtype, (self,))  # noqa: E704
    def reciprocal(self) -> "UOp": return UOp(Ops.RECIPROCAL, self.dtype, (self,))  # noqa: E704
    def trunc(self) -> "UOp": return UOp(Ops.TRUNC, self.dtype, (self,))  # noqa: E704

    def mulacc(self, b, c) -> "UOp":
        return self.alu(Ops.MULACC, b, c)
