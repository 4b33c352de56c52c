"""Linear UOp listing -> HIP C++ kernel for gfx950.

Counterpart of the reference's UOp renderer (alexandreteles/tinygrad-dx12
src/tinygrad_dx12/renderer/cstyle.py:303-678, which extends tinygrad's C-style renderer with HLSL
rules).  It renders a kernel listing -- the linear UOps of ``uop/linearize.py``, or any listing
that uses the same op and dtype names (it reads ``op.name`` and the dtype's name, so tinygrad's
own UOps render when their ops are among these) -- one statement per value:

* buffers (``PARAM`` in slot order, or ``DEFINE_GLOBAL``) become ``T* __restrict__`` kernel
  parameters (``const`` when nothing stores through them), ``DEFINE_VAR`` an ``int`` parameter;
  ``SPECIAL`` ``gidxN`` / ``lidxN`` / ``idxN`` are workgroup, work-item and global ids;
* ``RANGE`` / ``END`` are a ``for`` loop, ``IF`` / ``ENDIF`` an ``if`` block, ``BARRIER`` is
  ``__syncthreads()``, ``DEFINE_REG`` / ``DEFINE_LOCAL`` a register / LDS (``__shared__``) array;
* ``INDEX`` is an address (with an optional gate), ``LOAD`` reads through it (a false gate gives
  the alternative value, 0 by default), ``STORE`` writes through it (skipped under a false gate).

Arithmetic keeps each dtype's semantics, as the reference's dtype table requires
(ARCHITECTURE.md:224-268): integer results wrap to their width (add, sub, mul, shift-left and
negate of signed or narrow types are computed in an unsigned type at least as wide and truncated,
so overflow is defined); bf16 values are computed in fp32 and rounded to bf16 after every
operation; f16 uses gfx950's native f16 arithmetic; bool storage is a byte (loads test != 0, stores write 0 / 1);
FP8 (E4M3FN, E5M2) values live in fp32 registers: loads decode exactly, arithmetic and casts
compute in fp32 and round to the format after every operation, stores encode (round to nearest
even; E4M3FN turns NaN, infinities and overflow into NaN, E5M2 overflow into infinity, as
torch's conversions do).  Floating multiply and add are not contracted into FMA (``MULACC`` is the fused
operation); division and square root are correctly rounded; EXP2 / LOG2 / SIN use the device
math library.
"""

from __future__ import annotations

import math

NAME_ALIASES = {  # tinygrad dtype names -> the names used here
    "half": "float16", "float": "float32", "double": "float64", "char": "int8", "uchar": "uint8",
    "short": "int16", "ushort": "uint16", "int": "int32", "uint": "uint32", "long": "int64", "ulong": "uint64",
    "fp8e4m3": "float8_e4m3fn", "fp8e5m2": "float8_e5m2", "index": "int32",
}
VALUE_TYPES = {
    "bool": "bool", "int8": "signed char", "uint8": "unsigned char", "int16": "short", "uint16": "unsigned short",
    "int32": "int", "uint32": "unsigned int", "int64": "long long", "uint64": "unsigned long long",
    "float16": "_Float16", "bfloat16": "__bf16", "float32": "float", "float64": "double",
    "float8_e4m3fn": "float", "float8_e5m2": "float",
}
STORAGE_TYPES = {**VALUE_TYPES, "bool": "unsigned char", "float8_e4m3fn": "unsigned char",
                 "float8_e5m2": "unsigned char"}
# the type wrapping integer arithmetic is computed in: narrow types would otherwise promote to
# (signed) int, whose overflow is undefined
WRAP_TYPES = {"int8": "unsigned int", "uint8": "unsigned int", "int16": "unsigned int", "uint16": "unsigned int",
              "int32": "unsigned int", "int64": "unsigned long long"}
FP8 = ("float8_e4m3fn", "float8_e5m2")
INTS = ("int8", "uint8", "int16", "uint16", "int32", "uint32", "int64", "uint64")
FLOATS = ("float16", "bfloat16", "float32", "float64")

PRELUDE = r"""#include <hip/hip_runtime.h>
#pragma clang fp contract(off)
// exact FP8 decodes (OCP E4M3FN: bias 7, no infinities, S.1111.111 is NaN; E5M2: bias 15, IEEE-like)
__device__ __forceinline__ float tgm_e4m3_f32(unsigned char b) {
  const int e = (b >> 3) & 15, m = b & 7;
  float v = e == 0 ? ldexpf((float)m, -9) : ldexpf((float)(8 + m), e - 10);
  if (e == 15 && m == 7) v = __builtin_nanf("");
  return (b & 0x80) ? -v : v;
}
__device__ __forceinline__ float tgm_e5m2_f32(unsigned char b) {
  const int e = (b >> 2) & 31, m = b & 3;
  float v = e == 0 ? ldexpf((float)m, -16) : ldexpf((float)(4 + m), e - 17);
  if (e == 31) v = m == 0 ? __builtin_inff() : __builtin_nanf("");
  return (b & 0x80) ? -v : v;
}
// fp32 -> FP8, round to nearest even.  E4M3FN: NaN, infinities and magnitudes past 464 (which
// round beyond 448) give S.1111.111; E5M2: NaN gives S.11111.11, infinities and magnitudes of
// 61440 and more give S.11111.00.  Normal results round the fp32 significand to 3 (2) bits by
// integer addition; subnormal ones are rint(|x| * 2^9) (2^16) codes of the smallest step.
__device__ __forceinline__ unsigned char tgm_f32_e4m3(float f) {
  const unsigned u = __builtin_bit_cast(unsigned, f) & 0x7FFFFFFFu, s = (__builtin_bit_cast(unsigned, f) >> 24) & 0x80u;
  if (u > 0x43E80000u) return (unsigned char)(s | 0x7Fu);  // NaN, inf, |f| > 464
  if (u >= 0x3C800000u) {                                  // |f| >= 2^-6: normal
    const unsigned r = u + 0x7FFFFu + ((u >> 20) & 1u);
    return (unsigned char)(s | (((r >> 23) - 120u) << 3) | ((r >> 20) & 7u));
  }
  return (unsigned char)(s | (unsigned)__builtin_rintf(__builtin_bit_cast(float, u) * 512.0f));
}
__device__ __forceinline__ unsigned char tgm_f32_e5m2(float f) {
  const unsigned u = __builtin_bit_cast(unsigned, f) & 0x7FFFFFFFu, s = (__builtin_bit_cast(unsigned, f) >> 24) & 0x80u;
  if (u > 0x7F800000u) return (unsigned char)(s | 0x7Fu);  // NaN
  if (u >= 0x47700000u) return (unsigned char)(s | 0x7Cu);  // inf, |f| >= 61440
  if (u >= 0x38800000u) {                                  // |f| >= 2^-14: normal
    const unsigned r = u + 0xFFFFFu + ((u >> 21) & 1u);
    return (unsigned char)(s | (((r >> 23) - 112u) << 2) | ((r >> 21) & 3u));
  }
  return (unsigned char)(s | (unsigned)__builtin_rintf(__builtin_bit_cast(float, u) * 65536.0f));
}
"""


def dtype_name(dt) -> str:
    """Canonical name of a dtype given by name or as an object with ``.name`` (or a pointer dtype
    with ``.base``)."""
    if dt is None:
        return "void"
    dt = getattr(dt, "base", dt)
    name = dt if isinstance(dt, str) else getattr(dt, "name", str(dt).rsplit(".", 1)[-1])
    return NAME_ALIASES.get(name, name)


def _float_literal(v: float, dt: str) -> str:
    if math.isnan(v):
        core = "__builtin_nanf(\"\")" if dt != "float64" else "__builtin_nan(\"\")"
    elif math.isinf(v):
        core = ("(-" if v < 0 else "(") + ("__builtin_inff()" if dt != "float64" else "__builtin_inf()") + ")"
    else:
        core = v.hex() + ("" if dt == "float64" else "f")
    return core if dt in ("float32", "float64") else f"(({VALUE_TYPES[dt]})({core}))"


def _int_literal(v: int, dt: str) -> str:
    v = int(v)
    if dt in ("int64", "uint64", "uint32"):
        suffix = {"int64": "ll", "uint64": "ull", "uint32": "u"}[dt]
        if dt == "int64" and v == -(1 << 63):
            return "(-9223372036854775807ll - 1)"
        return f"{v}{suffix}" if v >= 0 or dt == "int64" else f"(({VALUE_TYPES[dt]}){v}ll)"
    if dt == "int32":
        return "(-2147483647 - 1)" if v == -(1 << 31) else str(v)
    return f"(({VALUE_TYPES[dt]}){v})"


def fp8_round(expr: str, dt: str) -> str:
    """``expr`` (an fp32 expression) rounded to FP8 format ``dt``, as the fp32 value of the code."""
    f = "e4m3" if dt == "float8_e4m3fn" else "e5m2"
    return f"tgm_{f}_f32(tgm_f32_{f}({expr}))"


def literal(value, dt: str) -> str:
    if dt in FP8:
        return fp8_round(_float_literal(float(value), "float32"), dt)
    if dt == "bool":
        return "true" if value else "false"
    if dt in FLOATS:
        return _float_literal(float(value), dt)
    if dt in INTS:
        return _int_literal(value, dt)
    raise ValueError(f"no {dt} constants")


class _Listing:
    def __init__(self, uops, name: str, local_size) -> None:
        self.uops = list(uops)
        self.name = name
        self.local_size = local_size
        self.names: dict[int, str] = {}
        self.ptrs: dict[int, tuple[str, str, str | None]] = {}  # INDEX -> (address, dtype, gate)
        self.lines: list[str] = []
        self.depth = 1
        self.counter = 0

    def fresh(self, prefix: str) -> str:
        self.counter += 1
        return f"{prefix}{self.counter}"

    def emit(self, line: str) -> None:
        self.lines.append("  " * self.depth + line)

    def ref(self, u) -> str:
        op = u.op.name
        if op == "CONST":
            return literal(u.arg, dtype_name(u.dtype))
        try:
            return self.names[id(u)]
        except KeyError:
            raise ValueError(f"{op} is used before it is listed") from None

    # ------------------------------------------------------------------ arithmetic
    def alu(self, op: str, dt: str, srcs) -> str:
        a = [self.ref(s) for s in srcs]
        sdt = dtype_name(srcs[0].dtype)
        if op == "WHERE":
            return f"({a[0]} ? {a[1]} : {a[2]})"
        if op in ("CMPLT", "CMPNE", "CMPEQ"):
            sym = {"CMPLT": "<", "CMPNE": "!=", "CMPEQ": "=="}[op]
            if sdt == "bfloat16":
                return f"((float){a[0]} {sym} (float){a[1]})"
            return f"({a[0]} {sym} {a[1]})"
        if dt == "bool":
            bool_ops = {"AND": "&&", "OR": "||", "XOR": "!=", "ADD": "||", "MUL": "&&", "MAX": "||",
                        "CMPNE": "!="}
            if op in bool_ops:
                return f"({a[0]} {bool_ops[op]} {a[1]})"
            raise ValueError(f"{op} on bool")
        if dt in FP8:  # fp32 arithmetic on the decoded values, one rounding to the format
            return fp8_round(self.float_alu(op, "float32", a), dt)
        if dt in FLOATS:
            return self.float_alu(op, dt, a)
        return self.int_alu(op, dt, a)

    def float_alu(self, op: str, dt: str, a: list[str]) -> str:
        ct = VALUE_TYPES[dt]
        wide = dt == "float64"
        f = "" if wide else "f"
        if dt == "bfloat16":  # fp32 arithmetic, one rounding to bf16
            a = [f"(float){x}" for x in a]
        binary = {"ADD": "+", "SUB": "-", "MUL": "*", "FDIV": "/"}
        if op in binary:
            expr = f"({a[0]} {binary[op]} {a[1]})"
        elif op == "MAX":
            expr = f"fmax{f}({a[0]}, {a[1]})" if dt != "float16" else f"(_Float16)fmaxf({a[0]}, {a[1]})"
        elif op == "NEG":
            expr = f"(-{a[0]})"
        elif op == "RECIPROCAL":
            expr = f"(({'1.0' if wide else '1.0f'}) / {a[0]})" if dt != "float16" else f"((_Float16)1.0f / {a[0]})"
        elif op == "MULACC":
            expr = f"fma{f}({a[0]}, {a[1]}, {a[2]})" if dt != "float16" else f"(_Float16)fmaf({a[0]}, {a[1]}, {a[2]})"
        elif op in ("EXP2", "LOG2", "SIN", "SQRT", "TRUNC"):
            fn = {"EXP2": "exp2", "LOG2": "log2", "SIN": "sin", "SQRT": "sqrt", "TRUNC": "trunc"}[op] + f
            expr = f"{fn}({a[0]})" if dt != "float16" else f"(_Float16){fn}((float){a[0]})"
        else:
            raise ValueError(f"{op} on {dt}")
        return f"(({ct}){expr})" if dt in ("bfloat16", "float16") else expr

    def int_alu(self, op: str, dt: str, a: list[str]) -> str:
        ct = VALUE_TYPES[dt]
        # results that may overflow are computed in an unsigned type at least as wide, then
        # truncated to the dtype
        wrap = WRAP_TYPES.get(dt)
        binary = {"ADD": "+", "SUB": "-", "MUL": "*", "SHL": "<<"}
        if op in binary:
            x, y = (f"({wrap}){a[0]}", f"({wrap}){a[1]}") if wrap else (a[0], a[1])
            if op == "SHL":
                y = a[1]
            return f"(({ct})({x} {binary[op]} {y}))"
        if op == "NEG":
            return f"(({ct})(-({wrap}){a[0]}))" if wrap else f"(({ct})(-{a[0]}))"
        if op == "MULACC":
            x, y, z = (f"({wrap}){v}" for v in a) if wrap else a
            return f"(({ct})({x} * {y} + {z}))"
        simple = {"IDIV": "/", "MOD": "%", "AND": "&", "OR": "|", "XOR": "^", "SHR": ">>"}
        if op in simple:
            return f"(({ct})({a[0]} {simple[op]} {a[1]}))"
        if op == "MAX":
            return f"({a[0]} < {a[1]} ? {a[1]} : {a[0]})"
        raise ValueError(f"{op} on {dt}")

    def cast(self, src, dt: str, bit: bool) -> str:
        x, sdt = self.ref(src), dtype_name(src.dtype)
        if bit:
            if dt in FP8 or sdt in FP8:
                raise ValueError("FP8 values live decoded in fp32 registers: no bit casts")
            return f"__builtin_bit_cast({VALUE_TYPES[dt]}, {x})"
        if dt in FP8:
            return fp8_round(f"(float)({x})", dt)
        if dt == "bool":
            return f"((bool)({x}))"
        if sdt == "bfloat16" and dt != "float32":
            x = f"(float){x}"
        return f"(({VALUE_TYPES[dt]})({x}))"

    # ------------------------------------------------------------------ memory
    def load(self, u) -> str:
        idx = u.src[0]
        addr, dt, gate = self.ptrs[id(idx)]
        if dt == "bool":
            value = f"(*{addr} != 0)"
        elif dt == "float8_e4m3fn":
            value = f"tgm_e4m3_f32(*{addr})"
        elif dt == "float8_e5m2":
            value = f"tgm_e5m2_f32(*{addr})"
        else:
            value = f"(*{addr})"
        if gate is None:
            return value
        alt = self.ref(u.src[1]) if len(u.src) > 1 else literal(0, dt if dt not in FP8 else "float32")
        return f"({gate} ? {value} : {alt})"

    def store(self, u) -> None:
        idx, val = u.src[0], u.src[1]
        addr, dt, gate = self.ptrs[id(idx)]
        v = self.ref(val)
        if dt in FP8:
            v = f"tgm_f32_{'e4m3' if dt == 'float8_e4m3fn' else 'e5m2'}({v})"
        if dt == "bool":
            v = f"(unsigned char)({v} ? 1 : 0)"
        if len(u.src) > 2:  # a separate store gate
            g = self.ref(u.src[2])
            gate = g if gate is None else f"({gate} && {g})"
        line = f"*{addr} = {v};"
        self.emit(line if gate is None else f"if ({gate}) {line}")

    # ------------------------------------------------------------------ listing
    def render(self) -> str:
        params, scalars, stored = [], [], set()
        for u in self.uops:
            if u.op.name == "STORE":
                base = u.src[0].src[0] if u.src[0].op.name == "INDEX" else u.src[0]
                stored.add(id(base))
        buffers = [u for u in self.uops if u.op.name in ("PARAM", "DEFINE_GLOBAL")]

        def slot(u) -> int:
            return getattr(u.arg, "slot", u.arg if isinstance(u.arg, int) else 0)

        for i, u in enumerate(sorted(buffers, key=slot)):
            dt = dtype_name(u.dtype)
            if dt not in STORAGE_TYPES:
                raise ValueError(f"buffer dtype {dt} is not rendered")
            name = f"data{slot(u)}"
            self.names[id(u)] = name
            const = "" if id(u) in stored else "const "
            params.append(f"{const}{STORAGE_TYPES[dt]}* __restrict__ {name}")
        for u in sorted((u for u in self.uops if u.op.name == "DEFINE_VAR"), key=lambda u: u.arg[0]):
            if dtype_name(u.dtype) != "int32":
                raise ValueError("variables are int32")
            self.names[id(u)] = str(u.arg[0])
            scalars.append(f"int {u.arg[0]}")
        body = self.lines
        for u in self.uops:
            op = u.op.name
            dt = dtype_name(u.dtype)
            if op in ("PARAM", "DEFINE_GLOBAL", "DEFINE_VAR", "CONST", "NOOP"):
                continue
            if op == "SPECIAL":
                n = str(u.arg)
                axis = "xyz"[int(n[-1])]
                expr = {"g": f"(int)blockIdx.{axis}", "l": f"(int)threadIdx.{axis}",
                        "i": f"(int)(blockIdx.{axis} * blockDim.{axis} + threadIdx.{axis})"}[n[0]]
                self.names[id(u)] = n
                self.emit(f"const int {n} = {expr};")
            elif op == "RANGE":
                v = self.fresh("ridx")
                self.names[id(u)] = v
                self.emit(f"for (int {v} = 0; {v} < {self.ref(u.src[0])}; ++{v}) {{")
                self.depth += 1
            elif op in ("END", "ENDRANGE", "ENDIF"):
                self.depth -= 1
                self.emit("}")
            elif op == "IF":
                self.emit(f"if ({self.ref(u.src[0])}) {{")
                self.depth += 1
            elif op == "BARRIER":
                self.emit("__syncthreads();")
            elif op in ("DEFINE_REG", "DEFINE_LOCAL", "DEFINE_ACC"):
                size = u.arg[0] if isinstance(u.arg, tuple) else int(u.arg)
                v = self.fresh("acc" if op != "DEFINE_LOCAL" else "lds")
                self.names[id(u)] = v
                shared = "__shared__ " if op == "DEFINE_LOCAL" else ""
                self.emit(f"{shared}{STORAGE_TYPES[dt]} {v}[{size}];")
            elif op == "INDEX":
                base = self.ref(u.src[0])
                gate = self.ref(u.src[2]) if len(u.src) > 2 else None
                bdt = dtype_name(u.src[0].dtype)
                self.ptrs[id(u)] = (f"({base} + {self.ref(u.src[1])})", bdt, gate)
            elif op == "LOAD":
                v = self.fresh("val")
                self.names[id(u)] = v
                self.emit(f"{VALUE_TYPES[dt]} {v} = {self.load(u)};")
            elif op == "STORE":
                self.store(u)
            elif op in ("CAST", "BITCAST"):
                v = self.fresh("cast")
                self.names[id(u)] = v
                self.emit(f"{VALUE_TYPES[dt]} {v} = {self.cast(u.src[0], dt, op == 'BITCAST')};")
            else:
                v = self.fresh("alu")
                self.names[id(u)] = v
                if dt not in VALUE_TYPES:
                    raise ValueError(f"{op} of dtype {dt} is not rendered")
                self.emit(f"{VALUE_TYPES[dt]} {v} = {self.alu(op, dt, u.src)};")
        if self.depth != 1:
            raise ValueError("unbalanced RANGE / IF blocks in the listing")
        threads = math.prod(self.local_size)
        head = (f'extern "C" __global__ void __launch_bounds__({threads}) '
                f'{self.name}({", ".join(params + scalars)}) {{')
        return PRELUDE + head + "\n" + "\n".join(body) + "\n}\n"


def render_uops(uops, name: str = "kernel", local_size: tuple[int, int, int] | None = None) -> str:
    """HIP C++ source of one kernel listing.  ``local_size`` defaults to the product of the
    listing's ``lidx`` SPECIAL bounds (its work-items per workgroup)."""
    if not name.isidentifier():
        raise ValueError(f"kernel name {name!r} is not an identifier")
    if local_size is None:
        dims = [1, 1, 1]
        for u in uops:
            if u.op.name == "SPECIAL" and str(u.arg).startswith("l") and u.src and u.src[0].op.name == "CONST":
                dims[int(str(u.arg)[-1])] = int(u.src[0].arg)
        local_size = tuple(dims)
    if math.prod(local_size) > 1024:
        raise ValueError(f"kernel {name}: more than 1024 work-items per workgroup")
    return _Listing(uops, name, local_size).render()
