"""HIP C++ -> gfx950 code object compiler for the MI355X device plugin.

Mirrors ``DX12Compiler`` of alexandreteles/tinygrad-dx12
(src/tinygrad_dx12/runtime/support/compiler_dx12.py:49-123): construction needs no GPU
and no toolchain, the cache key is a deterministic name derived from the compiler
identity and settings, compilation is serialised by a lock, and failures raise
``CompileError`` carrying the compiler's diagnostics.  The DXC-in-process call becomes
one ``amdclang++ -x hip --cuda-device-only`` invocation producing an AMDGPU code object
(ELF), which ``hipModuleLoadData`` loads.

The compiled object keeps its source and kernel signature in front of the code object
(as the reference keeps HLSL beside DXIL, compiler_dx12.py:122-123), so a Program can
validate buffer and scalar counts without parsing machine code.

With ``MI355X_DUMP_SRC=1`` every source the compiler compiles (each new source, once) is
printed to stderr first, as the reference's ``DX12_DUMP_SHADERS=1`` prints its HLSL
(compiler_dx12.py:81-82).
"""

from __future__ import annotations

import hashlib
import json
import os
import re
import subprocess
import sys
import tempfile
import threading
from dataclasses import dataclass
from pathlib import Path

MAGIC = b"TGMHSACO1\n"
# hipcc feature flag required for all HIP code on this pool (no packed-fp32 instructions).
SAFE_FLAGS = ("-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops")


class CompileError(RuntimeError):
    """Compilation failed; the message holds the compiler diagnostics."""


def _clang() -> str:
    root = os.environ.get("ROCM_PATH", "/opt/rocm")
    for candidate in (f"{root}/bin/amdclang++", f"{root}/lib/llvm/bin/clang++"):
        if os.path.exists(candidate):
            return candidate
    return "amdclang++"


@dataclass(frozen=True)
class KernelSignature:
    """Parameter kinds of one ``extern "C" __global__`` kernel, in order.

    Each kind is ``"ptr"`` (a device buffer) or a scalar type (``"i32"``, ``"u32"``,
    ``"i64"``, ``"u64"``, ``"f32"``, ``"f64"``).
    """

    name: str
    params: tuple[str, ...]

    @property
    def buffers(self) -> int:
        return sum(p == "ptr" for p in self.params)

    @property
    def scalars(self) -> int:
        return sum(p != "ptr" for p in self.params)


_SCALARS = {
    "int": "i32", "int32_t": "i32", "signed": "i32", "unsigned": "u32", "unsigned int": "u32", "uint32_t": "u32",
    "long": "i64", "long long": "i64", "int64_t": "i64", "unsigned long": "u64", "unsigned long long": "u64",
    "uint64_t": "u64", "size_t": "u64", "float": "f32", "double": "f64",
}


def parse_signature(source: str, name: str | None = None) -> KernelSignature:
    """Find the ``extern "C" __global__`` kernel (``name`` or the only one) and its parameter kinds."""
    pattern = re.compile(r'extern\s+"C"\s+__global__\s+(?:__launch_bounds__\([^)]*\)\s+)?void\s+'
                         r'(?:__launch_bounds__\([^)]*\)\s+)?(\w+)\s*\(([^)]*)\)', re.S)
    found = [(m.group(1), m.group(2)) for m in pattern.finditer(source)]
    if name is not None:
        found = [f for f in found if f[0] == name]
    if len(found) != 1:
        raise CompileError(f"expected exactly one extern \"C\" __global__ kernel{'' if name is None else ' ' + name}, "
                           f"found {len(found)}")
    kname, params = found[0]
    kinds = []
    for p in (x.strip() for x in params.split(",") if x.strip()):
        if "*" in p:
            kinds.append("ptr")
            continue
        words = [w for w in re.sub(r"\b(const|volatile|__restrict__|restrict)\b", " ", p).split()]
        ctype = " ".join(words[:-1])
        if ctype not in _SCALARS:
            raise CompileError(f"kernel {kname}: unsupported parameter {p!r}")
        kinds.append(_SCALARS[ctype])
    return KernelSignature(kname, tuple(kinds))


def pack_object(source: str, signature: KernelSignature, code: bytes) -> bytes:
    header = json.dumps({"name": signature.name, "params": list(signature.params), "source": source}).encode()
    return MAGIC + len(header).to_bytes(8, "little") + header + code


def unpack_object(obj: bytes) -> tuple[str, KernelSignature, bytes]:
    if not obj.startswith(MAGIC):
        raise ValueError("not an MI355X compiled object")
    off = len(MAGIC)
    n = int.from_bytes(obj[off:off + 8], "little")
    header = json.loads(obj[off + 8:off + 8 + n])
    return header["source"], KernelSignature(header["name"], tuple(header["params"])), obj[off + 8 + n:]


class MI355XCompiler:
    """Compile HIP C++ source to a gfx950 code object, cached by a deterministic key."""

    def __init__(self, arch: str = "gfx950", opt: str = "-O3", extra: tuple[str, ...] = ()) -> None:
        self.arch = arch
        self.settings = ("-x", "hip", f"--offload-arch={arch}", "--cuda-device-only", "--no-gpu-bundle-output", opt,
                         "-std=c++17", *SAFE_FLAGS, *extra)
        identity = repr((_clang(), self.settings, MAGIC))
        self.cachekey = "mi355x_" + hashlib.sha256(identity.encode()).hexdigest()
        self.lock = threading.Lock()
        self.diagnostics = ""
        self._cache: dict[str, bytes] = {}

    def compile(self, src: str) -> bytes:
        """Compile one kernel source; returns the packed object (source, signature, code object)."""
        signature = parse_signature(src)
        key = hashlib.sha256(src.encode()).hexdigest()
        with self.lock:
            if key in self._cache:
                return self._cache[key]
            if os.environ.get("MI355X_DUMP_SRC", "0") == "1":  # the reference's DX12_DUMP_SHADERS
                print(src, file=sys.stderr)
            with tempfile.TemporaryDirectory(prefix="mi355x_cc_") as tmp:
                path = Path(tmp) / "kernel.hip"
                out = Path(tmp) / "kernel.hsaco"
                path.write_text(src)
                proc = subprocess.run([_clang(), *self.settings, "-c", str(path), "-o", str(out)],
                                      capture_output=True, text=True)
                self.diagnostics = "\n".join(line for line in proc.stderr.splitlines()
                                             if "packed-fp32-ops" not in line)
                if proc.returncode != 0 or not out.exists():
                    raise CompileError(f"amdclang++ {self.arch} failed ({proc.returncode}):\n{self.diagnostics}")
                code = out.read_bytes()
            obj = pack_object(src, signature, code)
            self._cache[key] = obj
            return obj

    def compile_cached(self, src: str) -> bytes:
        return self.compile(src)
