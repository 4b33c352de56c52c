"""ctypes binding of the HIP runtime C API used by the MI355X device plugin.

This replaces the reference's D3D12/DXGI native layer (alexandreteles/tinygrad-dx12
src/tinygrad_dx12/runtime/support/dx12.py, runtime/autogen/*): instead of COM vtables,
plain ``hipError_t`` functions.  Every failure becomes ``RuntimeError("<op> failed:
<code> (<hipGetErrorString>)")``, the shape of the reference's ``check``
(runtime/support/dx12.py:11-15).

One process must hold one HIP runtime, so that device memory, streams and modules are shared
by torch, this binding and the kernel library.  ``runtime_path`` picks it: an explicit
``MI355X_HIP_RUNTIME``; else the instance already loaded (opened by its soname,
libamdhip64.so.7); else, when torch is installed, the copy torch ships and will load -- torch's
libraries ask for ``libamdhip64.so`` through their own rpath, a name the ROCm runtime's soname
does not match, so a ROCm runtime opened first would become a second runtime once torch is
imported; a torch runtime opened first by path is the very file torch later maps, and the
dynamic loader reuses it.  Nothing here imports torch or touches the GPU at import time.
"""

from __future__ import annotations

import ctypes
import os
import threading

# hipMemcpyKind
H2D, D2H, D2D = 1, 2, 3
# hipModuleLaunchKernel "extra" markers (HIP_LAUNCH_PARAM_*)
_PARAM_BUFFER_POINTER, _PARAM_BUFFER_SIZE, _PARAM_END = 1, 2, 3
# hipError_t values the runtime reports for "not finished yet"
HIP_ERROR_NOT_READY = 600
# hipDeviceAttribute_t
ATTR_CLOCK_RATE_KHZ = 5  # hipDeviceAttributeClockRate
ATTR_CU_COUNT = 63  # hipDeviceAttributeMultiprocessorCount

_P, _INT, _SZ, _U32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t, ctypes.c_uint

_SIGNATURES = {
    "hipInit": (_U32,),
    "hipGetDeviceCount": (ctypes.POINTER(_INT),),
    "hipSetDevice": (_INT,),
    "hipGetDevice": (ctypes.POINTER(_INT),),
    "hipDeviceGetAttribute": (ctypes.POINTER(_INT), _INT, _INT),
    "hipDeviceGetName": (ctypes.c_char_p, _INT, _INT),
    "hipDeviceSynchronize": (),
    "hipMalloc": (ctypes.POINTER(_P), _SZ),
    "hipFree": (_P,),
    "hipHostMalloc": (ctypes.POINTER(_P), _SZ, _U32),
    "hipHostFree": (_P,),
    "hipMemcpyAsync": (_P, _P, _SZ, _INT, _P),
    "hipMemcpyPeerAsync": (_P, _INT, _P, _INT, _SZ, _P),
    "hipMemsetAsync": (_P, _INT, _SZ, _P),
    "hipStreamCreate": (ctypes.POINTER(_P),),
    "hipStreamDestroy": (_P,),
    "hipStreamSynchronize": (_P,),
    "hipStreamQuery": (_P,),
    "hipEventCreate": (ctypes.POINTER(_P),),
    "hipEventDestroy": (_P,),
    "hipEventRecord": (_P, _P),
    "hipEventSynchronize": (_P,),
    "hipEventQuery": (_P,),
    "hipEventElapsedTime": (ctypes.POINTER(ctypes.c_float), _P, _P),
    "hipModuleLoadData": (ctypes.POINTER(_P), _P),
    "hipModuleUnload": (_P,),
    "hipModuleGetFunction": (ctypes.POINTER(_P), _P, ctypes.c_char_p),
    "hipModuleLaunchKernel": (_P, _U32, _U32, _U32, _U32, _U32, _U32, _U32, _P, _P, _P),
    "hipStreamBeginCapture": (_P, _INT),
    "hipStreamEndCapture": (_P, ctypes.POINTER(_P)),
    "hipGraphInstantiate": (ctypes.POINTER(_P), _P, _P, ctypes.c_char_p, _SZ),
    "hipGraphLaunch": (_P, _P),
    "hipGraphExecDestroy": (_P,),
    "hipGraphDestroy": (_P,),
    "hipGraphAddEventRecordNode": (ctypes.POINTER(_P), _P, ctypes.POINTER(_P), _SZ, _P),
    "hipStreamGetCaptureInfo_v2": (_P, ctypes.POINTER(_INT), ctypes.POINTER(ctypes.c_ulonglong), ctypes.POINTER(_P),
                                   ctypes.POINTER(ctypes.POINTER(_P)), ctypes.POINTER(_SZ)),
    "hipStreamUpdateCaptureDependencies": (_P, ctypes.POINTER(_P), _SZ, _U32),
}
CAPTURE_SET_DEPENDENCIES = 1  # hipStreamSetCaptureDependencies
# hipStreamCaptureMode: only this thread's HIP calls are checked against the capture
CAPTURE_THREAD_LOCAL = 1

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None
_initialised = False


def _loaded_runtimes() -> set[str]:
    """Paths of the HIP runtime files mapped into this process."""
    try:
        with open("/proc/self/maps") as maps:
            return {line.split()[-1] for line in maps if "libamdhip64" in line and "/" in line}
    except OSError:
        return set()


def runtime_path() -> str:
    """Which HIP runtime file this process should open (see the module docstring)."""
    explicit = os.environ.get("MI355X_HIP_RUNTIME")
    if explicit:
        return explicit
    if _loaded_runtimes():
        return "libamdhip64.so.7"
    import importlib.util

    try:
        spec = importlib.util.find_spec("torch")
    except (ImportError, ValueError):
        spec = None
    if spec is not None and spec.origin:
        bundled = os.path.join(os.path.dirname(spec.origin), "lib", "libamdhip64.so")
        if os.path.exists(bundled):
            return bundled
    return "libamdhip64.so.7"


def check_single_runtime() -> None:
    """RuntimeError when two HIP runtime files are mapped (e.g. torch imported after a plugin
    opened a different runtime with MI355X_HIP_RUNTIME): their devices, streams and memory do
    not mix."""
    loaded = _loaded_runtimes()
    if len(loaded) > 1:
        raise RuntimeError(f"two HIP runtimes are loaded in this process ({', '.join(sorted(loaded))}); torch and "
                           "the MI355X plugin must share one: import torch first or unset MI355X_HIP_RUNTIME")


def library() -> ctypes.CDLL:
    """Load and type the HIP runtime once (``runtime_path``)."""
    global _lib
    with _lock:
        if _lib is None:
            try:
                lib = ctypes.CDLL(runtime_path())
            except OSError:
                lib = ctypes.CDLL("/opt/rocm/lib/libamdhip64.so")
            for fn, args in _SIGNATURES.items():
                f = getattr(lib, fn)
                f.argtypes = args
                f.restype = _INT
            lib.hipGetErrorString.argtypes = (_INT,)
            lib.hipGetErrorString.restype = ctypes.c_char_p
            _lib = lib
        return _lib


def error_string(code: int) -> str:
    return (library().hipGetErrorString(code) or b"").decode(errors="replace")


def check(status: int, operation: str) -> None:
    """Raise the reference's native-failure error shape for a non-zero hipError_t."""
    if status != 0:
        raise RuntimeError(f"{operation} failed: {status} ({error_string(status)})")


def call(name: str, *args) -> None:
    check(getattr(library(), name)(*args), name)


def init() -> None:
    global _initialised
    if not _initialised:
        call("hipInit", 0)
        _initialised = True


def device_count() -> int:
    """Number of visible HIP devices (0 when none; never raises for a missing GPU)."""
    try:
        lib = library()
    except OSError:
        return 0
    n = ctypes.c_int(0)
    return n.value if lib.hipGetDeviceCount(ctypes.byref(n)) == 0 else 0


def set_device(ordinal: int) -> None:
    call("hipSetDevice", ordinal)


def attribute(attr: int, ordinal: int) -> int:
    v = ctypes.c_int(0)
    call("hipDeviceGetAttribute", ctypes.byref(v), attr, ordinal)
    return v.value


def device_name(ordinal: int) -> str:
    buf = ctypes.create_string_buffer(256)
    call("hipDeviceGetName", buf, 256, ordinal)
    return buf.value.decode(errors="replace")


def malloc(size: int) -> int:
    p = ctypes.c_void_p()
    call("hipMalloc", ctypes.byref(p), max(size, 1))
    return p.value or 0


def host_malloc(size: int) -> int:
    """Pinned host memory (hipHostMalloc, default flags)."""
    p = ctypes.c_void_p()
    call("hipHostMalloc", ctypes.byref(p), max(size, 1), 0)
    return p.value or 0


def stream_create() -> int:
    """A stream at the default priority."""
    s = ctypes.c_void_p()
    call("hipStreamCreate", ctypes.byref(s))
    return s.value or 0


def event_create() -> int:
    e = ctypes.c_void_p()
    call("hipEventCreate", ctypes.byref(e))
    return e.value or 0


def query(name: str, handle: int) -> bool:
    """True when the stream / event has completed, False while it runs; raises on failure."""
    status = getattr(library(), name)(handle)
    if status == HIP_ERROR_NOT_READY:
        return False
    check(status, name)
    return True


def elapsed_ms(start: int, end: int) -> float:
    ms = ctypes.c_float(0.0)
    call("hipEventElapsedTime", ctypes.byref(ms), start, end)
    return float(ms.value)


def module_load(image: bytes) -> tuple[int, ctypes.Array]:
    """Load a code object; returns the module and the buffer that must outlive the call."""
    buf = ctypes.create_string_buffer(image, len(image))
    m = ctypes.c_void_p()
    call("hipModuleLoadData", ctypes.byref(m), ctypes.cast(buf, ctypes.c_void_p))
    return m.value or 0, buf


def module_function(module: int, name: str) -> int:
    f = ctypes.c_void_p()
    call("hipModuleGetFunction", ctypes.byref(f), module, name.encode())
    return f.value or 0


def launch(function: int, grid: tuple[int, int, int], block: tuple[int, int, int], kernargs: bytes, stream: int,
           shared: int = 0) -> None:
    """hipModuleLaunchKernel with a packed kernarg buffer (HIP_LAUNCH_PARAM_BUFFER_POINTER)."""
    args = ctypes.create_string_buffer(kernargs, max(len(kernargs), 1))
    size = ctypes.c_size_t(len(kernargs))
    extra = (ctypes.c_void_p * 5)(_PARAM_BUFFER_POINTER, ctypes.cast(args, ctypes.c_void_p).value,
                                  _PARAM_BUFFER_SIZE, ctypes.cast(ctypes.byref(size), ctypes.c_void_p).value, _PARAM_END)
    call("hipModuleLaunchKernel", function, *grid, *block, shared, stream, None, extra)


def capture_begin(stream: int) -> None:
    """Start recording the work issued to ``stream`` (hipStreamBeginCapture, thread-local mode)."""
    call("hipStreamBeginCapture", stream, CAPTURE_THREAD_LOCAL)


def capture_end(stream: int) -> int:
    """Stop recording; returns the captured hipGraph_t."""
    g = ctypes.c_void_p()
    call("hipStreamEndCapture", stream, ctypes.byref(g))
    return g.value or 0


def capture_event(stream: int, event: int) -> None:
    """While ``stream`` is being captured: add a node that records ``event`` after everything
    captured so far, and make it what the next captured work depends on.  (hipEventRecord under
    capture becomes no graph node on this runtime, so the node is added to the capture graph.)"""
    status = ctypes.c_int(0)
    graph = ctypes.c_void_p()
    deps = ctypes.POINTER(ctypes.c_void_p)()
    count = ctypes.c_size_t(0)
    call("hipStreamGetCaptureInfo_v2", stream, ctypes.byref(status), None, ctypes.byref(graph), ctypes.byref(deps),
         ctypes.byref(count))
    node = ctypes.c_void_p()
    call("hipGraphAddEventRecordNode", ctypes.byref(node), graph, deps if count.value else None, count.value, event)
    call("hipStreamUpdateCaptureDependencies", stream, ctypes.byref(node), 1, CAPTURE_SET_DEPENDENCIES)


def graph_instantiate(graph: int) -> int:
    """hipGraphInstantiate; returns the executable graph."""
    e = ctypes.c_void_p()
    log = ctypes.create_string_buffer(512)
    status = library().hipGraphInstantiate(ctypes.byref(e), graph, None, log, 512)
    if status != 0:
        raise RuntimeError(f"hipGraphInstantiate failed: {status} ({error_string(status)}) {log.value.decode(errors='replace')}")
    return e.value or 0
