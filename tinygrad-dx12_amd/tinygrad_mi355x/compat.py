"""Device registration (alexandreteles/tinygrad-dx12 src/tinygrad_dx12/compat.py:69-177).

``register()`` makes ``MI355X`` the first device tinygrad tries, when tinygrad is
importable, by aliasing ``tinygrad.runtime.ops_mi355x`` to this package's runtime,
adding the name to ``Device._devices`` and prepending it to ``ALL_DEVICES``.  It
opens no hardware, downloads nothing and is idempotent.  Without tinygrad it records
the device in :data:`DEVICES`, the standalone registry used by
:func:`tinygrad_mi355x.runtime.ops_mi355x.get_device`.
"""

from __future__ import annotations

import importlib
import sys

DEVICE = "MI355X"
DEVICES: list[str] = []
_registered = False


def register() -> None:
    """Register MI355X for explicit use and automatic device selection (no hardware opened)."""
    global _registered
    if _registered:
        return
    if DEVICE not in DEVICES:
        DEVICES.insert(0, DEVICE)
    try:
        tinygrad_device = importlib.import_module("tinygrad.device")
    except ImportError:
        tinygrad_device = None
    if tinygrad_device is not None:
        runtime = importlib.import_module("tinygrad_mi355x.runtime.ops_mi355x")
        sys.modules["tinygrad.runtime.ops_mi355x"] = runtime
        devices = getattr(tinygrad_device.Device, "_devices", None)
        if isinstance(devices, list) and DEVICE not in devices:
            devices.append(DEVICE)
        all_devices = getattr(tinygrad_device, "ALL_DEVICES", None)
        if isinstance(all_devices, list) and DEVICE not in all_devices:
            all_devices.insert(0, DEVICE)
    _registered = True


def registered() -> bool:
    return _registered
