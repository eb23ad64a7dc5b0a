"""GPU detection for the profiler (reference autotune/src/autotune/runner/detect.py:7-20).

``detect_neuron_cores`` counted NeuronCores with ``neuron-ls`` and raised on
zero.  Here the C ABI reports the visible HIP devices and device 0's arch;
the kernels are built for gfx950 only, so another arch is an error too.
"""

from __future__ import annotations

import ctypes

TARGET_ARCH = "gfx950"


def detect_gpus() -> tuple[int, str, int]:
    """``(num_devices, arch of device 0, CUs of device 0)``.

    Raises:
        RuntimeError: no HIP device visible, or device 0 is not gfx950.
    """
    from kernel_library import _lib

    L = _lib.lib()
    n = ctypes.c_int(0)
    cus = ctypes.c_int(0)
    arch = ctypes.create_string_buffer(64)
    rc = L.mi_device_info(ctypes.byref(n), arch, len(arch), ctypes.byref(cus))
    if rc != 0:
        raise RuntimeError(f"HIP device query failed: {_lib.last_error()}")
    if n.value == 0:
        raise RuntimeError("no HIP device visible: the profiler needs an MI355X (gfx950)")
    name = arch.value.decode()
    if not name.startswith(TARGET_ARCH):
        raise RuntimeError(f"device 0 is {name!r}; the kernels are built for {TARGET_ARCH} only")
    return n.value, name, cus.value
