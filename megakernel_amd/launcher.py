"""Build and device detection (counterpart of /root/reference/host/launcher.py).

The reference detects an NVIDIA compute capability and runs nvcc
(launcher.py:25-132); here the target is fixed (gfx950) and the build is the
Makefile's ``lib`` target driven by hipcc.  Device facts come from the
library itself (``megakernel_device_info``), not from a GPU framework.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

from . import _lib
from .config import HBM_PEAK_GBPS

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def compile_shared_library(arch: str = "gfx950", verbose: bool = False) -> str:
    """Build megakernel_amd/megakernel.so (always recompiles every translation
    unit, eight in parallel)."""
    lib = os.path.join(REPO, "megakernel_amd", "megakernel.so")
    if os.path.exists(lib):
        os.remove(lib)
    cmd = ["make", "-C", REPO, "-B", "-j8", "lib", f"ARCH={arch}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if verbose or r.returncode != 0:
        print(r.stdout[-4000:], r.stderr[-4000:])
    if r.returncode != 0:
        raise RuntimeError("hipcc build of megakernel.so failed")
    return lib


def detect_gpu(lib_path: str | None = None) -> dict:
    """CU count, wall-clock rate and name of the current HIP device."""
    lib = _lib.load(lib_path)
    cus, khz = ctypes.c_int(0), ctypes.c_int(0)
    name = ctypes.create_string_buffer(256)
    _lib.check(lib, lib.megakernel_device_info(ctypes.byref(cus), ctypes.byref(khz), name, 256), "device_info")
    return {"name": name.value.decode(), "cu_count": cus.value, "wall_clock_khz": khz.value,
            "peak_bw_gbps": HBM_PEAK_GBPS}
