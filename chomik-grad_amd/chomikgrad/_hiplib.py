"""ctypes binding of ``libchomik_hip.so`` (declarations: include/chomik_hip.h).

The library is looked up at ``$CHOMIK_HIP_LIB`` or next to this file.  A
missing library raises ``ImportError`` and a failing call ``RuntimeError``
carrying ``chip_last_error()`` -- there is no fallback path.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Optional

c_int64_p = ctypes.POINTER(ctypes.c_int64)
c_void_pp = ctypes.POINTER(ctypes.c_void_p)


class ChipInfo(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char * 64),
        ("arch", ctypes.c_char * 32),
        ("compute_units", ctypes.c_int),
        ("wavefront_size", ctypes.c_int),
        ("total_memory", ctypes.c_size_t),
        ("lds_per_block", ctypes.c_size_t),
        ("clock_khz", ctypes.c_int),
        ("memory_clock_khz", ctypes.c_int),
        ("memory_bus_width", ctypes.c_int),
    ]


# name -> (argtypes); every function returns int except chip_last_error.
SIGNATURES = {
    "chip_init": [ctypes.c_int],
    "chip_device_info": [ctypes.POINTER(ChipInfo)],
    "chip_malloc": [ctypes.c_size_t, c_void_pp],
    "chip_free": [ctypes.c_void_p],
    "chip_empty_cache": [],
    "chip_memcpy_h2d": [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int],
    "chip_memcpy_d2h": [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t],
    "chip_memcpy_d2d": [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t],
    "chip_memset": [ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t],
    "chip_synchronize": [],
    "chip_errors": [ctypes.POINTER(ctypes.c_int)],
    "chip_plan_create": [c_int64_p, ctypes.c_size_t, c_void_pp],
    "chip_plan_bind": [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_void_p],
    "chip_plan_bind_many": [ctypes.c_void_p, ctypes.c_uint32,
                            ctypes.POINTER(ctypes.c_uint32), c_void_pp],
    "chip_plan_run": [ctypes.c_void_p],
    "chip_plan_info": [ctypes.c_void_p, c_int64_p, c_int64_p],
    "chip_plan_time_steps": [ctypes.c_void_p, ctypes.POINTER(ctypes.c_float), ctypes.c_int64],
    "chip_plan_time_repeat": [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int64), ctypes.c_int64, ctypes.c_int64,
                              ctypes.POINTER(ctypes.c_float)],
    "chip_plan_destroy": [ctypes.c_void_p],
    "chip_argmax": [ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_int64, c_int64_p],
    "chip_greedy_advance": [
        ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_int64,
        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
        ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64,
        ctypes.c_int, ctypes.c_int64,
    ],
    "chip_greedy_advance_noalloc": [
        ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_int64,
        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
        ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64,
        ctypes.c_int, ctypes.c_int64,
    ],
    "chip_peak_memory": [ctypes.POINTER(ctypes.c_size_t)],
    "chip_reset_peak_memory": [],
    "chip_event_create": [c_void_pp],
    "chip_event_record": [ctypes.c_void_p],
    "chip_event_elapsed_ms": [ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(ctypes.c_float)],
    "chip_event_destroy": [ctypes.c_void_p],
}

# Status codes (enum chip_status) and kernel error bits (enum chip_error_bits).
CHIP_OK = 0
CHIP_EKERNEL = 4
CHIP_ENODEV = 5
ERR_GATHER_INDEX = 1
ERR_POSITION = 2


def library_path() -> Path:
    override = os.environ.get("CHOMIK_HIP_LIB")
    return Path(override) if override else Path(__file__).resolve().parent / "libchomik_hip.so"


class Library:
    """Loaded library with checked wrappers: ``lib.call("chip_x", ...)``."""

    def __init__(self, path: Optional[Path] = None) -> None:
        self.path = Path(path) if path is not None else library_path()
        if not self.path.exists():
            raise ImportError(
                f"libchomik_hip.so not found at {self.path}; build it with "
                "`python chomik-grad_amd/build.py` (or __graft_entry__.build())"
            )
        self.raw = ctypes.CDLL(str(self.path))
        for name, argtypes in SIGNATURES.items():
            function = getattr(self.raw, name)
            function.argtypes = argtypes
            function.restype = ctypes.c_int
        self.raw.chip_last_error.argtypes = []
        self.raw.chip_last_error.restype = ctypes.c_char_p

    def last_error(self) -> str:
        message = self.raw.chip_last_error()
        return message.decode(errors="replace") if message else "unknown error"

    def call(self, name: str, *args) -> int:
        status = getattr(self.raw, name)(*args)
        if status != CHIP_OK:
            self.raise_status(status)
        return status

    def raise_status(self, status: int) -> None:
        message = self.last_error()
        if status == CHIP_EKERNEL:
            bits = ctypes.c_int(0)
            self.raw.chip_errors(ctypes.byref(bits))
            if bits.value & ERR_GATHER_INDEX:
                raise IndexError(f"gather index is outside the first dimension ({message})")
            if bits.value & ERR_POSITION:
                raise IndexError(f"position is outside the RoPE table or KV cache ({message})")
        if status == CHIP_ENODEV:
            raise RuntimeError(f"the hip backend requires an MI355X (gfx950) GPU: {message}")
        raise RuntimeError(message)


_LIBRARY: Optional[Library] = None


def load() -> Library:
    global _LIBRARY
    if _LIBRARY is None:
        _LIBRARY = Library()
    return _LIBRARY
