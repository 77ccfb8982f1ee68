"""The C ABI boundary on CPU: the library loads, exports every entry point
include/chomik_hip.h declares, its enums agree with the Python planner, and
bring-up fails cleanly (an error code and a message) without a gfx950 GPU.
No compute call is made here."""

from __future__ import annotations

import ctypes
import re

import pytest

from chomikgrad import _hiplib, _planner
from conftest import ROOT

HEADER = ROOT / "include" / "chomik_hip.h"


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(chip_\w+)\s*\(", text, re.M)))


def header_enum(name):
    text = HEADER.read_text()
    body = re.search(r"enum " + name + r" \{(.*?)\};", text, re.S).group(1)
    return {k: int(v) for k, v in re.findall(r"(CHIP_\w+)\s*=\s*(\d+)", body)}


@pytest.fixture(scope="module")
def lib():
    path = _hiplib.library_path()
    if not path.exists():
        pytest.fail(f"{path} is missing: run __graft_entry__.build() first")
    return _hiplib.Library(path)


def test_every_declared_entry_point_is_exported(lib):
    names = declared_functions()
    assert len(names) >= 25
    for name in names:
        assert hasattr(lib.raw, name), name
    assert set(names) - {"chip_last_error"} == set(_hiplib.SIGNATURES)


def test_step_kinds_match_the_planner():
    kinds = header_enum("chip_kind")
    for name, value in kinds.items():
        short = name[len("CHIP_K_"):]
        assert getattr(_planner, "K_" + short, value) == value, name
    dtypes = header_enum("chip_dtype")
    from chomikgrad import dtypes as d
    assert (d.DT_F32, d.DT_F16, d.DT_BF16, d.DT_I32, d.DT_I64) == (
        dtypes["CHIP_F32"], dtypes["CHIP_F16"], dtypes["CHIP_BF16"], dtypes["CHIP_I32"], dtypes["CHIP_I64"])


def test_calls_before_init_fail_with_a_message(lib):
    pointer = ctypes.c_void_p()
    status = lib.raw.chip_malloc(ctypes.c_size_t(16), ctypes.byref(pointer))
    assert status == _hiplib.CHIP_ENODEV
    assert "chip_init" in lib.last_error()


def test_bring_up_without_gpu_raises_runtime_error(lib):
    import os

    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU driver is present")
    status = lib.raw.chip_init(0)
    assert status == _hiplib.CHIP_ENODEV
    with pytest.raises(RuntimeError, match="gfx950|HIP device"):
        lib.raise_status(status)


def test_missing_library_raises_import_error(tmp_path, monkeypatch):
    monkeypatch.setenv("CHOMIK_HIP_LIB", str(tmp_path / "absent.so"))
    with pytest.raises(ImportError, match="not found"):
        _hiplib.Library()


def test_malformed_tape_is_rejected_before_init(lib):
    tape = (ctypes.c_int64 * 3)(1, 2, 3)
    handle = ctypes.c_void_p()
    assert lib.raw.chip_plan_create(tape, 3, ctypes.byref(handle)) != _hiplib.CHIP_OK
