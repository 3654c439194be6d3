"""The C-ABI library loads on a host without a GPU, exports every symbol that
include/fuel_rocm.h declares, and its host-only logic answers without a device
(no compute calls here)."""
import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fuel_rocm.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(frq_\w+)\s*\(", text)))


def test_header_declares_the_seams():
    syms = declared_symbols()
    for s in ("frq_qstorage_load", "frq_qstorage_zeros", "frq_qstorage_fwd", "frq_qstorage_dequantize",
              "frq_qstorage_data", "frq_qstorage_device_ptr", "frq_qmatmul", "frq_quantize_q8k",
              "frq_block_isums"):
        assert s in syms


def test_library_exports_every_declared_symbol():
    import fuel_amd

    lib = fuel_amd.lib()
    syms = declared_symbols()
    missing = [s for s in syms if not hasattr(lib, s)]
    assert not missing, missing
    # the Python binding types every declared entry point
    assert sorted(fuel_amd.SIGNATURES) == syms


def test_block_geometry_without_device():
    import fuel_amd

    assert [fuel_amd.type_size(t) for t in (8, 12, 14, 15)] == [34, 144, 210, 292]
    assert [fuel_amd.block_size(t) for t in (8, 12, 14, 15)] == [32, 256, 256, 256]
    assert fuel_amd.type_size(2) == 0  # Q4_0 is not handled by this backend


def test_errors_are_status_codes_not_crashes():
    import fuel_amd

    if fuel_amd.device_count() > 0:
        pytest.skip("a GPU is present; the no-device path is not reachable")
    with pytest.raises(fuel_amd.FuelRocmError) as ei:
        fuel_amd.RocmDevice(0)
    assert ei.value.status == 2
    lib = fuel_amd.lib()
    assert lib.frq_qmatmul(None, 12, 1, 1, 1, 256, None, 1024, None, 144, None, 4) == 2
    assert b"null device" in lib.frq_last_error()
