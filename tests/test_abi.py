"""The C-ABI library loads without a GPU and exports every function that
include/ic_abi.h declares (no compute calls here)."""

import ctypes
import os

import pytest

from int_crush_converter_amd import _native as nat


@pytest.fixture(scope="module")
def libicq():
    if not os.path.exists(nat.LIB_PATH):
        from int_crush_converter_amd import build
        build.build()
    return ctypes.CDLL(nat.LIB_PATH)


def test_header_declares_functions():
    names = nat.header_functions()
    assert "ic_rotate_rows" in names and "ic_last_error" in names
    assert len(names) >= 10


def test_library_exports_header_symbols(libicq):
    missing = [n for n in nat.header_functions() if not hasattr(libicq, n)]
    assert not missing, f"symbols declared in ic_abi.h but not exported: {missing}"


def test_loader_signatures_cover_header():
    assert set(nat.header_functions()) <= set(nat._SIGS), "every ABI function needs a ctypes signature"


def test_version_and_error_without_gpu(libicq):
    libicq.ic_abi_version.restype = ctypes.c_int
    assert libicq.ic_abi_version() == 1
    libicq.ic_last_error.restype = ctypes.c_char_p
    assert isinstance(libicq.ic_last_error(), bytes)


def test_argument_validation_without_gpu(libicq):
    """Bad arguments are rejected on the host before any HIP call."""
    nat.load(require_gpu=False)
    L = nat._lib
    rc = L.ic_rotate_rows(None, 0, 4, 16, 16, None, 16, 16, 16, 0.0, None, None)
    assert rc == -1 and b"null" in L.ic_last_error()
    rc = L.ic_rotate_rows(1, 0, 4, 16, 16, 1, 16, 16, 12, 0.0, None, None)
    assert rc == -1 and b"power of 2" in L.ic_last_error()
