"""CPU checks of the C ABI: the library loads and exports every declared symbol."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

from conftest import REPO

HEADER = os.path.join(REPO, "include", "dattri_amd.h")


def declared_functions() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(da_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_functions()
    assert "da_ghost_gram" in names and "da_last_error" in names


def test_library_exports_every_declared_symbol():
    from dattri_llm_amd import _native

    if not os.path.exists(_native.library_path()):
        pytest.fail("libdattri_amd.so is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(_native.library_path())
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    # the Python binding types exactly the declared set
    assert sorted(_native.SIGNATURES) == declared_functions()


def test_abi_version_and_error_plumbing():
    from dattri_llm_amd import _native

    lib = _native.load()
    assert lib.da_abi_version() == _native.ABI_VERSION
    # an invalid call fails without touching a GPU and leaves a message
    status = lib.da_selftest_mfma(0, 32, None, None, None, None)
    assert status == _native.DA_ERR_INVALID
    assert b"null" in lib.da_last_error()
