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


def test_argument_checks_fail_before_any_gpu_work():
    """Each entry point validates its arguments on the host first: a bad call
    returns its status and message without touching a device.  Pointers here
    are aligned placeholders that no rejected call dereferences."""
    from dattri_llm_amd import _native

    lib = _native.load()
    X, OUT = 0x10000, 0x20000  # 16-byte aligned, never dereferenced
    bf, f32 = _native.DA_BF16, _native.DA_F32

    def check(status, code, words):
        assert status == code, (status, lib.da_last_error())
        msg = lib.da_last_error().decode()
        assert all(w in msg for w in words), msg

    # da_row_gram(x, dtype, rows, width, x_stride, out, ld_out, accumulate, workspace, workspace_bytes, stream)
    check(lib.da_row_gram(X, f32, 10, 8, 8, OUT, 8, 0, None, 0, None), _native.DA_ERR_UNSUPPORTED, ["bf16 or fp16"])
    check(lib.da_row_gram(X, bf, -1, 8, 8, OUT, 8, 0, None, 0, None), _native.DA_ERR_INVALID, ["negative"])
    check(lib.da_row_gram(None, bf, 10, 8, 8, OUT, 8, 0, None, 0, None), _native.DA_ERR_INVALID, ["NULL"])
    check(lib.da_row_gram(X, bf, 10, 8, 8, None, 8, 0, None, 0, None), _native.DA_ERR_INVALID, ["NULL"])
    check(lib.da_row_gram(X, bf, 10, 12, 12, OUT, 12, 0, None, 0, None), _native.DA_ERR_INVALID, ["multiples of 8"])
    check(lib.da_row_gram(X + 8, bf, 10, 8, 8, OUT, 8, 0, None, 0, None), _native.DA_ERR_INVALID, ["aligned"])
    check(lib.da_row_gram(X, bf, 10, 8, 8, OUT, 6, 0, None, 0, None), _native.DA_ERR_INVALID, ["out row stride"])
    # nothing to do: no launch, success (no rows with accumulate, or no width)
    assert lib.da_row_gram(None, bf, 0, 8, 8, OUT, 8, 1, None, 0, None) == _native.DA_OK
    assert lib.da_row_gram(X, bf, 10, 0, 8, OUT, 8, 0, None, 0, None) == _native.DA_OK

    # da_nonzero_rows(x, dtype, rows, width, x_stride, out, stream)
    check(lib.da_nonzero_rows(X, 9, 4, 8, 8, OUT, None), _native.DA_ERR_INVALID, ["bad dtype"])
    check(lib.da_nonzero_rows(None, bf, 4, 8, 8, OUT, None), _native.DA_ERR_INVALID, ["NULL"])
    check(lib.da_nonzero_rows(X, bf, 4, 12, 12, OUT, None), _native.DA_ERR_INVALID, ["16 bytes"])
    assert lib.da_nonzero_rows(None, bf, 0, 8, 8, None, None) == _native.DA_OK

    # da_materialize_linear(a, g, dtype, batch, tokens, K, D, a_bs, a_ts, g_bs, g_ts, bias,
    #                       out, out_dtype, out_bs, out_rs, out_blk, stream)
    def mat(dtype=bf, k=64, d=64, a=X, blk=64, out_rs=64, tokens=4):
        return lib.da_materialize_linear(a, X, dtype, 2, tokens, k, d, 4 * k, k, 4 * d, d, 0, OUT, f32,
                                         d * out_rs, out_rs, blk, None)

    check(mat(dtype=9), _native.DA_ERR_INVALID, ["bad dtype"])
    check(mat(k=12), _native.DA_ERR_INVALID, ["multiples of 8"])
    check(mat(a=None), _native.DA_ERR_INVALID, ["NULL"])
    check(mat(blk=32), _native.DA_ERR_INVALID, ["out_blk"])
    check(mat(out_rs=32), _native.DA_ERR_INVALID, ["row stride"])
    check(mat(tokens=0), _native.DA_ERR_INVALID, ["tokens"])

    # da_project_outer: projected widths above 64 are refused before anything else
    st = lib.da_project_outer(X, X, bf, 2, 16, 64, 64, 1024, 64, 1024, 64, X, 65, 64, None, X, 64, 64,
                              OUT, f32, 65 * 64, None, 0, None)
    check(st, _native.DA_ERR_UNSUPPORTED, ["projected widths"])


def test_grouped_side_record_has_the_struct_layout():
    """The numpy records the grouped launches fill read back field for field
    through the ctypes mirror of da_factor_side."""
    import numpy as np

    from dattri_llm_amd import _native as nat
    from dattri_llm_amd import kernels

    assert kernels._SIDE_RECORD.itemsize == ctypes.sizeof(nat.FactorSide)
    rec = np.zeros(2, dtype=kernels._SIDE_RECORD)
    for i, (name, _t) in enumerate(nat.FactorSide._fields_):
        rec[name] = [1000 * (i + 1) + 1, 1000 * (i + 1) + 2]
    sides = (nat.FactorSide * 2).from_buffer(rec)
    for j in range(2):
        for i, (name, _t) in enumerate(nat.FactorSide._fields_):
            assert getattr(sides[j], name) == 1000 * (i + 1) + 1 + j, name
