"""The C-ABI library builds for gfx950, loads, and exports every entry point
include/quail_mi355x.h declares; argument errors are reported without
touching a GPU."""

import ctypes

import pytest

from quail_amd import _lib


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _lib.declared_symbols()
    assert len(declared) >= 14
    missing = [name for name in declared if not hasattr(lib, name)]
    assert not missing
    assert set(declared) == set(_lib.SIGNATURES)
    assert lib.qx_version() == 1


def test_argument_errors_return_minus_one_with_a_message():
    with pytest.raises(_lib.QxError, match="null pointer"):
        _lib.call("qx_gemm_fp8_blockscaled", None, None, None, None, None, 1, 256, 128, 128,
                  256, 1, 0, None)
    with pytest.raises(_lib.QxError, match="not a multiple of 128"):
        _lib.call("qx_gemm_fp8_blockscaled", 16, 16, 16, 16, 16, 1, 256, 100, 128, 256, 1, 0,
                  None)
    with pytest.raises(_lib.QxError, match="head_dim"):
        _lib.call("qx_paged_attention", 16, 8, 16, 16, 16, 16, 16, 1, 1, 1, 64, 4, 2, 96, 16,
                  0.1, 1, 16, None, 8, None, 0, None)
    with pytest.raises(_lib.QxError, match="1..16"):
        _lib.call("qx_answer_head", 16, 8, 16, 8, 17, 1, 8, 0, None, 1.0, None, None, None,
                  None, None)
