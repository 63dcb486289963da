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
    assert lib.qx_version() == _lib.ABI_VERSION == _lib.header_abi_version()


def test_argument_errors_return_minus_one_with_a_message():
    with pytest.raises(_lib.QxError, match="null pointer"):
        _lib.call("qx_gemm_fp8_blockscaled", None, None, None, None, None, 1, 256, 128, 128,
                  256, 1, 0, None)
    with pytest.raises(_lib.QxError, match="not a multiple of 128"):
        _lib.call("qx_gemm_fp8_blockscaled", 16, 16, 16, 16, 16, 1, 256, 100, 128, 256, 1, 0,
                  None)
    with pytest.raises(_lib.QxError, match="head_dim"):
        _lib.call("qx_paged_attention", 16, 8, 16, 16, 16, 16, 16, 1, 1, 1, 64, 4, 2, 96, 16,
                  0.1, 1, 16, None, 8, None, 0, None, 0, 0, 1, None)
    with pytest.raises(_lib.QxError, match="query rows per workgroup"):
        _lib.call("qx_paged_attention", 16, 8, 16, 16, 16, 16, 16, 1, 1, 1, 64, 4, 2, 64, 16,
                  0.1, 1, 16, None, 8, None, 0, None, 0, 32, 1, None)
    with pytest.raises(_lib.QxError, match="1..16"):
        _lib.call("qx_answer_head", 16, 8, 16, 8, 17, 1, 8, 0, None, 1.0, None, None, None,
                  None, None)


def test_attention_work_list_is_heaviest_first_and_covers_every_tile():
    import numpy as np
    # 3 sequences of 100, 1, 200 query rows over 150, 40, 260 keys (causal)
    cu_q = np.array([0, 100, 101, 301], dtype=np.int32)
    used = np.array([150, 40, 260], dtype=np.int32)
    work = np.zeros(2 * 16, dtype=np.int32)
    n = _lib.count("qx_paged_attention_work", cu_q.ctypes.data, used.ctypes.data, 3, 32, 8,
                   128, 1, 0, work.ctypes.data, 16)
    items = [tuple(work[2 * i:2 * i + 2]) for i in range(n)]
    # query tiles of 64 rows (G = 4): 2 + 1 + 4 of them
    assert sorted(items) == [(0, 0), (0, 1), (1, 0), (2, 0), (2, 1), (2, 2), (2, 3)]
    keys = {(0, 0): 114, (0, 1): 150, (1, 0): 40, (2, 0): 124, (2, 1): 188, (2, 2): 252,
            (2, 3): 260}
    loads = [keys[it] for it in items]
    assert loads == sorted(loads, reverse=True)
    with pytest.raises(_lib.QxError, match="capacity"):
        _lib.count("qx_paged_attention_work", cu_q.ctypes.data, used.ctypes.data, 3, 32, 8,
                   128, 1, 0, work.ctypes.data, 3)


def test_attention_tile_rows_choice_and_32_row_work_list():
    """qx_paged_attention_tile_rows picks 32 query rows per workgroup for
    packs whose 64-row items read few key tiles (at most 8 on average) and
    the default 64 otherwise; only D = 128 with 4 heads per workgroup offers
    32 (G = 2 keeps its default of 128). A 32-row work list covers every
    32-row tile that holds rows, heaviest first."""
    import numpy as np

    def rows(q_lens, used, hq=32, hk=8, d=128):
        cu_q = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
        used = np.asarray(used, dtype=np.int32)
        return _lib.count("qx_paged_attention_tile_rows", cu_q.ctypes.data, used.ctypes.data,
                          len(used), hq, hk, d, 1)

    # 512-token documents after a 64-token prefix: 5.5 key tiles per item
    assert rows([512] * 4, [576] * 4) == 32
    # 1024-token documents: 9.5 key tiles per item
    assert rows([1024] * 4, [1088] * 4) == 64
    assert rows([512] * 4, [576] * 4, d=64) == 64
    assert rows([512] * 4, [576] * 4, hq=16, hk=8) == 128
    cu_q = np.array([0, 100, 101, 301], dtype=np.int32)
    used = np.array([150, 40, 260], dtype=np.int32)
    work = np.zeros(2 * 32, dtype=np.int32)
    n = _lib.count("qx_paged_attention_work", cu_q.ctypes.data, used.ctypes.data, 3, 32, 8,
                   128, 1, 32, work.ctypes.data, 32)
    items = [tuple(work[2 * i:2 * i + 2]) for i in range(n)]
    assert sorted(items) == sorted([(0, t) for t in range(4)] + [(1, 0)] +
                                   [(2, t) for t in range(7)])
    keys = [min(u, u - ql + min(qt * 32 + 32, ql)) for s_, qt in items
            for u, ql in [(int(used[s_]), int(cu_q[s_ + 1] - cu_q[s_]))]]
    assert keys == sorted(keys, reverse=True)
    with pytest.raises(_lib.QxError, match="query rows per workgroup"):
        _lib.count("qx_paged_attention_work", cu_q.ctypes.data, used.ctypes.data, 3, 16, 8,
                   128, 1, 32, work.ctypes.data, 32)


def test_gemm_config_choice_by_shape(monkeypatch):
    """The arithmetic family is a function of N alone: widths that are a
    multiple of 256 or 320 take the promotion family (config 31's 256 x 320
    tiles where those take fewer full-wave units than 256 x 256 ones, or
    where N is not a multiple of 256; config 30 otherwise), the rest config
    11; the environment variable forces one."""
    from quail_amd.engine import GEMM_CONFIG_ENV, gemm_config
    monkeypatch.delenv(GEMM_CONFIG_ENV, raising=False)
    assert gemm_config(6144, 2560, 16294) == 30     # qkv of a Qwen3-4B pack
    assert gemm_config(6144, 2688, 16294) == 30     # 21 K-blocks
    assert gemm_config(6144, 2560, 256) == 30       # fewer tiles than CUs
    assert gemm_config(4096, 4096, 37) == 30        # Qwen3-8B o_proj, a few final rows
    assert gemm_config(2560, 4096, 16294) == 31     # 512 tiles of 256 x 320, not 640
    assert gemm_config(2560, 9728, 8192) == 31      # 256 tiles, not 320
    assert gemm_config(2560, 4096, 13056) == 30     # 510 tiles of 256 x 256: 2 waves
    assert gemm_config(2560, 4096, 2048) == 30      # 80 tiles: 64 wide ones cost more
    assert gemm_config(2560, 2688, 12000) == 30     # 470 tiles against 376 wide ones
    assert gemm_config(10240, 5120, 16294) == 30    # Qwen3-32B qkv: 10 waves either way
    assert gemm_config(5120, 8192, 16294) == 30     # Qwen3-32B o_proj: 5 waves either way
    assert gemm_config(2688, 2560, 16294) == 11
    assert gemm_config(640, 256, 100) == 31         # a multiple of 320 but not of 256
    monkeypatch.setenv(GEMM_CONFIG_ENV, "11")
    assert gemm_config(6144, 2560, 16294) == 11


def test_gemm_family_depends_on_width_only():
    """Rows never change arithmetic with the number of rows in the launch:
    for every width, all M choose configs of one family."""
    from quail_amd.engine import RESCALE_CONFIGS, gemm_config
    for n in (256, 512, 1280, 2560, 4096, 5120, 6144, 10240, 19456, 2688, 640):
        fams = {gemm_config(n, 2560, m) in RESCALE_CONFIGS
                for m in (1, 37, 255, 2048, 8192, 13056, 16294, 16384, 32768)}
        assert len(fams) == 1, n


def test_swiglu_config_choice_by_shape(monkeypatch):
    from quail_amd.engine import GEMM_CONFIG_ENV, SWIGLU_CONFIG_ENV, swiglu_config
    monkeypatch.delenv(GEMM_CONFIG_ENV, raising=False)
    monkeypatch.delenv(SWIGLU_CONFIG_ENV, raising=False)
    assert swiglu_config(19456, 2560, 16294) == 30
    assert swiglu_config(19456, 2560, 9000) == 30
    assert swiglu_config(19456, 2688, 16294) == 30   # 21 K-blocks
    monkeypatch.setenv(SWIGLU_CONFIG_ENV, "10")
    assert swiglu_config(19456, 2560, 16294) == 10
