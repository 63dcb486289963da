"""ctypes binding of libquail_mi355x.so, the gfx950 C-ABI library.

The library is the only compute path: there is no fallback. A missing or
unbuildable library raises `QxUnavailable` at the first call, so a GPU run
without the native kernels fails loudly instead of computing elsewhere.

Every entry point returns an int status: 0, -1 (argument error, message in
`qx_last_error()`), or a positive hipError_t from the launch.
"""

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libquail_mi355x.so"
HEADER = Path(__file__).resolve().parent.parent / "include" / "quail_mi355x.h"

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float

# QX_ABI_VERSION of include/quail_mi355x.h, which these signatures follow
ABI_VERSION = 2

# name -> argument types (the declarations in include/quail_mi355x.h)
SIGNATURES = {
    "qx_version": [],
    "qx_last_error": [],
    "qx_device_is_gfx950": [],
    "qx_gemm_fp8_blockscaled": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64,
                                _i32, _p],
    "qx_add_rmsnorm_quant": [_p, _i64, _p, _i64, _p, _p, _i64, _p, _i64, _i64, _i64, _f32, _p],
    "qx_rmsnorm_quant": [_p, _i64, _p, _p, _i64, _p, _i64, _i64, _i64, _f32, _p],
    "qx_embed_rmsnorm_quant": [_p, _i64, _p, _p, _i64, _p, _p, _i64, _p, _i64, _i64, _i64,
                               _f32, _p],
    "qx_add_rmsnorm": [_p, _i64, _p, _i64, _p, _p, _p, _i64, _p, _i64, _i64, _i64, _f32, _p],
    "qx_qk_norm_rope": [_p, _i64, _p, _i64, _p, _i64, _p, _i32, _p, _p, _p, _i64, _i64, _i64,
                        _i64, _f32, _p],
    "qx_qk_norm_rope_kv": [_p, _i64, _p, _i64, _p, _p, _p, _p, _p, _p, _p, _i32, _p, _p, _p,
                           _i64, _i64, _i64, _i64, _f32, _i32, _p],
    "qx_silu_mul_quant": [_p, _i64, _p, _i64, _p, _i64, _i64, _i64, _p],
    "qx_gemm_fp8_swiglu_quant": [_p, _p, _p, _p, _p, _i64, _p, _i64, _i64, _i64, _i64, _i64,
                                 _i64, _i32, _p],
    "qx_vocab_logprobs_workspace": [_i64, _i64, _i64],
    "qx_vocab_logprobs": [_p, _i64, _p, _i64, _p, _i64, _p, _i64, _i64, _i64, _i64, _p, _i64,
                          _p],
    "qx_vocab_logprobs_noalloc_max_bytes": [],
    "qx_vocab_logprobs_noalloc": [_p, _i64, _p, _i64, _p, _i64, _p, _i64, _i64, _i64, _i64, _p],
    "qx_group_quant": [_p, _i64, _p, _i64, _p, _i64, _i64, _i64, _p],
    "qx_kv_scatter": [_p, _i64, _p, _i64, _p, _p, _p, _p, _i64, _i64, _i32, _p],
    "qx_embed": [_p, _i64, _p, _p, _i64, _i64, _i64, _p],
    "qx_paged_attention": [_p, _i64, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64,
                           _i64, _i64, _f32, _i32, _p, _p, _i64, _p, _i64, _p, _i64, _i64, _i32,
                           _p],
    "qx_paged_attention_tile_rows": [_p, _p, _i64, _i64, _i64, _i64, _i32],
    "qx_paged_attention_max_keys": [_i64],
    "qx_paged_attention_qnorm": [_p, _i64, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64,
                                 _i64, _i64, _i64, _f32, _i32, _p, _i64, _p, _i64, _p, _i64,
                                 _i64, _i32, _p, _p, _i32, _p, _f32, _p],
    "qx_paged_attention_work": [_p, _p, _i64, _i64, _i64, _i64, _i32, _i64, _p, _i64],
    "qx_attention_lse": [_p, _i64, _p, _p, _p, _p, _p, _p, _i64, _p, _i64, _i64, _i64, _i64,
                         _i64, _i64, _f32, _i32, _p, _i64, _p, _i64, _p, _i64, _i32, _p],
    "qx_merge_attn_quant": [_p, _i64, _p, _i64, _p, _i64, _p, _i64, _p, _i64, _i64, _i64, _p,
                            _i64, _p, _i64, _p],
    "qx_merge_partial": [_p, _i64, _p, _i64, _p, _p, _i64, _p, _i64, _i64, _i64, _i64, _p],
    "qx_prefix_tree": [_p, _p, _i64, _i64, _p, _p, _p],
    "qx_pages_create": [_i64, _i64, _p],
    "qx_pages_destroy": [_p],
    "qx_pages_alloc": [_p, _i64, _i64, _i64, _p, _i64, _p],
    "qx_pages_shared": [_p, _i64, _i64, _i64, _p, _i64, _p],
    "qx_pages_table": [_p, _i64, _p, _i64, _p],
    "qx_pages_stats": [_p, _p],
    "qx_pages_keys": [_p, _p, _i64, _p],
    "qx_pages_free_key": [_p, _i64, _p],
    "qx_pages_drop_leading": [_p, _i64, _i64, _p],
    "qx_pages_rewind": [_p, _i64, _i64, _p],
    "qx_pages_grow": [_p, _i64, _i64, _p],
    "qx_pages_set_tokens": [_p, _i64, _i64],
    "qx_pages_pin": [_p, _i64],
    "qx_pages_retain": [_p, _i64, _i32, ctypes.c_double],
    "qx_pages_pop_victim": [_p, _p, _i64, _p],
    "qx_pages_free_list": [_p, _p, _i64, _p],
    "qx_pack_unified": [_p, _p, _i64, _p, _p, _p, _p, _p],
    "qx_pack_array": [_p, _i64, _p, _p],
    "qx_pack_destroy": [_p],
    "qx_answer_head": [_p, _i64, _p, _i64, _i64, _i64, _i64, _i32, _p, _f32, _p, _p, _p, _p,
                       _p],
}


# entry points returning a count (>= 0) or -1 instead of a status
RETURNS_COUNT = {"qx_paged_attention_work", "qx_paged_attention_tile_rows",
                 "qx_paged_attention_max_keys", "qx_vocab_logprobs_workspace",
                 "qx_vocab_logprobs_noalloc_max_bytes"}


class QxUnavailable(RuntimeError):
    """The native library is not built or cannot be loaded."""


class QxError(RuntimeError):
    """A native entry point rejected its arguments or failed to launch."""


_LIB = None


def load(path: Path = LIB_PATH):
    """Load the library once and bind every declared entry point."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not path.exists():
        raise QxUnavailable(
            f"{path} is not built; run `python -m quail_amd.build` (hipcc, gfx950)")
    try:
        lib = ctypes.CDLL(str(path))
    except OSError as err:
        raise QxUnavailable(f"cannot load {path}: {err}") from err
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = (ctypes.c_char_p if name == "qx_last_error" else
                      ctypes.c_int64 if name in RETURNS_COUNT else ctypes.c_int)
    built = lib.qx_version()
    if built != ABI_VERSION:
        raise QxUnavailable(f"{path} has ABI version {built}; this binding (and "
                            f"include/quail_mi355x.h) is version {ABI_VERSION}: rebuild it")
    _LIB = lib
    return lib


def call(name: str, *args) -> None:
    """Call an entry point; raise QxError with the library's message on failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        if rc < 0:
            msg = lib.qx_last_error().decode(errors="replace")
        else:
            msg = f"hipError_t {rc}"
        raise QxError(f"{name}: {msg}")


def count(name: str, *args) -> int:
    """Call an entry point that returns a count; raise QxError on -1."""
    lib = load()
    n = getattr(lib, name)(*args)
    if n < 0:
        raise QxError(f"{name}: {lib.qx_last_error().decode(errors='replace')}")
    return int(n)


def header_abi_version(header: Path = HEADER) -> int:
    """QX_ABI_VERSION as include/quail_mi355x.h defines it."""
    import re
    return int(re.search(r"#define\s+QX_ABI_VERSION\s+(\d+)", header.read_text()).group(1))


def declared_symbols(header: Path = HEADER) -> list:
    """The qx_* functions include/quail_mi355x.h declares."""
    import re
    text = header.read_text()
    return sorted(set(re.findall(r"\b(qx_[a-z0-9_]+)\s*\(", text)))
