"""ctypes binding of libaoakv.so (C ABI in include/aoakv.h).

Loading fails loudly: there is no CPU or PyTorch fallback for any op.
"""
from __future__ import annotations

import ctypes
import os

# the package's own build; AOAKV_LIB names another build of the library to
# load instead (how a driver picks the tree it measures)
LIB_PATH = os.environ.get("AOAKV_LIB") or os.path.join(
    os.path.dirname(os.path.abspath(__file__)), "libaoakv.so")

AOAKV_OK = 0
AOAKV_ERR_INVALID = 1
AOAKV_ERR_UNSUPPORTED = 2
AOAKV_ERR_HIP = 3

FLAG_VALUE_AWARE = 1
FLAG_FIXED = 2
FLAG_SINGLE_LAUNCH = 4
FLAG_QUEST_KERNEL = 8
FLAG_GROUPED_DECODE = 16

_u32 = ctypes.c_uint32
_p = ctypes.c_void_p
_sz = ctypes.c_size_t
_int = ctypes.c_int
_f32 = ctypes.c_float

# name -> argument types (all return int status unless listed in _RESTYPES)
SIGNATURES = {
    "aoakv_last_error": [],
    "aoakv_version": [],
    "aoakv_append_kv_cache_prefill": [_p, _p, _u32, _p, _p, _u32, _u32, _p, _p, _p, _p,
                                      _u32, _u32, _u32, _u32, _p],
    "aoakv_append_kv_cache_decode": [_p, _p, _u32, _p, _p, _p, _p, _p, _p, _p, _p, _p,
                                     _u32, _u32, _u32, _u32, _p],
    "aoakv_estimate_attn_score": [_p, _p, _u32, _p, _p, _p, _p, _p, _p, _p, _u32, _u32,
                                  _u32, _u32, _u32, _u32, _u32, _u32, _p],
    "aoakv_topk_filtering": [_p, _u32, _p, _p, _p, _u32, _p, _p, _u32, _u32, _u32, _u32,
                             _u32, _p, _p],
    "aoakv_decode_workspace_size": [_u32, _u32, _u32, _u32, _u32],
    "aoakv_layer_workspace_size": [_u32, _u32, _u32, _u32, _u32, _u32],
    "aoakv_workspace_init": [_p, _sz, _p],
    "aoakv_decode_sparse_attn": [_p, _p, _p, _p, _p, _p, _p, _u32, _u32, _p, _p, _sz, _u32,
                                 _u32, _u32, _u32, _u32, _u32, _u32, _u32, _p],
    "aoakv_sparse_decode_layer": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _u32, _p,
                                  _u32, _u32, _p, _p, _sz, _u32, _u32, _u32, _u32, _u32,
                                  _u32, _u32, _u32, _p],
    "aoakv_sparse_decode_layer_noalloc": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _u32,
                                          _p, _u32, _u32, _p, _u32, _u32, _u32, _u32, _u32,
                                          _u32, _u32, _u32, _p],
    "aoakv_noalloc_init": [],
    "aoakv_noalloc_error": [_p, _u32, _p],
    "aoakv_estimate_topk": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _u32, _p, _u32, _u32, _p, _p,
                            _sz, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _p],
    "aoakv_prefill_with_paged_kv_cache": [_p, _p, _p, _p, _u32, _u32, _u32, _u32, _u32,
                                          _u32, _u32, _u32, _u32, _p],
    "aoakv_apply_rope_in_place": [_p, _p, _u32, _u32, _u32, _u32, _u32, _f32, _f32, _p],
    "aoakv_rms_norm_forward": [_p, _p, _p, _u32, _u32, _f32, _p],
    "aoakv_rope_append_kv_cache_decode": [_p, _p, _p, _u32, _u32, _p, _p, _p, _p, _p, _p, _p,
                                          _p, _p, _u32, _u32, _u32, _u32, _f32, _f32, _p],
}
_RESTYPES = {
    "aoakv_last_error": ctypes.c_char_p,
    "aoakv_version": ctypes.c_char_p,
    "aoakv_decode_workspace_size": _sz,
    "aoakv_layer_workspace_size": _sz,
}


class AoakvError(RuntimeError):
    """An entry point of libaoakv.so returned a non-zero status."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed (code {code}): {msg}")
        self.code = code


_lib = None
_loaded_path = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load libaoakv.so once and declare every entry point's signature."""
    global _lib, _loaded_path
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ImportError(
            f"libaoakv.so not found at {path}; build it with "
            "`python aoa-kv_amd/aoakv/_build.py` (hipcc, gfx950) -- there is no fallback")
    lib = ctypes.CDLL(path)
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _RESTYPES.get(name, _int)
    _lib = lib
    _loaded_path = os.path.abspath(path)
    return lib


def loaded_path() -> str:
    """Path of the library this process loaded."""
    load()
    return _loaded_path


def call(name: str, *args) -> None:
    """Call an entry point and raise AoakvError on a non-zero status."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != AOAKV_OK:
        raise AoakvError(name, rc, lib.aoakv_last_error().decode())


def version() -> str:
    return load().aoakv_version().decode()
