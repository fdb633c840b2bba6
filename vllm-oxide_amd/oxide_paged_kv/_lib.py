"""ctypes binding of include/oxide_paged_kv.h (liboxide_paged_kv.so).

There is no fallback: if the HIP library is not built, importing the ops raises.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent.parent
# OXIDE_PAGED_KV_LIB points at another build of the same library (e.g. a tuning variant).
LIB_PATH = Path(os.environ.get("OXIDE_PAGED_KV_LIB", PKG_DIR / "liboxide_paged_kv.so"))

DTYPE_F16, DTYPE_BF16, DTYPE_F32 = 0, 1, 2
OXIDE_OK = 0

# Every symbol the header declares, with its ctypes signature.
_p = ctypes.c_void_p
_i64 = ctypes.c_int64
SIGNATURES = {
    "reshape_and_cache": (None, [_p, _p, _p, _p, _p, _i64, _i64, _i64, ctypes.c_int, _p]),
    "copy_blocks": (None, [_p, _p, _p, _i64, _i64, ctypes.c_int, _p]),
    "gather_blocks": (None, [_p, _p, _p, _p, _p, _i64, _i64, ctypes.c_int, _p]),
    "paged_decode_attention": (None, [
        _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, ctypes.c_int32,
        ctypes.c_float, _p, ctypes.c_size_t, ctypes.c_int, _p]),
    "paged_decode_attention_append": (None, [
        _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
        ctypes.c_int32, ctypes.c_float, _p, ctypes.c_size_t, ctypes.c_int, _p]),
    "paged_decode_attention_noalloc": (None, [
        _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
        ctypes.c_int32, ctypes.c_float, ctypes.c_int, _p]),
    "paged_decode_attention_workspace_size": (ctypes.c_size_t, [_i64, _i64, _i64, _i64, _i64]),
    "paged_decode_attention_shared_prefix": (None, [
        _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
        ctypes.c_int32, ctypes.c_float, _i64, _p, ctypes.c_size_t, ctypes.c_int, _p]),
    "paged_decode_attention_shared_prefix_mode": (None, [
        ctypes.c_int, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
        ctypes.c_int32, ctypes.c_float, _i64, _p, ctypes.c_size_t, ctypes.c_int, _p]),
    "paged_decode_attention_shared_prefix_plan": (ctypes.c_int, [_i64, _i64, _i64, _i64, _i64, _i64, _i64]),
    "paged_decode_attention_shared_prefix_workspace_size": (ctypes.c_size_t, [_i64, _i64, _i64, _i64, _i64, _i64,
                                                                              _i64]),
    "paged_decode_attention_split_tokens": (_i64, [_i64, _i64, _i64]),
    "paged_decode_attention_path_split_tokens": (_i64, [ctypes.c_int, _i64, _i64, _i64]),
    "paged_decode_attention_pass1": (_i64, [ctypes.c_int, _i64, _i64, _i64, _i64, _i64, _i64]),
    "paged_decode_attention_path": (None, [
        ctypes.c_int, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
        ctypes.c_int32, ctypes.c_float, _p, ctypes.c_size_t, ctypes.c_int, _p]),
    "paged_prefill_attention": (None, [
        _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
        ctypes.c_int32, ctypes.c_float, ctypes.c_int, _p]),
    "varlen_prefill_attention": (None, [
        _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, ctypes.c_int32,
        ctypes.c_float, ctypes.c_int, _p]),
    "qk_norm_rope_and_cache": (None, [
        _p, _p, _p, _i64, _p, _p, ctypes.c_double, _p, _i64, _p, _p, _p, _p, _i64, _i64, _i64, _i64,
        ctypes.c_int, _p]),
    "oxide_rope_cos_sin_cache": (ctypes.c_int, [_p, _i64, _i64, ctypes.c_float]),
    "build_decode_metadata_device": (None, [_p, _p, _i64, _i64, _i64, _p, _p, _p]),
    "oxide_fill_normal": (ctypes.c_int, [_p, _i64, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int, ctypes.c_int]),
    "oxide_last_error": (ctypes.c_int, []),
    "oxide_clear_error": (None, []),
    "oxide_error_string": (ctypes.c_char_p, [ctypes.c_int]),
}

_lib = None


class OxideError(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    """Loads the in-tree HIP library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python vllm-oxide_amd/build.py` "
                "(there is no CPU fallback)")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check() -> None:
    """Raises OxideError if the calling thread has a pending library error."""
    L = load()
    code = L.oxide_last_error()
    if code != OXIDE_OK:
        L.oxide_clear_error()
        raise OxideError(f"oxide error {code}: {L.oxide_error_string(code).decode()}")
