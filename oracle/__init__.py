"""numpy front end of the C oracle (liboxide_oracle.so).

TEST INFRASTRUCTURE ONLY.  Imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker; the product library never
imports or calls it.  Each function names the reference code it restates (the C
side, oracle/oxide_oracle.c, carries the same citations and the list of checks
that pin each function).
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

_DIR = Path(__file__).resolve().parent
_LIB_PATH = _DIR / "liboxide_oracle.so"
_lib = None

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32


def build() -> Path:
    """Compiles the oracle with its Makefile (gcc, OpenMP, IEEE arithmetic)."""
    subprocess.run(["make", "-s", "-B", "-C", str(_DIR)], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(_LIB_PATH))
        L.oracle_half_to_float.restype = ctypes.c_float
        L.oracle_half_to_float.argtypes = [ctypes.c_uint16, ctypes.c_int]
        L.oracle_float_to_half.restype = ctypes.c_uint16
        L.oracle_float_to_half.argtypes = [ctypes.c_float, ctypes.c_int]
        L.oracle_compute_slot_mapping.argtypes = [_p, _i64, _i64, _i64, _i64, _p]
        L.oracle_build_decode_metadata.restype = _i64
        L.oracle_build_decode_metadata.argtypes = [_p, _i64, _p, _p]
        L.oracle_pad_block_table.restype = _i64
        L.oracle_pad_block_table.argtypes = [_p, _p, _i64, _p]
        L.oracle_reshape_and_cache.argtypes = [_p, _p, _p, _p, _p, _i64, _i64, _i64, ctypes.c_int]
        L.oracle_copy_blocks.argtypes = [_p, _p, _p, _i64, _i64, ctypes.c_int]
        L.oracle_gather_blocks.argtypes = [_p, _p, _p, _p, _p, _i64, _i64, ctypes.c_int]
        L.oracle_paged_decode_attention.argtypes = [
            _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i32, ctypes.c_float,
            ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.oracle_prefill_attention.argtypes = [
            _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i32, ctypes.c_float,
            ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.oracle_rope_cos_sin_cache.argtypes = [_p, _i64, _i64, ctypes.c_float]
        L.oracle_qk_norm_rope_and_cache.argtypes = [
            _p, _p, _p, _i64, _p, _p, ctypes.c_double, _p, _i64, _p, _p, _p, _p, _i64, _i64, _i64,
            _i64, ctypes.c_int]
        L.oracle_xxh64.restype = ctypes.c_uint64
        L.oracle_xxh64.argtypes = [_p, ctypes.c_size_t, ctypes.c_uint64]
        _lib = L
    return _lib


def _ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


DTYPE_CODE = {"f16": 0, "bf16": 1, "f32": 2}


# ---------------------------------------------------------------- formats
def half_to_float(bits: np.ndarray, dtype: str) -> np.ndarray:
    """16-bit patterns -> fp32 (exact)."""
    f = np.vectorize(lambda h: lib().oracle_half_to_float(int(h), DTYPE_CODE[dtype]), otypes=[np.float32])
    return f(np.asarray(bits, dtype=np.uint16))


def float_to_half(x: np.ndarray, dtype: str) -> np.ndarray:
    """fp32 -> 16-bit patterns, round to nearest even."""
    f = np.vectorize(lambda v: lib().oracle_float_to_half(float(v), DTYPE_CODE[dtype]), otypes=[np.uint16])
    return f(np.asarray(x, dtype=np.float32))


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """Vectorised bf16 -> fp32 (bf16 is the top half of fp32)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Vectorised fp32 -> bf16 round-to-nearest-even (finite inputs), same rule
    as oracle_float_to_half(dtype=bf16)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def bits_to_f32(bits: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return bf16_bits_to_f32(bits)
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


# ------------------------------------------------------------- host logic
def compute_slot_mapping(block_table, block_size: int, token_offset: int, num_tokens: int) -> np.ndarray:
    """KvCacheManager::compute_slot_mapping (engine/kv_cache_manager.rs:115-135)."""
    bt = np.ascontiguousarray(block_table, dtype=np.int64)
    out = np.empty(num_tokens, dtype=np.int64)
    lib().oracle_compute_slot_mapping(_ptr(bt), bt.size, block_size, token_offset, num_tokens, _ptr(out))
    return out


def build_decode_metadata(context_lens):
    """build_decode_metadata (attention/metadata.rs:20-47) -> (cu_q, cu_k, max_seqlen_k)."""
    cl = np.ascontiguousarray(context_lens, dtype=np.uint32)
    cu_q = np.empty(cl.size + 1, dtype=np.uint32)
    cu_k = np.empty(cl.size + 1, dtype=np.uint32)
    mx = lib().oracle_build_decode_metadata(_ptr(cl), cl.size, _ptr(cu_q), _ptr(cu_k))
    return cu_q, cu_k, int(mx)


def pad_block_table(rows) -> np.ndarray:
    """block_table_tensor (attention/flash_attn.rs:74-86): pad rows with 0."""
    lens = np.array([len(r) for r in rows], dtype=np.int64)
    flat = np.ascontiguousarray(np.concatenate([np.asarray(r, dtype=np.int32) for r in rows])
                                if len(rows) and lens.sum() else np.zeros(0, np.int32), dtype=np.int32)
    width = int(lens.max()) if len(rows) else 0
    out = np.empty((len(rows), width), dtype=np.int32)
    lib().oracle_pad_block_table(_ptr(flat), _ptr(lens), len(rows), _ptr(out))
    return out


# ---------------------------------------------------------- cache copies
def reshape_and_cache(key, value, key_cache, value_cache, slot_mapping) -> None:
    """reshape_and_cache (kernels/reshape_and_cache.cu:6-28), in place on the caches.
    key/value [T, H, D]; caches [NB, BS, H, D] (any 2- or 4-byte dtype)."""
    T, H, D = key.shape
    sm = np.ascontiguousarray(slot_mapping, dtype=np.int64)
    lib().oracle_reshape_and_cache(_ptr(key), _ptr(value), _ptr(key_cache), _ptr(value_cache),
                                   _ptr(sm), T, H, D, key.dtype.itemsize)


def copy_blocks(key_cache, value_cache, block_mapping) -> None:
    """copy_blocks (kernels/copy_blocks.cu:8-28), in place."""
    bm = np.ascontiguousarray(block_mapping, dtype=np.int64).reshape(-1, 2)
    stride = int(np.prod(key_cache.shape[1:]))
    lib().oracle_copy_blocks(_ptr(key_cache), _ptr(value_cache), _ptr(bm), bm.shape[0], stride,
                             key_cache.dtype.itemsize)


def gather_blocks(key_cache, value_cache, block_ids):
    ids = np.ascontiguousarray(block_ids, dtype=np.int32)
    kd = np.empty((ids.size,) + key_cache.shape[1:], dtype=key_cache.dtype)
    vd = np.empty_like(kd) if value_cache is not None else None
    stride = int(np.prod(key_cache.shape[1:]))
    lib().oracle_gather_blocks(_ptr(kd), _ptr(vd), _ptr(key_cache), _ptr(value_cache), _ptr(ids),
                               ids.size, stride, key_cache.dtype.itemsize)
    return kd, vd


# -------------------------------------------------------------- attention
def paged_decode_attention(q, k_cache, v_cache, cu_seqlens_k, block_table, softmax_scale: float,
                           window_left: int = -1, dtype: str = "bf16", use_f64: bool = False,
                           threads: int = 0) -> np.ndarray:
    """Decode call of flash_attn_varlen_paged_windowed (attention/flash_attn.rs:52-67).
    q [B, Hq, D] and caches [NB, BS, Hkv, D] as uint16 bit patterns; returns fp32 [B, Hq, D]."""
    B, Hq, D = q.shape
    NB, BS, Hkv, D2 = k_cache.shape
    assert D == D2 and q.dtype == np.uint16 and k_cache.dtype == np.uint16
    bt = np.ascontiguousarray(block_table, dtype=np.int32)
    cu = np.ascontiguousarray(cu_seqlens_k, dtype=np.uint32)
    out = np.empty((B, Hq, D), dtype=np.float32)
    lib().oracle_paged_decode_attention(_ptr(out), _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(cu),
                                        _ptr(bt), bt.shape[1] if bt.ndim == 2 else 0, B, Hq, Hkv, D,
                                        BS, window_left, softmax_scale, DTYPE_CODE[dtype],
                                        int(use_f64), threads)
    return out


def prefill_attention(q, k, v, cu_seqlens_q, cu_seqlens_k, softmax_scale: float, block_table=None,
                      window_left: int = -1, dtype: str = "bf16", use_f64: bool = False,
                      threads: int = 0) -> np.ndarray:
    """Causal varlen prefill attention (attention/flash_attn.rs:15-37, and the
    seqlen_q >= 1 call of flash_attn_varlen_paged_windowed, :52-67), masks aligned
    bottom-right.  q [total_q, Hq, D]; k/v are the paged caches [NB, BS, Hkv, D]
    with `block_table` [B, max_blocks], or contiguous [total_k, Hkv, D] when
    block_table is None.  uint16 bit patterns in, fp32 [total_q, Hq, D] out."""
    Tq, Hq, D = q.shape
    assert q.dtype == np.uint16 and k.dtype == np.uint16 and v.dtype == np.uint16
    if block_table is None:
        _, Hkv, D2 = k.shape
        BS, bt, maxb = 1, None, 0
    else:
        _, BS, Hkv, D2 = k.shape
        bt = np.ascontiguousarray(block_table, dtype=np.int32)
        maxb = bt.shape[1]
    assert D == D2
    cq = np.ascontiguousarray(cu_seqlens_q, dtype=np.uint32)
    ck = np.ascontiguousarray(cu_seqlens_k, dtype=np.uint32)
    B = len(cq) - 1
    assert len(ck) == B + 1 and int(cq[-1]) == Tq
    out = np.empty((Tq, Hq, D), dtype=np.float32)
    lib().oracle_prefill_attention(_ptr(out), _ptr(q), _ptr(k), _ptr(v), _ptr(cq), _ptr(ck), _ptr(bt),
                                   maxb, B, Hq, Hkv, D, BS, window_left, softmax_scale,
                                   DTYPE_CODE[dtype], int(use_f64), threads)
    return out


def rope_cos_sin_cache(max_position: int, rotary_dim: int, base: float) -> np.ndarray:
    """RotaryEmbedding::new's cos_sin_cache (layers/rope.rs:50-83), fp32 [max_position, rotary_dim]."""
    out = np.empty((max_position, rotary_dim), np.float32)
    lib().oracle_rope_cos_sin_cache(_ptr(out), max_position, rotary_dim, base)
    return out


def qk_norm_rope_and_cache(qkv, num_heads: int, num_kv_heads: int, head_dim: int, q_norm_weight,
                           k_norm_weight, eps: float, cos_sin_cache, positions, key_cache=None,
                           value_cache=None, slot_mapping=None, dtype: str = "bf16"):
    """Qwen3Attention::forward's prologue (models/qwen3.rs:161-199) on uint16 bit patterns:
    returns (q_out [T, Hq, D], k_out [T, Hkv, D]) and appends k/v into the caches in place."""
    T = qkv.shape[0]
    qkv = np.ascontiguousarray(qkv)
    q_out = np.empty((T, num_heads, head_dim), np.uint16)
    k_out = np.empty((T, num_kv_heads, head_dim), np.uint16)
    cs = np.ascontiguousarray(cos_sin_cache, np.float32)
    pos = np.ascontiguousarray(positions, np.int32)
    sm = None if slot_mapping is None else np.ascontiguousarray(slot_mapping, np.int64)
    lib().oracle_qk_norm_rope_and_cache(_ptr(q_out), _ptr(k_out), _ptr(qkv), qkv.shape[1],
                                        _ptr(q_norm_weight), _ptr(k_norm_weight), eps, _ptr(cs),
                                        cs.shape[0], _ptr(pos), _ptr(key_cache), _ptr(value_cache),
                                        _ptr(sm), T, num_heads, num_kv_heads, head_dim, DTYPE_CODE[dtype])
    return q_out, k_out


def xxh64(data: bytes, seed: int = 0) -> int:
    buf = ctypes.create_string_buffer(data, len(data))
    return int(lib().oracle_xxh64(buf, len(data), seed))
