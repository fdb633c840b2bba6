"""torch-tensor front end of the C ABI, shaped like the reference's Rust wrappers.

* reshape_and_cache / copy_blocks mirror crates/vllm-oxide/src/attention/kernels.rs:106-180
  (dims taken from the tensors, dtype code from the key dtype, the tensor's stream).
* decode_attn mirrors flash_attn_varlen_paged_windowed as called at
  crates/vllm-oxide/src/attention/flash_attn.rs:39-68 (the callee allocates the output).
* gather_blocks is the prefix-hit gather (no reference counterpart).
* prefill_attn mirrors prefill_attn (flash_attn.rs:15-37, flash_attn_varlen, causal) over
  contiguous K/V, and, given a block table, the seqlen_q >= 1 call of
  flash_attn_varlen_paged_windowed (flash_attn.rs:52-67) over the paged cache.

Tensors must be contiguous CUDA (HIP) tensors; every call goes to the HIP library
on torch's current stream and raises OxideError if the library reports an error.
"""
from __future__ import annotations

import torch

from . import _lib

_DTYPE_CODE = {torch.float16: _lib.DTYPE_F16, torch.bfloat16: _lib.DTYPE_BF16,
               torch.float32: _lib.DTYPE_F32}


def dtype_code(dt: torch.dtype) -> int:
    """kernels.rs:97-104: f16 -> 0, bf16 -> 1, f32 -> 2; anything else is an error."""
    try:
        return _DTYPE_CODE[dt]
    except KeyError:
        raise _lib.OxideError(f"unsupported KV cache dtype: {dt}") from None


def _ptr(t: torch.Tensor | None) -> int | None:
    if t is None:
        return None
    if not t.is_cuda:
        raise _lib.OxideError("expected a device tensor")
    if not t.is_contiguous():
        raise _lib.OxideError("expected a contiguous tensor")
    return t.data_ptr()


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def reshape_and_cache(key: torch.Tensor, value: torch.Tensor, key_cache: torch.Tensor,
                      value_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """Append: key/value [T, Hkv, D] into the per-layer caches [NB, BS, Hkv, D] at slot_mapping (int64)."""
    L = _lib.load()
    if slot_mapping.dtype != torch.int64:
        raise _lib.OxideError("slot_mapping must be int64")
    T, H, D = key.shape
    L.reshape_and_cache(_ptr(key), _ptr(value), _ptr(key_cache), _ptr(value_cache),
                        _ptr(slot_mapping), T, H, D, dtype_code(key.dtype), _stream(key))
    _lib.check()


def copy_blocks(key_cache: torch.Tensor, value_cache: torch.Tensor,
                block_mapping: torch.Tensor) -> None:
    """Copy-on-write: block_mapping int64 [P, 2] of (src, dst) block ids."""
    L = _lib.load()
    if block_mapping.dtype != torch.int64:
        raise _lib.OxideError("block_mapping must be int64")
    num_pairs = block_mapping.shape[0]
    d = key_cache.shape
    block_stride = d[1] * d[2] * d[3]  # kernels.rs:164-165
    L.copy_blocks(_ptr(key_cache), _ptr(value_cache), _ptr(block_mapping), num_pairs, block_stride,
                  dtype_code(key_cache.dtype), _stream(key_cache))
    _lib.check()


def gather_blocks(key_cache: torch.Tensor, value_cache: torch.Tensor | None,
                  block_ids: torch.Tensor, key_out: torch.Tensor | None = None,
                  value_out: torch.Tensor | None = None):
    """Prefix-hit gather: returns contiguous [n * BS, Hkv, D] K (and V) of the listed blocks."""
    L = _lib.load()
    if block_ids.dtype != torch.int32:
        raise _lib.OxideError("block_ids must be int32")
    n = block_ids.shape[0]
    NB, BS, H, D = key_cache.shape
    if key_out is None:
        key_out = torch.empty((n * BS, H, D), dtype=key_cache.dtype, device=key_cache.device)
    if value_cache is not None and value_out is None:
        value_out = torch.empty_like(key_out)
    L.gather_blocks(_ptr(key_out), _ptr(value_out) if value_cache is not None else None,
                    _ptr(key_cache), _ptr(value_cache), _ptr(block_ids), n, BS * H * D,
                    dtype_code(key_cache.dtype), _stream(key_cache))
    _lib.check()
    return key_out, value_out


def workspace_size(batch: int, num_heads: int, num_kv_heads: int, head_dim: int,
                   max_seqlen_k: int) -> int:
    return int(_lib.load().paged_decode_attention_workspace_size(batch, num_heads, num_kv_heads,
                                                                 head_dim, max_seqlen_k))


def split_tokens(batch: int, num_kv_heads: int, max_seqlen_k: int, path: int | str = 0,
                 num_heads: int | None = None, head_dim: int = 128, page_block_size: int = 256) -> int:
    """Tokens per KV split of the decode pass 1; 0 for the persistent balanced pass, -1 for
    the wave-level stream pass, -2 for the row pass (only reported when num_heads is given:
    the row pass depends on the query heads).  path: as for decode_attn (0 / "auto" = by
    shape)."""
    L = _lib.load()
    path = DECODE_PATHS[path] if isinstance(path, str) else int(path)
    if num_heads is not None:
        return int(L.paged_decode_attention_pass1(path, batch, num_heads, num_kv_heads, head_dim, page_block_size,
                                                  max_seqlen_k))
    if path == 0:
        return int(L.paged_decode_attention_split_tokens(batch, num_kv_heads, max_seqlen_k))
    return int(L.paged_decode_attention_path_split_tokens(path, batch, num_kv_heads, max_seqlen_k))


# Forms of a cascaded call (paged_decode_attention_shared_prefix_mode).
CASCADE_MODES = {"auto": 0, "serial": 1, "overlap": 2, "plain": 3}


def shared_prefix_plan(batch: int, num_heads: int, num_kv_heads: int, head_dim: int, page_block_size: int,
                       max_seqlen_k: int, shared_blocks_hint: int) -> str:
    """The form the by-shape cascaded call takes: "serial", "overlap" or "plain"."""
    code = int(_lib.load().paged_decode_attention_shared_prefix_plan(
        batch, num_heads, num_kv_heads, head_dim, page_block_size, max_seqlen_k, shared_blocks_hint))
    return {v: k for k, v in CASCADE_MODES.items()}[code]


def shared_prefix_workspace_size(batch: int, num_heads: int, num_kv_heads: int, head_dim: int,
                                 page_block_size: int, max_seqlen_k: int, shared_blocks_hint: int) -> int:
    """Workspace bytes of a cascaded call (paged_decode_attention_shared_prefix)."""
    return int(_lib.load().paged_decode_attention_shared_prefix_workspace_size(
        batch, num_heads, num_kv_heads, head_dim, page_block_size, max_seqlen_k, shared_blocks_hint))


# First-pass names of paged_decode_attention_path.
DECODE_PATHS = {"auto": 0, "split": 1, "persistent": 2, "stream": 3, "rows": 4}


def decode_attn(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                cu_seqlens_k: torch.Tensor, block_table: torch.Tensor, max_seqlen_k: int,
                softmax_scale: float, window_left: int | None = None,
                page_block_size: int = 256, out: torch.Tensor | None = None,
                workspace: torch.Tensor | None = None, append=None, path: int | str = 0,
                noalloc: bool = False, shared_prefix_blocks: int | None = None,
                shared_prefix_mode: int | str = "auto") -> torch.Tensor:
    """Paged decode attention.

    q [B, Hq, D]; k_cache/v_cache [NB, page_block_size, Hkv, D]; cu_seqlens_k uint32-valued
    int32 tensor [B + 1] (torch has no uint32 arithmetic; the bits are passed as is);
    block_table int32 [B, max_blocks] padded with 0; window_left None = unbounded.
    append=(key, value, slot_mapping): first append each sequence's new token (key/value
    [B, Hkv, D], int64 slots) -- fused into the same launch (paged_decode_attention_append).
    path: the first pass, by name or code of DECODE_PATHS; anything but "auto" / 0 goes
    through paged_decode_attention_path for this call only.
    noalloc: call paged_decode_attention_noalloc (partials in the library's static device
    scratch; no workspace is allocated or passed; path must be "auto").
    shared_prefix_blocks: an upper bound on the leading block-table entries every row
    shares -> paged_decode_attention_shared_prefix (the shared keys attended once for the
    whole batch; the library finds the actual count); path must be "auto".
    shared_prefix_mode: the cascade's form by name or code of CASCADE_MODES; anything but
    "auto" goes through paged_decode_attention_shared_prefix_mode.
    """
    L = _lib.load()
    B, Hq, D = q.shape
    NB, BS, Hkv, D2 = k_cache.shape
    if D2 != D or BS != page_block_size or v_cache.shape != k_cache.shape:
        raise _lib.OxideError("q / k_cache / v_cache shapes disagree")
    if block_table.dtype != torch.int32 or cu_seqlens_k.dtype not in (torch.int32, torch.uint32):
        raise _lib.OxideError("block_table must be int32 and cu_seqlens_k 32-bit")
    if k_cache.dtype != q.dtype or v_cache.dtype != q.dtype:
        raise _lib.OxideError("q and caches must share a dtype")
    if out is None:
        out = torch.empty_like(q)
    path = DECODE_PATHS[path] if isinstance(path, str) else int(path)
    if append is not None:
        key, value, slot_mapping = append
        if key.shape != (B, Hkv, D) or value.shape != key.shape or slot_mapping.dtype != torch.int64:
            raise _lib.OxideError("append needs key/value [B, Hkv, D] and int64 slot_mapping [B]")
    max_blocks = block_table.shape[1] if block_table.dim() == 2 else 0
    w = -1 if window_left is None else int(window_left)
    if noalloc:
        if path != 0 or workspace is not None:
            raise _lib.OxideError("noalloc takes no workspace and no forced path")
        kv = (None, None, None) if append is None else (_ptr(key), _ptr(value), _ptr(slot_mapping))
        L.paged_decode_attention_noalloc(_ptr(out), _ptr(q), *kv, _ptr(k_cache), _ptr(v_cache), _ptr(cu_seqlens_k),
                                         _ptr(block_table), max_blocks, NB, B, Hq, Hkv, D, BS, max_seqlen_k, w,
                                         float(softmax_scale), dtype_code(q.dtype), _stream(q))
        _lib.check()
        return out
    if shared_prefix_blocks is not None:
        if path != 0 or noalloc:
            raise _lib.OxideError("shared_prefix_blocks takes no forced path and no noalloc")
        need = shared_prefix_workspace_size(B, Hq, Hkv, D, BS, max_seqlen_k, int(shared_prefix_blocks))
        if workspace is None or workspace.numel() * workspace.element_size() < need:
            workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
        kv = (None, None, None) if append is None else (_ptr(key), _ptr(value), _ptr(slot_mapping))
        mode = CASCADE_MODES[shared_prefix_mode] if isinstance(shared_prefix_mode, str) else int(shared_prefix_mode)
        args = (_ptr(out), _ptr(q), *kv, _ptr(k_cache), _ptr(v_cache), _ptr(cu_seqlens_k), _ptr(block_table),
                max_blocks, NB, B, Hq, Hkv, D, BS, max_seqlen_k, w, float(softmax_scale), int(shared_prefix_blocks),
                _ptr(workspace), workspace.numel() * workspace.element_size(), dtype_code(q.dtype), _stream(q))
        if mode == 0:
            L.paged_decode_attention_shared_prefix(*args)
        else:
            L.paged_decode_attention_shared_prefix_mode(mode, *args)
        _lib.check()
        return out
    need = workspace_size(B, Hq, Hkv, D, max_seqlen_k)
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    tail = (_ptr(k_cache), _ptr(v_cache), _ptr(cu_seqlens_k), _ptr(block_table),
            max_blocks, NB, B, Hq, Hkv, D, BS, max_seqlen_k, w, float(softmax_scale),
            _ptr(workspace), workspace.numel() * workspace.element_size(), dtype_code(q.dtype),
            _stream(q))
    if path != 0:
        kv = (None, None, None) if append is None else (_ptr(key), _ptr(value), _ptr(slot_mapping))
        L.paged_decode_attention_path(path, _ptr(out), _ptr(q), *kv, *tail)
    elif append is None:
        L.paged_decode_attention(_ptr(out), _ptr(q), *tail)
    else:
        L.paged_decode_attention_append(_ptr(out), _ptr(q), _ptr(key), _ptr(value),
                                        _ptr(slot_mapping), *tail)
    _lib.check()
    return out


def prefill_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens_q: torch.Tensor,
                 cu_seqlens_k: torch.Tensor, max_seqlen_q: int, max_seqlen_k: int,
                 softmax_scale: float, block_table: torch.Tensor | None = None,
                 window_left: int | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """Causal varlen prefill attention, masks aligned bottom-right (FlashAttention 2).

    q [total_q, Hq, D].  With block_table (int32 [B, max_blocks], 0-padded), k/v are the
    paged caches [NB, BS, Hkv, D]; without, contiguous [total_k, Hkv, D].  cu_seqlens_q /
    cu_seqlens_k are 32-bit [B + 1] (uint32 bits).  window_left None = unbounded.
    """
    L = _lib.load()
    Tq, Hq, D = q.shape
    if cu_seqlens_q.dtype not in (torch.int32, torch.uint32) or \
            cu_seqlens_k.dtype not in (torch.int32, torch.uint32):
        raise _lib.OxideError("cu_seqlens_q / cu_seqlens_k must be 32-bit")
    if k.dtype != q.dtype or v.dtype != q.dtype or v.shape != k.shape:
        raise _lib.OxideError("q, k and v must share a dtype and k/v a shape")
    B = cu_seqlens_q.shape[0] - 1
    if cu_seqlens_k.shape[0] != B + 1:
        raise _lib.OxideError("cu_seqlens_q and cu_seqlens_k disagree on the batch")
    if out is None:
        out = torch.empty_like(q)
    w = -1 if window_left is None else int(window_left)
    if block_table is not None:
        NB, BS, Hkv, D2 = k.shape
        if D2 != D or block_table.dtype != torch.int32:
            raise _lib.OxideError("k_cache [NB, BS, Hkv, D] and int32 block_table expected")
        max_blocks = block_table.shape[1] if block_table.dim() == 2 else 0
        L.paged_prefill_attention(_ptr(out), _ptr(q), _ptr(k), _ptr(v), _ptr(cu_seqlens_q),
                                  _ptr(cu_seqlens_k), _ptr(block_table), max_blocks, NB, B, Hq, Hkv,
                                  D, BS, max_seqlen_q, max_seqlen_k, w, float(softmax_scale),
                                  dtype_code(q.dtype), _stream(q))
    else:
        Tk, Hkv, D2 = k.shape
        if D2 != D:
            raise _lib.OxideError("k [total_k, Hkv, D] expected")
        L.varlen_prefill_attention(_ptr(out), _ptr(q), _ptr(k), _ptr(v), _ptr(cu_seqlens_q),
                                   _ptr(cu_seqlens_k), Tk, B, Hq, Hkv, D, max_seqlen_q, max_seqlen_k,
                                   w, float(softmax_scale), dtype_code(q.dtype), _stream(q))
    _lib.check()
    return out


def rope_cos_sin_cache(max_position: int, rotary_dim: int, base: float = 1_000_000.0,
                       device=None) -> torch.Tensor:
    """RotaryEmbedding's fp32 cos_sin_cache [max_position, rotary_dim] (layers/rope.rs:50-83),
    built on the host by the library and moved to `device`."""
    L = _lib.load()
    cache = torch.empty((max_position, rotary_dim), dtype=torch.float32)
    rc = L.oxide_rope_cos_sin_cache(cache.data_ptr(), max_position, rotary_dim, float(base))
    if rc != _lib.OXIDE_OK:
        raise _lib.OxideError(f"oxide_rope_cos_sin_cache: error {rc}")
    return cache.to(device) if device is not None else cache


def qk_norm_rope_and_cache(qkv: torch.Tensor, num_heads: int, num_kv_heads: int,
                           q_norm_weight: torch.Tensor | None, k_norm_weight: torch.Tensor | None,
                           eps: float, cos_sin_cache: torch.Tensor, positions: torch.Tensor,
                           key_cache: torch.Tensor | None = None, value_cache: torch.Tensor | None = None,
                           slot_mapping: torch.Tensor | None = None, return_k: bool = False,
                           q_out: torch.Tensor | None = None, k_out: torch.Tensor | None = None):
    """Qwen3 attention prologue + KV append in one launch (models/qwen3.rs:161-199).

    qkv [T, (Hq + 2 Hkv) D] (row = q | k | v); returns q [T, Hq, D] (and k [T, Hkv, D]
    with return_k).  positions int32 [T]; cos_sin_cache fp32 [max_position, D];
    key/value caches [NB, BS, Hkv, D] with int64 slot_mapping [T] (-1 = skip).
    q_out / k_out: optional preallocated contiguous outputs of those shapes (a
    serving loop reuses its buffers); k_out implies return_k.
    """
    L = _lib.load()
    T = qkv.shape[0]
    D = cos_sin_cache.shape[1]
    if positions.dtype != torch.int32 or cos_sin_cache.dtype != torch.float32:
        raise _lib.OxideError("positions must be int32 and cos_sin_cache float32")
    if slot_mapping is not None and slot_mapping.dtype != torch.int64:
        raise _lib.OxideError("slot_mapping must be int64")
    if qkv.dim() != 2 or qkv.stride(1) != 1:
        raise _lib.OxideError("qkv must be [T, row] with unit element stride")
    for name, t, heads in (("q_out", q_out, num_heads), ("k_out", k_out, num_kv_heads)):
        if t is not None and (tuple(t.shape) != (T, heads, D) or t.dtype != qkv.dtype
                              or not t.is_contiguous() or t.device != qkv.device):
            raise _lib.OxideError(f"{name} must be a contiguous [{T}, {heads}, {D}] tensor like qkv")
    return_k = return_k or k_out is not None
    q = q_out if q_out is not None else torch.empty((T, num_heads, D), dtype=qkv.dtype, device=qkv.device)
    k = k_out if k_out is not None else (
        torch.empty((T, num_kv_heads, D), dtype=qkv.dtype, device=qkv.device) if return_k else None)
    L.qk_norm_rope_and_cache(_ptr(q), _ptr(k), qkv.data_ptr(), qkv.stride(0), _ptr(q_norm_weight),
                             _ptr(k_norm_weight), float(eps), _ptr(cos_sin_cache), cos_sin_cache.shape[0],
                             _ptr(positions), _ptr(key_cache), _ptr(value_cache), _ptr(slot_mapping), T,
                             num_heads, num_kv_heads, D, dtype_code(qkv.dtype), _stream(qkv))
    _lib.check()
    return (q, k) if return_k else q


def build_decode_metadata(context_lens: torch.Tensor, block_table: torch.Tensor, block_size: int = 256):
    """Device-side decode metadata: (cu_seqlens_k [B+1] as int32 bits of uint32,
    slot_mapping int64 [B]) from context_lens (int32 bits of uint32, [B]) and the
    0-padded int32 block table [B, max_blocks]."""
    L = _lib.load()
    if context_lens.dtype not in (torch.int32, torch.uint32) or block_table.dtype != torch.int32:
        raise _lib.OxideError("context_lens must be 32-bit and block_table int32")
    B = context_lens.shape[0]
    cu = torch.empty(B + 1, dtype=torch.int32, device=context_lens.device)
    slots = torch.empty(B, dtype=torch.int64, device=context_lens.device)
    max_blocks = block_table.shape[1] if block_table.dim() == 2 else 0
    L.build_decode_metadata_device(_ptr(context_lens), _ptr(block_table) if block_table.numel() else None,
                                   max_blocks, B, block_size, _ptr(cu), _ptr(slots) if B else None,
                                   _stream(context_lens))
    _lib.check()
    return cu, slots
